"""MI355X slot-stream engine: HIP kernel wrappers (``kernels``) and the engine (``slot_engine``)."""
