"""MI355X slot-stream engine: per-slot state pools, packed ticks, one hipGraph per (rows, tokens) bucket.

Host orchestration mirrors SlotStreamEngineV7/V8 (src/hs_guard/engine/slot_engine_v7.py:117-167,
slot_engine_v8.py:30-89): a request list is cut into ticks of at most ``max_tick_tokens`` tokens per slot
and at most the largest session bucket of rows; each tick is one H2D copy of a packed int64 buffer, one
graph replay, one D2H copy of the per-token class probabilities of both roles and one stream sync.

Differences by design (the device program is the MI355X one, not a translation):
* Tokens are PACKED: row n owns tokens offsets[n] .. offsets[n] + lens[n] - 1 of the tick, so GEMMs and
  per-token kernels run over the tick's real tokens rounded up to a token bucket instead of
  rows x 64-token buckets.
* Projections are fused per layer (GDN: qkv|z|b|a; attention: q|k|v; MLP: gate|up; both heads' first
  Linear), each one hipBLASLt GEMM.
* Every other op is a libhsg.so kernel: embed+RMSNorm, conv+SiLU+pool update, GDN step with the gated
  RMSNorm fused, q/k RMSNorm+RoPE in one launch, ring attention with the gate and the in-place ring write
  for any tick length, add+RMSNorm, SiLU-mul, both risk heads, ring_pos update.
* GDN state is fp32 by default (``state_dtype='float16'`` gives the reference StreamingGuard's storage).
"""
from __future__ import annotations

import itertools
import warnings

import numpy as np
import torch

from .. import _hostpack
from .._lib import HSG_ERR_SHAPE, HSG_GDN_BURST_MIN_DEFAULT, HSG_GEMM_SKINNY_M_MAX, check, lib
from ..model import ROLES, GuardModel
from .gemm_plan import WORKSPACE_BYTES as GEMM_WORKSPACE_BYTES
from .gemm_plan import GemmPlans

SESSION_BUCKETS = (1, 2, 4, 8, 16, 32, 48, 64, 96, 128, 160, 192, 224, 256, 320, 352, 384, 448, 512)
STATE_DTYPES = {"float32": torch.float32, "float16": torch.float16}
_STATE_CODE = {torch.float32: 0, torch.float16: 1}


def bucket(value, choices):
    """Smallest choice >= value (src/hs_guard/engine/bucketed_engine.py:12-16)."""
    for choice in choices:
        if value <= choice:
            return choice
    raise ValueError(f"{value} exceeds the largest bucket {choices[-1]}")


def token_buckets(max_tokens):
    """Packed-token buckets: 1, 2, 4, 8, 16, then steps of 16 to 512 (a decode tick of n slots pads to at most
    15 tokens), steps of 128 to 4096, then steps of 2048."""
    out = [1, 2, 4, 8]
    out += list(range(16, 513, 16))
    out += list(range(640, 4097, 128))
    out += list(range(6144, max(max_tokens, 6144) + 2048, 2048))
    out = sorted({b for b in out if b < max_tokens} | {max_tokens})
    return tuple(out)


def pack_ticks(chunks, slots, length, nb, tb, max_slots, out):
    """Packed tick layout in one int64 buffer ``[ids tb | pos tb | offsets nb | lens nb | slots nb | starts nb]``.

    Rows n >= len(chunks) are padding: offset = total tokens, len 0, the scratch slot ``max_slots``, start 0
    (the packed counterpart of pack_inputs, src/hs_guard/engine/slot_engine_v7.py:7-25). Token positions
    beyond the real tokens carry id 0 and position 0. Returns (lens [n], offsets [n])."""
    n = len(chunks)
    lens = np.fromiter(map(len, chunks), dtype=np.int64, count=n)
    total = int(lens.sum())
    ids = out[:tb]
    pos = out[tb:2 * tb]
    offs = out[2 * tb:2 * tb + nb]
    lns = out[2 * tb + nb:2 * tb + 2 * nb]
    sls = out[2 * tb + 2 * nb:2 * tb + 3 * nb]
    sts = out[2 * tb + 3 * nb:2 * tb + 4 * nb]
    ids[:total] = np.fromiter(itertools.chain.from_iterable(chunks), dtype=np.int64, count=total)
    ids[total:] = 0
    offsets = np.zeros(n, dtype=np.int64)
    if n > 1:
        np.cumsum(lens[:-1], out=offsets[1:])
    starts = np.asarray(length, dtype=np.int64)[slots]
    pos[:total] = np.repeat(starts - offsets, lens) + np.arange(total, dtype=np.int64)
    pos[total:] = 0
    offs[:n] = offsets
    offs[n:] = total
    lns[:n] = lens
    lns[n:] = 0
    sls[:n] = slots
    sls[n:] = max_slots
    sts[:n] = starts
    sts[n:] = 0
    return lens, offsets


def gdn_proj_width(cfg):
    """Columns of a GDN layer's fused projection qkv|z|b|a, padded with zero weight rows to a multiple of 256:
    hipBLASLt serves N = 8,224 (the baseline geometry) with a stream-K kernel at 38-40 us for M ~ 1,500 tokens
    and N = 8,448 with a regular one at 27-31 us. The padding columns are computed and never read."""
    n = cfg.conv_dim + cfg.value_dim + 2 * cfg.linear_num_value_heads
    return -(-n // 256) * 256


def request_order(flat, lens, offsets):
    """Tick outputs [R, T, 3] (row r at positions offsets[r] .. offsets[r] + lens[r] - 1) gathered so that the
    rows follow one another in request order: row r then starts at sum(lens[:r])."""
    starts = np.zeros(len(lens), dtype=np.int64)
    if len(lens) > 1:
        np.cumsum(lens[:-1], out=starts[1:])
    gather = np.repeat(np.asarray(offsets, dtype=np.int64) - starts, lens) + np.arange(int(np.sum(lens)),
                                                                                         dtype=np.int64)
    return np.ascontiguousarray(flat[:, gather])


def padded_rows(flat, lens, offsets, lb):
    """Tick outputs [R, T, 3] (row r at positions offsets[r] .. offsets[r] + lens[r] - 1) as [R, n, lb, 3] with
    request r's outputs at [:, r, :lens[r]] and zeros after (step_packed's layout), in one scatter."""
    lens = np.asarray(lens, dtype=np.int64)
    n = len(lens)
    out = np.zeros((flat.shape[0], n, lb, 3), dtype=np.float32)
    row = np.repeat(np.arange(n, dtype=np.int64), lens)
    col = np.arange(int(lens.sum()), dtype=np.int64) - np.repeat(np.cumsum(lens) - lens, lens)
    out[:, row, col] = flat[:, np.repeat(np.asarray(offsets, dtype=np.int64), lens) + col]
    return out


class PreparedWeights:
    """The backbone's weights in the kernels' layouts: fused projections (GDN qkv|z|b|a, attention q|k|v, MLP
    gate|up, both heads' first Linear), RMSNorm gains as fp32 1 + w, rotary inverse frequencies. Needs
    ``model``, ``cfg``, ``kind``, ``roles`` and ``device`` set."""

    @classmethod
    def of(cls, model, roles=ROLES):
        """The prepared weights of ``model`` alone (no pools, no kernels), on the model's device."""
        self = cls.__new__(cls)
        self.model, self.cfg, self.roles, self.device = model, model.config, tuple(roles), model.device
        types = list(self.cfg.layer_types)
        self.kind = [(t, sum(1 for u in types[:i] if u == t)) for i, t in enumerate(types)]
        self._prepare_weights()
        return self

    def _prepare_weights(self):
        m, cfg = self.model, self.cfg
        f32 = torch.float32
        self.layers = []
        for i, (kind, _) in enumerate(self.kind):
            p = f"backbone.layers.{i}."
            L = {"in_w1": (1.0 + m[p + "input_layernorm.weight"].float()).contiguous(),
                 "post_w1": (1.0 + m[p + "post_attention_layernorm.weight"].float()).contiguous(),
                 "w_gu": torch.cat([m[p + "mlp.gate_proj.weight"], m[p + "mlp.up_proj.weight"]]).contiguous(),
                 "w_down": m[p + "mlp.down_proj.weight"].contiguous()}
            if kind == "linear_attention":
                a = p + "linear_attn."
                w_in = torch.cat([m[a + "in_proj_qkv.weight"], m[a + "in_proj_z.weight"],
                                  m[a + "in_proj_b.weight"], m[a + "in_proj_a.weight"]])
                pad = gdn_proj_width(cfg) - w_in.shape[0]
                L["w_in"] = torch.cat([w_in, w_in.new_zeros(pad, w_in.shape[1])]).contiguous()
                L["conv_w"] = m[a + "conv1d.weight"].reshape(cfg.conv_dim, -1).contiguous()
                L["A_log"] = m[a + "A_log"].contiguous()
                L["dt_bias"] = m[a + "dt_bias"].contiguous()
                L["norm_w"] = m[a + "norm.weight"].contiguous()
                L["w_out"] = m[a + "out_proj.weight"].contiguous()
            else:
                a = p + "self_attn."
                L["w_in"] = torch.cat([m[a + "q_proj.weight"], m[a + "k_proj.weight"],
                                       m[a + "v_proj.weight"]]).contiguous()
                L["q_w1"] = (1.0 + m[a + "q_norm.weight"].float()).contiguous()
                L["k_w1"] = (1.0 + m[a + "k_norm.weight"].float()).contiguous()
                L["w_out"] = m[a + "o_proj.weight"].contiguous()
            self.layers.append(L)
        self.final_w1 = (1.0 + m["backbone.norm.weight"].float()).contiguous()
        self.emb = m["backbone.embed_tokens.weight"].contiguous()
        rot = cfg.rotary_dim
        self.inv_freq = (1.0 / (cfg.rope_theta ** (torch.arange(0, rot, 2, dtype=f32) / rot))).to(self.device)
        # streaming readout (slot_engine_v7.py:44-61): both Linears' weights and biases cast to bf16, the
        # LayerNorm in float32
        bf16 = torch.bfloat16
        self.head_w1 = torch.cat([m[f"heads.{r}.projection.0.weight"] for r in self.roles]).to(bf16).contiguous()
        self.head_b1 = torch.cat([m[f"heads.{r}.projection.0.bias"] for r in self.roles]).to(bf16).contiguous()
        self.head_ln_w = torch.stack([m[f"heads.{r}.projection.1.weight"] for r in self.roles]).float().contiguous()
        self.head_ln_b = torch.stack([m[f"heads.{r}.projection.1.bias"] for r in self.roles]).float().contiguous()
        self.head_w2 = torch.stack([m[f"heads.{r}.risk.weight"] for r in self.roles]).to(bf16).contiguous()
        self.head_b2 = torch.stack([m[f"heads.{r}.risk.bias"] for r in self.roles]).to(bf16).contiguous()


class SlotStreamEngine(PreparedWeights):
    """Fixed per-slot state for ``max_slots`` live streams (row ``max_slots`` of every pool is the scratch
    slot of padding rows)."""

    def __init__(self, model: GuardModel, max_slots, state_dtype="float32", use_graphs=True, roles=ROLES,
                 session_buckets=None, max_tick_tokens=64, chunk_min_tokens=16, fuse_conv=True,
                 gdn_burst_min=HSG_GDN_BURST_MIN_DEFAULT, gemm_skinny_rows=HSG_GEMM_SKINNY_M_MAX):
        if not isinstance(max_slots, int) or max_slots < 1:
            raise ValueError("max_slots must be a positive integer")
        if state_dtype not in STATE_DTYPES:
            raise ValueError("state_dtype must be float32 or float16")
        if not 1 <= max_tick_tokens <= 64:
            raise ValueError("max_tick_tokens must be in [1, 64]")
        if chunk_min_tokens < 0:
            raise ValueError("chunk_min_tokens must be >= 0")
        # In prefill-like ticks (at least 8 tokens per row on average: initial contexts and re-prefills) the GDN
        # rows of at least chunk_min_tokens tokens go to the chunked kernels (WY/UT form on MFMA, one launch set
        # for the tick's long rows); every other row, and every row of a mixed or decode tick, runs the slot step.
        # 0 keeps every row on the slot step. In a mixed tick the few long rows do not repay the chunk path's
        # extra launches (conv, prep, order, state, gate per layer), so those stay with the slot step.
        self.chunk_min_tokens = chunk_min_tokens
        # slot-step rows of at least gdn_burst_min tokens run 8 tokens at a time in the chunk form on MFMA inside
        # the slot-step kernel (no extra launch); 0 runs every row token by token
        if gdn_burst_min < 0:
            raise ValueError("gdn_burst_min must be >= 0")
        self.gdn_burst_min = int(gdn_burst_min)
        # projections of at most gemm_skinny_rows tokens (the small decode ticks) run on hsg_gemm_bf16_skinny, which
        # streams the weights at HBM rate where hipBLASLt's smallest tiles do not; 0 sends every product to hipBLASLt
        if not 0 <= gemm_skinny_rows <= HSG_GEMM_SKINNY_M_MAX:
            raise ValueError(f"gemm_skinny_rows must be in [0, {HSG_GEMM_SKINNY_M_MAX}]")
        self.gemm_skinny_rows = int(gemm_skinny_rows)
        lib()  # fail loudly here if the HIP library is missing
        cfg = model.config
        # the GDN layers' causal conv runs inside the slot step (hsg_gdn_conv_slot_step_gated) when every value
        # head has its own key head and no rows of the tick go to the chunk kernels; otherwise as its own kernel
        self.fuse_conv = bool(fuse_conv) and cfg.linear_num_value_heads == cfg.linear_num_key_heads
        self.model, self.cfg = model, cfg
        self.max_slots, self.roles, self.use_graphs = max_slots, tuple(roles), use_graphs
        self.window = cfg.window_tokens
        # a tick never holds more steps than the window: its steps then own distinct ring columns
        self.max_tick_tokens = min(max_tick_tokens, self.window)
        if session_buckets is None:
            session_buckets = tuple(x for x in SESSION_BUCKETS if x <= max_slots)
            if not session_buckets or session_buckets[-1] != max_slots:
                session_buckets += (max_slots,)
        self.session_buckets = tuple(session_buckets)
        self.max_rows = self.session_buckets[-1]
        self.max_tokens = self.max_rows * self.max_tick_tokens
        self.token_buckets = token_buckets(self.max_tokens)
        types = list(cfg.layer_types)
        self.kind = [(t, sum(1 for u in types[:i] if u == t)) for i, t in enumerate(types)]
        n_gdn, n_att = types.count("linear_attention"), types.count("full_attention")
        dev = model.device
        self.device = dev
        S = max_slots + 1
        bf16 = torch.bfloat16
        self.state_dtype = STATE_DTYPES[state_dtype]
        # ---- per-slot pools (layouts of src/hs_guard/engine/bucketed_engine.py:37-45, slot_engine.py:14-17) ----
        self.rec = torch.zeros(n_gdn, S, cfg.linear_num_value_heads, cfg.linear_key_head_dim,
                               cfg.linear_value_head_dim, dtype=self.state_dtype, device=dev)
        self.conv = torch.zeros(n_gdn, S, cfg.linear_conv_kernel_dim - 1, cfg.conv_dim, dtype=bf16, device=dev)
        self.ring_k = torch.zeros(n_att, S, cfg.num_key_value_heads, self.window + 1, cfg.head_dim, dtype=bf16,
                                  device=dev)
        self.ring_v = torch.zeros_like(self.ring_k)
        self.ring_pos = torch.full((S, self.window + 1), -1, dtype=torch.long, device=dev)
        self.length = np.zeros(max_slots, dtype=np.int64)
        self.stats = {"graph_replays": 0, "eager_steps": 0, "captures": 0}
        self.graphs = {}
        self.pool = None
        self._prepare_weights()
        self._allocate_buffers()

    # ------------------------------------------------------------------------------------------------
    def _allocate_buffers(self):
        cfg, T, dev = self.cfg, self.max_tokens, self.device
        bf16 = torch.bfloat16
        hq, hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.gdn_in = gdn_proj_width(cfg)       # row stride of the GDN projection (padded, see gdn_proj_width)
        self.att_in = hq * 2 * D + 2 * hkv * D
        widest = max(self.gdn_in, self.att_in, 2 * cfg.intermediate_size)
        self.buf = {
            "hidden": torch.zeros(T * cfg.hidden_size, dtype=bf16, device=dev),
            # the residual stream's second buffer for ticks whose add + RMSNorm runs inside the next product
            "hidden2": torch.zeros(max(self.gemm_skinny_rows, 1) * cfg.hidden_size, dtype=bf16, device=dev),
            "normed": torch.zeros(T * cfg.hidden_size, dtype=bf16, device=dev),
            "mix": torch.zeros(T * cfg.hidden_size, dtype=bf16, device=dev),
            "proj": torch.zeros(T * widest, dtype=bf16, device=dev),
            "conv": torch.zeros(T * cfg.conv_dim, dtype=bf16, device=dev),
            "mid": torch.zeros(T * max(cfg.value_dim, hq * D, cfg.intermediate_size), dtype=bf16, device=dev),
            "q": torch.zeros(T * hq * D, dtype=bf16, device=dev),
            "k": torch.zeros(T * hkv * D, dtype=bf16, device=dev),
            "head": torch.zeros(T * cfg.head_hidden * len(self.roles), dtype=bf16, device=dev),
            "probs": torch.zeros(len(self.roles) * T * 3, dtype=torch.float32, device=dev),
            "inputs": torch.zeros(2 * T + 4 * self.max_rows, dtype=torch.long, device=dev),
        }
        # hipBLASLt workspace of the projection GEMMs and their committed solution table (hs_guard/engine/gemm_plan.py)
        self.gemm_plans = GemmPlans.load()
        self.gemm_ws = torch.empty(GEMM_WORKSPACE_BYTES, dtype=torch.uint8, device=dev)
        # decode workspace for the single-step rows of a tick (used by hsg_ring_decode above 8 query heads per kv head)
        ws = lib().hsg_ring_decode_workspace_bytes(self.max_rows, hkv, hq // hkv, self.window)
        self.ring_ws = torch.empty(max(int(ws), 16), dtype=torch.uint8, device=dev)
        # chunked-GDN scratch for the long rows of a tick (one 64-token chunk per row) and their raw outputs
        if self.chunk_min_tokens:
            ws = lib().hsg_gdn_chunk_workspace_bytes(self.max_rows, self.max_tick_tokens, cfg.linear_num_value_heads)
            self.chunk_ws = torch.empty(max(int(ws), 256), dtype=torch.uint8, device=dev)
            self.buf["gdn_o"] = torch.zeros(T * cfg.value_dim, dtype=bf16, device=dev)

    def mm(self, x, w, out):
        """out[M, N] = x[M, K] . w[N, K]^T (bf16, row-major, unit column stride) on the current stream: through
        hsg_gemm_bf16_skinny for M <= gemm_skinny_rows (when K, the row strides and the operands are aligned as it
        needs), else through hsg_gemm_bf16 with the committed solution for (M, N, K) (hipBLASLt's first heuristic
        candidate for shapes the table lacks). Every projection of the tick goes through here, so a test that wants
        the engine's exact products calls this too."""
        M, K = x.shape
        N = w.shape[0]
        if w.shape[1] != K or out.shape != (M, N) or x.stride(1) != 1 or w.stride(1) != 1 or out.stride(1) != 1:
            raise ValueError("mm: shapes or strides do not match D[M, N] = A[M, K] . W[N, K]^T")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        if self._skinny(x, w, K):
            check(lib().hsg_gemm_bf16_skinny(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(),
                                             out.stride(0), M, N, K, stream), "hsg_gemm_bf16_skinny")
            return out
        index = self.gemm_plans.index(M, N, K)
        rc = lib().hsg_gemm_bf16(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(), out.stride(0),
                                 M, N, K, index, self.gemm_ws.data_ptr(), self.gemm_ws.numel(), stream)
        if rc == HSG_ERR_SHAPE and index >= 0:
            # the running hipBLASLt rejected the table's solution before launching anything: use the heuristic's
            # first candidate for this shape from now on
            warnings.warn(f"hipBLASLt rejected solution {index} for ({M}, {N}, {K}); using its heuristic instead")
            self.gemm_plans.drop(M, N, K)
            rc = lib().hsg_gemm_bf16(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(),
                                     out.stride(0), M, N, K, -1, self.gemm_ws.data_ptr(), self.gemm_ws.numel(), stream)
        check(rc, "hsg_gemm_bf16")
        return out

    def _skinny(self, x, w, K):
        """Whether the product of x's rows with w ([N, K]) runs on the skinny kernels."""
        return (x.shape[0] <= self.gemm_skinny_rows and K % 8 == 0 and x.stride(0) % 8 == 0 and w.stride(0) % 8 == 0
                and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0)

    def mm_silu(self, gu, w, out, act):
        """out[M, N] = act . w[N, I]^T with act = bf16(bf16(silu(gu[:, :I])) * gu[:, I:]) (the MLP's SiLU gate and
        down projection, src/hs_guard/engine/slot_engine_v8.py:52-53): one hsg_gemm_bf16_skinny_silu launch when
        the skinny route applies (act is not written), else hsg_silu_mul into ``act`` and ``mm``. Bitwise the same
        either way."""
        M, I = gu.shape[0], gu.shape[1] // 2
        if w.shape[1] != I or out.shape != (M, w.shape[0]) or gu.stride(1) != 1 or out.stride(1) != 1:
            raise ValueError("mm_silu: shapes or strides do not match")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        if self._skinny(gu, w, I) and w.stride(1) == 1:
            check(lib().hsg_gemm_bf16_skinny_silu(gu.data_ptr(), gu.stride(0), w.data_ptr(), w.stride(0),
                                                  out.data_ptr(), out.stride(0), M, w.shape[0], I, stream),
                  "hsg_gemm_bf16_skinny_silu")
            return out
        check(lib().hsg_silu_mul(gu.data_ptr(), gu.stride(0), I, act.data_ptr(), M, stream), "hsg_silu_mul")
        return self.mm(act, w, out)

    def _view(self, name, *shape):
        n = 1
        for s in shape:
            n *= s
        return self.buf[name][:n].view(*shape)

    # ------------------------------------------------------------------------------------------------
    def state_bytes_per_session(self):
        tensors = (self.rec, self.conv, self.ring_k, self.ring_v, self.ring_pos)
        return sum(t.element_size() * t.numel() for t in tensors) // (self.max_slots + 1)

    def reset(self, slots=None):
        """Zero the state of every slot (``slots=None``, the reference's reset,
        src/hs_guard/engine/bucketed_engine.py:51-55) or of the given slots only."""
        if slots is None:
            for t in (self.rec, self.conv, self.ring_k, self.ring_v):
                t.zero_()
            self.ring_pos.fill_(-1)
            self.length = np.zeros(self.max_slots, dtype=np.int64)
            return
        idx = torch.as_tensor(list(slots), dtype=torch.long, device=self.device)
        self.rec[:, idx] = 0
        self.conv[:, idx] = 0
        self.ring_k[:, idx] = 0
        self.ring_v[:, idx] = 0
        self.ring_pos[idx] = -1
        self.length[idx.cpu().numpy()] = 0

    def snapshot(self, slot):
        """Copy of one slot's state (the pool rows examples/demo/runtime_v10.py:117-122 clones)."""
        return {"rec": self.rec[:, slot].clone(), "conv": self.conv[:, slot].clone(),
                "ring_k": self.ring_k[:, slot].clone(), "ring_v": self.ring_v[:, slot].clone(),
                "ring_pos": self.ring_pos[slot].clone(), "length": int(self.length[slot])}

    def restore(self, slot, snap):
        """Write a snapshot back into a slot (examples/demo/runtime_v10.py:98-111)."""
        self.rec[:, slot] = snap["rec"]
        self.conv[:, slot] = snap["conv"]
        self.ring_k[:, slot] = snap["ring_k"]
        self.ring_v[:, slot] = snap["ring_v"]
        self.ring_pos[slot] = snap["ring_pos"]
        self.length[slot] = snap["length"]

    # ------------------------------------------------------------------------------------------------
    def _inputs(self, nb, tb):
        x = self.buf["inputs"]
        return {"ids": x[:tb], "pos": x[tb:2 * tb], "offsets": x[2 * tb:2 * tb + nb],
                "lens": x[2 * tb + nb:2 * tb + 2 * nb], "slots": x[2 * tb + 2 * nb:2 * tb + 3 * nb],
                "starts": x[2 * tb + 3 * nb:2 * tb + 4 * nb], "all": x[:2 * tb + 4 * nb]}

    def _forward(self, nb, tb, inp):
        """The tick's device program (src/hs_guard/engine/slot_engine_v8.py:30-58), launched on the current
        stream. Reads only device memory, so it can be captured into a hipGraph."""
        L = lib()
        cfg = self.cfg
        st = torch.cuda.current_stream(self.device).cuda_stream
        H, W = cfg.hidden_size, self.window
        S = self.max_slots + 1
        eps = cfg.rms_norm_eps
        hq, hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        G = hq // hkv
        nh, hv, kd, vd = cfg.linear_num_key_heads, cfg.linear_num_value_heads, cfg.linear_key_head_dim, \
            cfg.linear_value_head_dim
        ids, pos, offsets, lens, slots, starts = (inp[k] for k in ("ids", "pos", "offsets", "lens", "slots",
                                                                    "starts"))
        hid = [self._view("hidden", tb, H)]
        normed = self._view("normed", tb, H)
        mix = self._view("mix", tb, H)
        check(L.hsg_embed_rmsnorm(ids.data_ptr(), self.emb.data_ptr(), cfg.vocab_size,
                                  self.layers[0]["in_w1"].data_ptr(), eps, hid[0].data_ptr(), normed.data_ptr(), tb,
                                  H, st), "hsg_embed_rmsnorm")
        # Each residual add + RMSNorm (hidden += mix, normed = norm(hidden) * w1) is applied by the product that
        # reads normed. In ticks of at most gemm_skinny_rows tokens both run in one hsg_gemm_bf16_skinny_addnorm
        # launch, which writes the residual to the other of two buffers (hid[0] -> hid[1] -> hid[0] ...); otherwise
        # hsg_add_rmsnorm updates hid[0] in place and the product follows.
        fuse = tb <= self.gemm_skinny_rows and H == 1024
        if fuse:
            hid.append(self._view("hidden2", tb, H))
        pending = []    # the (mix, w1) of an add + RMSNorm not yet applied

        def norm_mm(w, out):
            if not pending:
                return self.mm(normed, w, out)
            mx, w1 = pending.pop()
            if fuse and self._skinny(normed, w, H):
                check(L.hsg_gemm_bf16_skinny_addnorm(hid[0].data_ptr(), H, mx.data_ptr(), H, w1.data_ptr(), eps,
                                                     hid[1].data_ptr(), H, w.data_ptr(), w.stride(0),
                                                     out.data_ptr(), out.stride(0), tb, w.shape[0], H, None, st),
                      "hsg_gemm_bf16_skinny_addnorm")
                hid.reverse()
                return out
            check(L.hsg_add_rmsnorm(hid[0].data_ptr(), mx.data_ptr(), w1.data_ptr(), eps, normed.data_ptr(), tb, H,
                                    st), "hsg_add_rmsnorm")
            return self.mm(normed, w, out)

        for i, ((kind, idx), Lw) in enumerate(zip(self.kind, self.layers)):
            if kind == "linear_attention":
                C = cfg.conv_dim
                proj = self._view("proj", tb, self.gdn_in)
                norm_mm(Lw["w_in"], proj)
                out = self._view("mid", tb, cfg.value_dim)
                base = proj.data_ptr()
                # rows are packed longest first: in a prefill-like tick the rows of >= chunk_min_tokens tokens go
                # to the chunked kernels (one WY/UT chunk each), the rest to the slot step
                R = self._chunk_rows(nb, tb)
                if self.fuse_conv and R == 0:
                    # causal conv + SiLU inside the slot step, from the raw projection and the conv history pool
                    check(L.hsg_gdn_conv_slot_step_gated(
                        base, self.gdn_in, 0, cfg.key_dim, 2 * cfg.key_dim, Lw["conv_w"].data_ptr(),
                        self.conv[idx].data_ptr(), C, base + 2 * (C + cfg.value_dim + hv),
                        base + 2 * (C + cfg.value_dim), self.gdn_in, Lw["A_log"].data_ptr(), Lw["dt_bias"].data_ptr(),
                        self.rec[idx].data_ptr(), _STATE_CODE[self.state_dtype], S, slots.data_ptr(), lens.data_ptr(),
                        offsets.data_ptr(), nb, nh, hv, kd, vd, kd ** -0.5, base + 2 * C, self.gdn_in,
                        Lw["norm_w"].data_ptr(), eps, out.data_ptr(), self.gdn_burst_min, st),
                          "hsg_gdn_conv_slot_step_gated")
                else:
                    conv = self._view("conv", tb, C)
                    check(L.hsg_conv_silu_update(proj.data_ptr(), self.gdn_in, self.conv[idx].data_ptr(), S,
                                                 Lw["conv_w"].data_ptr(), cfg.linear_conv_kernel_dim,
                                                 slots.data_ptr(), lens.data_ptr(), offsets.data_ptr(), nb, 0, C,
                                                 conv.data_ptr(), C, st), "hsg_conv_silu_update")
                    check(L.hsg_gdn_slot_step_gated(
                        conv.data_ptr(), C, 0, cfg.key_dim, 2 * cfg.key_dim,
                        base + 2 * (C + cfg.value_dim + hv), base + 2 * (C + cfg.value_dim), self.gdn_in,
                        Lw["A_log"].data_ptr(), Lw["dt_bias"].data_ptr(), self.rec[idx].data_ptr(),
                        _STATE_CODE[self.state_dtype], S, slots.data_ptr(), lens.data_ptr(), offsets.data_ptr(), nb,
                        0, nh, hv, kd, vd, kd ** -0.5, base + 2 * C, self.gdn_in, Lw["norm_w"].data_ptr(), eps,
                        out.data_ptr(), R, max(self.chunk_min_tokens, 1), self.gdn_burst_min, st),
                          "hsg_gdn_slot_step_gated")
                    if R:
                        check(L.hsg_gdn_chunk_prefill_gated(
                            conv.data_ptr(), C, 0, cfg.key_dim, 2 * cfg.key_dim,
                            base + 2 * (C + cfg.value_dim + hv), base + 2 * (C + cfg.value_dim), self.gdn_in,
                            Lw["A_log"].data_ptr(), Lw["dt_bias"].data_ptr(), self.rec[idx].data_ptr(),
                            _STATE_CODE[self.state_dtype], S, slots.data_ptr(), lens.data_ptr(), offsets.data_ptr(),
                            R, self.max_tick_tokens, nh, hv, kd, vd, kd ** -0.5,
                            self._view("gdn_o", tb, cfg.value_dim).data_ptr(), base + 2 * C, self.gdn_in,
                            Lw["norm_w"].data_ptr(), eps, out.data_ptr(), self.chunk_min_tokens,
                            self.chunk_ws.data_ptr(), self.chunk_ws.numel(), st), "hsg_gdn_chunk_prefill_gated")
                self.mm(out, Lw["w_out"], mix)
            else:
                proj = self._view("proj", tb, self.att_in)
                norm_mm(Lw["w_in"], proj)
                q = self._view("q", tb, hq * D)
                k = self._view("k", tb, hkv * D)
                base = proj.data_ptr()
                att = self._view("mid", tb, hq * D)
                if tb == 1 and cfg.rotary_dim == 64 and D == 256:
                    # a one-token tick: the q / k norm and RoPE run inside the decode's scores kernel (one launch
                    # fewer), bitwise hsg_norm_rope + hsg_ring_decode; k receives the new keys
                    check(L.hsg_ring_decode_rope(
                        base, self.att_in, 2 * D, Lw["q_w1"].data_ptr(), eps,
                        base + 2 * hq * 2 * D, self.att_in, D, Lw["k_w1"].data_ptr(), eps,
                        pos.data_ptr(), self.inv_freq.data_ptr(), cfg.rotary_dim, k.data_ptr(), hkv * D,
                        self.ring_k[idx].data_ptr(), self.ring_v[idx].data_ptr(), S, W,
                        base + 2 * (hq * 2 * D + hkv * D), self.att_in, D,
                        base, self.att_in, G * 2 * D, 2 * D, D,
                        self.ring_pos.data_ptr(), slots.data_ptr(), starts.data_ptr(), lens.data_ptr(),
                        offsets.data_ptr(), nb, hkv, G, D, D ** -0.5, 1,
                        att.data_ptr(), hq * D, G * D, D, self.ring_ws.data_ptr(), self.ring_ws.numel(), st),
                        "hsg_ring_decode_rope")
                else:
                    check(L.hsg_norm_rope(base, self.att_in, 2 * D, hq, Lw["q_w1"].data_ptr(), eps, q.data_ptr(),
                                          hq * D, D, base + 2 * hq * 2 * D, self.att_in, D, hkv,
                                          Lw["k_w1"].data_ptr(), eps, k.data_ptr(), hkv * D, D, pos.data_ptr(),
                                          self.inv_freq.data_ptr(), cfg.rotary_dim, tb, D, st), "hsg_norm_rope")
                    # single-step rows: hsg_ring_decode; rows of two or more steps: the tiled kernel (min_len 2)
                    check(L.hsg_ring_decode(
                        q.data_ptr(), 0, hq * D, G * D, D,
                        self.ring_k[idx].data_ptr(), self.ring_v[idx].data_ptr(), S, W,
                        k.data_ptr(), 0, hkv * D, D,
                        base + 2 * (hq * 2 * D + hkv * D), 0, self.att_in, D,
                        base, 0, self.att_in, G * 2 * D, 2 * D, D,
                        self.ring_pos.data_ptr(), slots.data_ptr(), starts.data_ptr(), lens.data_ptr(),
                        offsets.data_ptr(), nb, hkv, G, D, D ** -0.5, 1,
                        att.data_ptr(), 0, hq * D, G * D, D, self.ring_ws.data_ptr(), self.ring_ws.numel(), st),
                        "hsg_ring_decode")
                    if tb >= 2:
                        # a one-token bucket has no row of two or more steps: its program leaves the tiled kernel
                        # out
                        check(L.hsg_ring_attention(
                            q.data_ptr(), 0, hq * D, G * D, D,
                            self.ring_k[idx].data_ptr(), self.ring_v[idx].data_ptr(), S, W,
                            k.data_ptr(), 0, hkv * D, D,
                            base + 2 * (hq * 2 * D + hkv * D), 0, self.att_in, D,
                            base, 0, self.att_in, G * 2 * D, 2 * D, D,
                            self.ring_pos.data_ptr(), slots.data_ptr(), starts.data_ptr(), lens.data_ptr(),
                            offsets.data_ptr(), nb, self.max_tick_tokens, hkv, G, D, D ** -0.5, 1, 2,
                            att.data_ptr(), 0, hq * D, G * D, D, st), "hsg_ring_attention")
                self.mm(att, Lw["w_out"], mix)
            pending.append((mix, Lw["post_w1"]))
            I = cfg.intermediate_size
            gu = self._view("proj", tb, 2 * I)
            norm_mm(Lw["w_gu"], gu)
            self.mm_silu(gu, Lw["w_down"], mix, self._view("mid", tb, I))
            nxt = self.layers[i + 1]["in_w1"] if i + 1 < len(self.layers) else self.final_w1
            pending.append((mix, nxt))
        # the final norm feeds the heads' first Linear (with bias): one skinny launch in small ticks, else the norm
        # and torch.addmm
        mx, w1 = pending.pop()
        R, E = len(self.roles), cfg.head_hidden
        y = self._view("head", tb, R * E)
        if fuse and self._skinny(normed, self.head_w1, H):
            check(L.hsg_gemm_bf16_skinny_addnorm(hid[0].data_ptr(), H, mx.data_ptr(), H, w1.data_ptr(), eps,
                                                 hid[1].data_ptr(), H, self.head_w1.data_ptr(), self.head_w1.stride(0),
                                                 y.data_ptr(), y.stride(0), tb, R * E, H, self.head_b1.data_ptr(), st),
                  "hsg_gemm_bf16_skinny_addnorm")
        else:
            check(L.hsg_add_rmsnorm(hid[0].data_ptr(), mx.data_ptr(), w1.data_ptr(), eps, normed.data_ptr(), tb, H,
                                    st), "hsg_add_rmsnorm")
            torch.addmm(self.head_b1, normed, self.head_w1.t(), out=y)
        probs = self._view("probs", R, tb, 3)
        check(L.hsg_risk_head(y.data_ptr(), R * E, self.head_ln_w.data_ptr(), self.head_ln_b.data_ptr(),
                              self.head_w2.data_ptr(), self.head_b2.data_ptr(), cfg.layer_norm_eps, R, E,
                              probs.data_ptr(), tb, st), "hsg_risk_head")
        check(L.hsg_ring_pos_update(self.ring_pos.data_ptr(), S, W, slots.data_ptr(), starts.data_ptr(),
                                    lens.data_ptr(), nb, self.max_tick_tokens, st), "hsg_ring_pos_update")
        return probs

    def _chunk_rows(self, nb, tb):
        """How many leading rows of an (nb, tb) tick may take the chunked GDN path (a constant per graph): every
        row when the tick is prefill-like (>= 8 tokens per row on average), else none."""
        if not self.chunk_min_tokens or tb < 8 * nb:
            return 0
        return nb

    def _static(self, nb, tb):
        key = (nb, tb)
        if key not in self.graphs:
            inp = self._inputs(nb, tb)
            inp["all"].zero_()
            inp["slots"].fill_(self.max_slots)       # empty rows on the scratch slot: no state is touched
            graph = None
            if self.use_graphs:
                side = torch.cuda.Stream(self.device)
                side.wait_stream(torch.cuda.current_stream(self.device))
                with torch.cuda.stream(side):
                    for _ in range(2):
                        self._forward(nb, tb, inp)
                torch.cuda.current_stream(self.device).wait_stream(side)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=self.pool):
                    probs = self._forward(nb, tb, inp)
                self.pool = graph.pool()
                self.stats["captures"] += 1
                # the first replay of a graph pays a one-time upload; pay it here (inputs still address only
                # the scratch slot with zero-length rows, so no state changes)
                graph.replay()
                torch.cuda.current_stream(self.device).synchronize()
            else:
                probs = self._view("probs", len(self.roles), tb, 3)
            host_in = torch.zeros(2 * tb + 4 * nb, dtype=torch.long, pin_memory=True)
            host_out = torch.zeros(len(self.roles), tb, 3, dtype=torch.float32, pin_memory=True)
            self.graphs[key] = (graph, inp, probs, host_in, host_in.numpy(), host_out, host_out.numpy())
        return self.graphs[key]

    @torch.inference_mode()
    def prepare(self, rows, token_counts):
        """Capture ahead of time the step graphs for ticks of ``rows`` rows and each total token count in
        ``token_counts`` (by bucket), so that a serving loop never pays a capture inside a tick."""
        nb = bucket(rows, self.session_buckets)
        for tb in sorted({bucket(t, self.token_buckets) for t in token_counts}):
            self._static(nb, tb)

    def _run_arrays(self, chunks, slots):
        """One tick: <= max_rows rows of <= max_tick_tokens tokens. Returns (probs [R, T, 3] numpy, lens,
        offsets) with row r's probabilities at [:, offsets[r] : offsets[r] + lens[r]]."""
        n = len(chunks)
        row_lens = np.fromiter(map(len, chunks), dtype=np.int64, count=n)
        total = int(row_lens.sum())
        nb = bucket(n, self.session_buckets)
        tb = bucket(total, self.token_buckets)
        graph, inp, probs, host_in, host_np, host_out, out_np = self._static(nb, tb)
        # rows go to the device longest first: the per-row kernels then start their longest rows first
        # instead of finishing on them (every kernel treats rows independently, so results do not change)
        order = np.argsort(-row_lens, kind="stable")
        lens_p, offsets_p = pack_ticks([chunks[r] for r in order], np.asarray(slots)[order], self.length, nb, tb,
                                       self.max_slots, host_np)
        lens = np.empty(n, dtype=np.int64)
        offsets = np.empty(n, dtype=np.int64)
        lens[order] = lens_p
        offsets[order] = offsets_p
        self._replay(nb, tb, graph, inp, probs, host_in, host_out)
        self.length[slots] += lens
        return out_np[:, :total].copy(), lens, offsets

    def _validate(self, requests):
        slots = [s for s, _ in requests]
        if len(set(slots)) != len(slots):
            raise ValueError("a session may appear once per tick")
        for s, ids in requests:
            if not 0 <= s < self.max_slots:
                raise ValueError("Slot is outside the allocated range")
            if len(ids) == 0:
                raise ValueError("Each request requires nonempty token IDs")
            a = np.asarray(ids)
            if a.dtype.kind not in "iu" or a.ndim != 1 or int(a.min()) < 0 or int(a.max()) >= self.cfg.vocab_size:
                # the reference's contract (docs/ENGINE.md:9): the embedding gather must never see an id it lacks
                raise ValueError("Each request requires nonempty in-vocabulary integer token IDs")

    def _replay(self, nb, tb, graph, inp, probs, host_in, host_out):
        """Send the packed inputs, run the tick (graph replay, or eagerly without graphs) and bring the
        probabilities back; returns when they are on the host."""
        inp["all"].copy_(host_in, non_blocking=True)
        if graph is not None:
            graph.replay()
            self.stats["graph_replays"] += 1
        else:
            probs = self._forward(nb, tb, inp)
            self.stats["eager_steps"] += 1
        host_out.copy_(probs, non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()

    def _run_native(self, requests, n, total):
        """One tick of requests that passed _hostpack.scan (n rows, total tokens, within the tick limits), packed
        by _hostpack.fill. Returns (outputs [R, tb, 3] numpy, valid until the next tick of the same shape, tb,
        lens [n], offsets [n]) with request r's outputs at [:, offsets[r] : offsets[r] + lens[r]]."""
        nb = bucket(n, self.session_buckets)
        tb = bucket(total, self.token_buckets)
        graph, inp, probs, host_in, host_np, host_out, out_np = self._static(nb, tb)
        lens = np.empty(n, dtype=np.int64)
        offsets = np.empty(n, dtype=np.int64)
        slots = np.empty(n, dtype=np.int64)
        _hostpack.fill(requests, self.length, nb, tb, self.max_slots, self.cfg.vocab_size, host_np, lens, offsets,
                       slots)
        self._replay(nb, tb, graph, inp, probs, host_in, host_out)
        self.length[slots] += lens
        return out_np, tb, lens, offsets

    @torch.inference_mode()
    def step_packed(self, requests):
        """One tick without per-row objects (src/hs_guard/engine/slot_engine_v7.py:138-145): requests as
        step(), each <= max_tick_tokens tokens and at most the largest session bucket of them. Returns
        (probs [R, n, lb, 3] numpy, lens [n]); row r holds request r's first lens[r] positions.

        The host work runs in hs_guard._hostpack (checks, packing, the padded result): the same layout and
        values as pack_ticks / padded_rows, at a few microseconds instead of a few hundred per tick."""
        scan = _hostpack.scan(requests, self.max_slots, self.cfg.vocab_size)
        if scan is not None and scan[0] > 0:
            n, total, max_len = scan
            if n > self.max_rows or max_len > self.max_tick_tokens:
                raise ValueError("step_packed takes one tick: too many rows or tokens")
            out_np, tb, lens, offsets = self._run_native(requests, n, total)
            lb = bucket(max_len, (1, 2, 4, 8, 16, 32, 64))
            out = np.empty((len(self.roles), n, lb, 3), dtype=np.float32)
            _hostpack.scatter_padded(out_np, len(self.roles), tb, lens, offsets, lb, out)
            return out, lens
        # a request the native checks do not accept: the reference's checks raise its error (or, for inputs they
        # accept, such as non-integer slot types, the numpy route below runs the tick)
        self._validate(requests)
        if len(requests) > self.max_rows or any(len(c) > self.max_tick_tokens for _, c in requests):
            raise ValueError("step_packed takes one tick: too many rows or tokens")
        n = len(requests)
        slots = np.fromiter((s for s, _ in requests), dtype=np.int64, count=n)
        flat, lens, offsets = self._run_arrays([c if isinstance(c, list) else list(c) for _, c in requests], slots)
        lb = bucket(int(lens.max()), (1, 2, 4, 8, 16, 32, 64))
        return padded_rows(flat, lens, offsets, lb), lens

    def one_tick(self, scan):
        """Whether requests whose ``_hostpack.scan`` result is ``scan`` (they passed its checks) fit one tick."""
        return scan is not None and 0 < scan[0] <= self.max_rows and scan[2] <= self.max_tick_tokens

    @torch.inference_mode()
    def step_flat(self, requests, scan):
        """One tick of checked requests (``one_tick(scan)``), host work native: (probabilities [roles, total, 3]
        float32 with the requests' tokens one after another in request order, lens [n] int64)."""
        n, total, _ = scan
        out_np, tb, lens, offsets = self._run_native(requests, n, total)
        flat = np.empty((len(self.roles), total, 3), dtype=np.float32)
        _hostpack.gather_rows(out_np, len(self.roles), tb, lens, offsets, flat)
        return flat, lens

    @torch.inference_mode()
    def step(self, requests):
        """requests: list of (slot, token_ids), each slot at most once. Returns {role: [CPU tensor [L_i, 3]]}
        (src/hs_guard/engine/slot_engine_v7.py:147-167)."""
        scan = _hostpack.scan(requests, self.max_slots, self.cfg.vocab_size)
        if self.one_tick(scan):
            # one tick (the serving case), host work native: the request-ordered outputs split per role
            flat, lens = self.step_flat(requests, scan)
            probs = torch.from_numpy(flat)
            sizes = lens.tolist()
            return {role: list(torch.split(probs[r], sizes)) for r, role in enumerate(self.roles)}
        self._validate(requests)
        largest, rows = self.max_tick_tokens, self.max_rows
        if len(requests) <= rows and all(len(ids) <= largest for _, ids in requests):
            # one tick (the serving case): split the request-ordered outputs directly
            slots = np.fromiter((s for s, _ in requests), dtype=np.int64, count=len(requests))
            flat, lens, offsets = self._run_arrays([ids for _, ids in requests], slots)
            probs = torch.from_numpy(request_order(flat, lens, offsets))
            sizes = lens.tolist()
            return {role: list(torch.split(probs[r], sizes)) for r, role in enumerate(self.roles)}
        results = {role: [[] for _ in requests] for role in self.roles}
        pending = [(i, s, list(ids)) for i, (s, ids) in enumerate(requests)]
        while pending:
            batch = [(i, s, ids[:largest]) for i, s, ids in pending]
            for start in range(0, len(batch), rows):
                part = batch[start:start + rows]
                slots = np.fromiter((s for _, s, _ in part), dtype=np.int64, count=len(part))
                flat, lens, offsets = self._run_arrays([c for _, _, c in part], slots)
                # one gather into request order, then one split per role (per-row slicing in Python cost ~700
                # tensor constructions per 352-row tick)
                probs = torch.from_numpy(request_order(flat, lens, offsets))
                sizes = lens.tolist()
                for role_index, role in enumerate(self.roles):
                    for (i, _, _), piece in zip(part, torch.split(probs[role_index], sizes)):
                        results[role][i].append(piece)
            pending = [(i, s, ids[largest:]) for i, s, ids in pending if len(ids) > largest]
        return {role: [chunks[0] if len(chunks) == 1 else torch.cat(chunks) for chunks in rows_]
                for role, rows_ in results.items()}
