/*
 * hsg.h -- C ABI of libhsg.so, the MI355X (gfx950) kernels of HS-Guard's streaming slot step.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers (HIP global memory); sizes and strides are in ELEMENTS.
 *   - bf16 / fp16 tensors are passed as raw 16-bit storage (void*); int64 index tensors as int64_t*.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *   - Nothing allocates, synchronizes or reads device memory on the host, so every call can be
 *     recorded into a hipGraph. Kernels mutate the per-slot pools in place at rows slots[n].
 *   - Row layout: when `offsets` is NULL, row n's tokens are positions n*L .. n*L+L-1 (the reference's
 *     padded [N, L, ...] layout; positions >= lens[n] are written as zeros). When `offsets` is non-NULL
 *     (packed layout) row n's tokens are positions offsets[n] .. offsets[n]+lens[n]-1 and nothing else is
 *     written.
 *   - A row whose slot lies outside [0, state_rows) is treated as empty (lens 0).
 *   - Return value: HSG_OK (0), a negative HSG_ERR_* for a rejected argument (nothing launched), or a
 *     positive hipError_t from the launch.
 *
 * Reference interfaces each entry point replaces are cited as path:line in the HS-Guard repository.
 */
#ifndef HSG_H_
#define HSG_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HSG_OK 0
#define HSG_ERR_ARG (-1)     /* null pointer or non-positive / inconsistent size */
#define HSG_ERR_ALIGN (-2)   /* pointer or stride breaks the vector-load alignment the kernel needs */
#define HSG_ERR_SHAPE (-3)   /* head size / window outside what the kernels are built for */
#define HSG_ERR_BLAS (-4)    /* a hipBLASLt call failed (hsg_gemm_*) */

#define HSG_STATE_F32 0
#define HSG_STATE_F16 1

/* Library version (major*10000 + minor*100 + patch). */
int hsg_version(void);

/* Human-readable text for an HSG_ERR_* or hipError_t code. */
const char* hsg_error_string(int code);

/*
 * Gated-delta-rule recurrent slot step.
 * Replaces gdn_slot_v8 (src/hs_guard/engine/fused_kernels.py:197-211; kernel :140-194) and
 * gdn_slot_recurrent (src/hs_guard/engine/gdn_slot_kernel.py:57-73).
 *   qkv      [tokens, qkv_stride] bf16; q of key head h at q_off + h*K, k at k_off + h*K,
 *            v of value head hv at v_off + hv*V (conv_silu_update output layout).
 *   a, b     [tokens, ab_stride] bf16 raw projections (column hv).
 *   A_log, dt_bias [HV] bf16.
 *   state    [state_rows, HV, K, V] fp32 (state_dtype HSG_STATE_F32) or fp16; V contiguous.
 *   o        [tokens, HV, V] bf16;  sq [tokens, HV, V] fp32 = bf16(o)^2 (sq may be NULL).
 *   burst_min: rows of at least this many tokens (>= 1) run their tokens 8 at a time in the WY/UT chunk form on
 *            fp32 MFMA (the token recurrence unrolled over the burst; equal in exact arithmetic, within fp32
 *            rounding of it); shorter rows, and every row when burst_min is 0, run token by token.
 * Supported: K == V == 128, HV % H == 0.
 */
/* The engine's burst_min: a row of 8-15 tokens would take two bursts (the second partial) for no gain in a mixed
 * tick, whose time the state reads set; from 16 tokens on the bursts shorten the row (a lone 64-token row 70.4 ->
 * 58.0 us on MI355X). */
#define HSG_GDN_BURST_MIN_DEFAULT 16
int hsg_gdn_slot_step(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off, int32_t v_off,
                      const void* a, const void* b, int64_t ab_stride, const void* A_log,
                      const void* dt_bias, void* state, int32_t state_dtype, int64_t state_rows,
                      const int64_t* slots, const int64_t* lens, const int64_t* offsets, int32_t n_rows,
                      int32_t L, int32_t H, int32_t HV, int32_t K, int32_t V, float scale, void* o,
                      float* sq, int32_t burst_min, void* stream);

/*
 * The same step with Qwen3.5's gated RMSNorm fused into the epilogue.
 * Replaces gdn_slot_v8 followed by gated_finish (src/hs_guard/engine/fused_kernels.py:215-233,
 * composed at src/hs_guard/engine/slot_engine_v8.py:67-71):
 *   out[tok, hv*V + c] = bf16( bf16(w[c] * bf16(o*rsqrt(mean(bf16(o)^2)+eps))) * silu(z[tok, hv*V + c]) )
 *   z [tokens, z_stride] bf16, norm_w [V] bf16, out [tokens, HV*V] bf16.
 * Packed layout: rows n < skip_rows with lens[n] >= skip_min_len (>= 1) are left alone (no output, state
 * untouched), for hsg_gdn_chunk_prefill_gated to take; skip_rows 0 processes every row. burst_min as
 * hsg_gdn_slot_step.
 */
int hsg_gdn_slot_step_gated(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off,
                            int32_t v_off, const void* a, const void* b, int64_t ab_stride,
                            const void* A_log, const void* dt_bias, void* state, int32_t state_dtype,
                            int64_t state_rows, const int64_t* slots, const int64_t* lens,
                            const int64_t* offsets, int32_t n_rows, int32_t L, int32_t H, int32_t HV,
                            int32_t K, int32_t V, float scale, const void* z, int64_t z_stride,
                            const void* norm_w, float eps, void* out, int32_t skip_rows, int32_t skip_min_len,
                            int32_t burst_min, void* stream);

/*
 * hsg_gdn_slot_step_gated with the causal conv + SiLU of its inputs fused in (conv_silu_update,
 * src/hs_guard/engine/fused_kernels.py:94-136, followed by gdn_slot_v8 and gated_finish, as composed at
 * src/hs_guard/engine/slot_engine_v8.py:66-71): `proj` holds the raw
 * projection rows (stride proj_stride), whose first `channels` columns are the conv channels with q, k, v at
 * q_off, k_off, v_off; conv_w [channels, 4] bf16; conv_pool [state_rows, 3, channels] bf16, the per-slot conv
 * history, updated in place at slots[n] for rows with lens[n] > 0. Each (row, head) workgroup convolves its own
 * q, k, v channels from the pool and the raw rows, with the conv kernel's arithmetic, so outputs, state and pool
 * equal hsg_conv_silu_update followed by hsg_gdn_slot_step_gated bit for bit (with the same burst_min). Packed
 * rows only (offsets required), HV == H (every q / k channel belongs to one workgroup), no chunk-routing filter.
 * out must not alias proj, z or conv_pool; rows must name distinct slots. burst_min as hsg_gdn_slot_step.
 */
int hsg_gdn_conv_slot_step_gated(const void* proj, int64_t proj_stride, int32_t q_off, int32_t k_off, int32_t v_off,
                                 const void* conv_w, void* conv_pool, int32_t channels, const void* a, const void* b,
                                 int64_t ab_stride, const void* A_log, const void* dt_bias, void* state,
                                 int32_t state_dtype, int64_t state_rows, const int64_t* slots, const int64_t* lens,
                                 const int64_t* offsets, int32_t n_rows, int32_t H, int32_t HV, int32_t K, int32_t V,
                                 float scale, const void* z, int64_t z_stride, const void* norm_w, float eps,
                                 void* out, int32_t burst_min, void* stream);

/*
 * Chunked gated-delta-rule prefill: the same recurrence and contract as hsg_gdn_slot_step, evaluated
 * 64 tokens at a time in the WY/UT chunk form on MFMA, for rows of any length (initial contexts).
 * Replaces FLA's chunk_gated_delta_rule with initial_state = rec[slots] and output_final_state
 * (call sites src/hs_guard/runtime.py:80-89, src/hs_guard/engine/bucketed_engine.py:109-111).
 * Arguments as hsg_gdn_slot_step, except L: the padded row length, and in the packed layout the bound on
 * every row's length (rows with lens[n] > L are treated as empty). o must not alias qkv; o 8-byte and sq
 * 16-byte aligned.
 * Rows with lens[n] < min_len are left alone (min_len <= 1: every row).
 * Three launches on `stream`: the state-independent part of every (row, chunk, value head) in parallel, the
 * rows' order (most chunks first), then the sequential state products per row in that order. workspace: device memory of at least
 * hsg_gdn_chunk_workspace_bytes(n_rows, L, HV) bytes, 256-byte aligned; no initialisation needed, garbage
 * afterwards.
 */
size_t hsg_gdn_chunk_workspace_bytes(int32_t n_rows, int32_t L, int32_t HV);
int hsg_gdn_chunk_prefill(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off, int32_t v_off,
                          const void* a, const void* b, int64_t ab_stride, const void* A_log,
                          const void* dt_bias, void* state, int32_t state_dtype, int64_t state_rows,
                          const int64_t* slots, const int64_t* lens, const int64_t* offsets, int32_t n_rows,
                          int32_t L, int32_t H, int32_t HV, int32_t K, int32_t V, float scale, void* o,
                          float* sq, int32_t min_len, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The same with the gated RMSNorm of hsg_gdn_slot_step_gated applied (packed layout only): o receives the raw
 * outputs of the processed rows, out[tok, hv*V + c] their gated RMSNorm with z (z [tokens, z_stride] bf16,
 * norm_w [V] bf16, out [tokens, HV*V] bf16). A third launch. Together with the skip filter of
 * hsg_gdn_slot_step_gated it splits one tick's rows between the two kernels: rows n < n_rows with
 * lens >= min_len here, the others in the slot step. No counterpart of its own in the reference (it composes
 * chunk_gated_delta_rule and gated_finish, src/hs_guard/engine/fused_kernels.py:215-233).
 */
int hsg_gdn_chunk_prefill_gated(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off, int32_t v_off,
                                const void* a, const void* b, int64_t ab_stride, const void* A_log,
                                const void* dt_bias, void* state, int32_t state_dtype, int64_t state_rows,
                                const int64_t* slots, const int64_t* lens, const int64_t* offsets, int32_t n_rows,
                                int32_t L, int32_t H, int32_t HV, int32_t K, int32_t V, float scale, void* o,
                                const void* z, int64_t z_stride, const void* norm_w, float eps, void* out,
                                int32_t min_len, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Window-W GQA attention of this tick's queries over the slot's ring plus this tick's new keys.
 * Replaces ring_attention_v8 (src/hs_guard/engine/fused_kernels.py:358-376; kernel :288-356),
 * ring_attention (src/hs_guard/engine/ring_attention_kernel.py:91-105) and the Lb > 1 ring scatter
 * (src/hs_guard/engine/slot_engine_v8.py:86-88).
 * Element addresses (row base B(x) = offsets ? offsets[n]*x_sl : n*x_sn):
 *   q[n,l,h,g,:]     = q     + B(q) + l*q_sl + h*q_sh + g*q_sg
 *   new_k[n,l,h,:]   = new_k + B(nk) + l*nk_sl + h*nk_sh         (same for new_v)
 *   gate[n,l,h,g,:]  = gate  + B(g) + l*g_sl + h*g_sh + g*g_sg + g_off   (gate may be NULL: no gating)
 *   out[n,l,h,g,:]   = out   + B(o) + l*o_sl + h*o_sh + g*o_sg
 *   ring_k/ring_v    [ring_rows, hkv, window+1, head_dim] bf16, ring_pos [ring_rows, window+1] int64.
 * Key j of the ring (column c < window, position ring_pos[slot,c]) or of the tick (position start+j when
 * j < len) is visible to query step l (position start+l, l < len) iff 0 <= kpos <= qpos and
 * kpos > qpos - window. Output = softmax-weighted values, rounded to bf16, times bf16(sigmoid(gate)).
 * write_ring != 0: after every read, new key/value of each valid step j go to ring column
 * (start+j) % window. ring_pos itself is not written (see hsg_ring_pos_update).
 * Packed layout only: rows with lens[n] < min_len are skipped (no output, no ring write), so that a tick's
 * single-step rows can go to hsg_ring_decode (min_len 2); min_len <= 1 processes every row.
 * Supported: head_dim == 256, window <= 512 and a multiple of 32, lb <= 64. Padded layout: steps past lb are
 * not computed (rows with lens[n] > 64 are treated as empty); packed layout: lb bounds every row's length and
 * rows with lens[n] > lb are treated as empty. write_ring needs lb <= window so that the steps of one tick own
 * distinct columns; with write_ring the call is two launches on `stream` (attention, then the ring write).
 */
int hsg_ring_attention(const void* q, int64_t q_sn, int64_t q_sl, int64_t q_sh, int64_t q_sg,
                       void* ring_k, void* ring_v, int64_t ring_rows, int32_t window, const void* new_k,
                       int64_t nk_sn, int64_t nk_sl, int64_t nk_sh, const void* new_v, int64_t nv_sn,
                       int64_t nv_sl, int64_t nv_sh, const void* gate, int64_t g_sn, int64_t g_sl,
                       int64_t g_sh, int64_t g_sg, int64_t g_off, const int64_t* ring_pos,
                       const int64_t* slots, const int64_t* starts, const int64_t* lens,
                       const int64_t* offsets, int32_t n_rows, int32_t lb, int32_t hkv, int32_t groups,
                       int32_t head_dim, float scale, int32_t write_ring, int32_t min_len, void* out,
                       int64_t o_sn, int64_t o_sl, int64_t o_sh, int64_t o_sg, void* stream);

/*
 * Ring attention for decode steps: the same contract and numerics as hsg_ring_attention for rows with
 * lens[n] == 1 (one query position; lb is 1 and the padded layout is [n_rows, 1, ...]). Replaces
 * ring_attention_v8 at its decode shape (src/hs_guard/engine/fused_kernels.py:358-376 with Lb == 1,
 * write_ring True, the reference's per-token streaming step). The running maximum of each 32-key block is
 * recovered as the prefix maximum of the block maxima, so the blocks are processed in parallel. groups <= 8:
 * one launch on `stream` (one workgroup per row and kv head, scores in LDS, the workspace untouched); groups
 * 9..16: three launches (scores and block maxima per quarter of the ring columns into the workspace; per-block
 * probabilities times values; combine, gate, ring write). With groups <= 8, calls of at most
 * HSG_RING_DECODE_SPLIT_UNITS rows x kv heads that pass a large enough workspace also take the three launches:
 * there a row's ring is read by 4 workgroups instead of 1 (one CU moves only a few tens of GB/s of it), e.g. a
 * lone row at W = 512 in 16 instead of 21.5 us. Packed layout: rows with lens[n] != 1 are not touched. Padded
 * layout: rows with lens[n] == 0 (or a slot outside [0, ring_rows)) get zero outputs.
 * workspace (required for groups > 8; up to 8 optional, may be NULL): device memory of at least
 * hsg_ring_decode_workspace_bytes(n_rows, hkv, groups, window) bytes, 16-byte aligned; its contents need no
 * initialisation and are garbage afterwards. Supported: head_dim == 256, window <= 512 and a multiple of 32,
 * groups <= 16.
 */
#define HSG_RING_DECODE_SPLIT_UNITS 64
size_t hsg_ring_decode_workspace_bytes(int32_t n_rows, int32_t hkv, int32_t groups, int32_t window);
int hsg_ring_decode(const void* q, int64_t q_sn, int64_t q_sl, int64_t q_sh, int64_t q_sg, void* ring_k,
                    void* ring_v, int64_t ring_rows, int32_t window, const void* new_k, int64_t nk_sn,
                    int64_t nk_sl, int64_t nk_sh, const void* new_v, int64_t nv_sn, int64_t nv_sl,
                    int64_t nv_sh, const void* gate, int64_t g_sn, int64_t g_sl, int64_t g_sh, int64_t g_sg,
                    int64_t g_off, const int64_t* ring_pos, const int64_t* slots, const int64_t* starts,
                    const int64_t* lens, const int64_t* offsets, int32_t n_rows, int32_t hkv, int32_t groups,
                    int32_t head_dim, float scale, int32_t write_ring, void* out, int64_t o_sn, int64_t o_sl,
                    int64_t o_sh, int64_t o_sg, void* workspace, size_t workspace_bytes, void* stream);

/*
 * hsg_ring_decode (three-launch split-K path, packed layout) with the attention front's per-head q / k norm and
 * partial RoPE applied on the fly: replaces square_rows + norm_rope + ring_attention_v8 at the decode shape
 * (src/hs_guard/engine/fused_kernels.py:237-284,358-376; slot_engine_v8.py:79-85) for a tick's single-step rows,
 * bitwise hsg_norm_rope followed by hsg_ring_decode's split-K path. q_raw / k_raw: the projection's raw query and
 * key rows (token t, query head j at q_raw + t q_row + j q_head; kv head h at k_raw + t k_row + h k_head), q_w1 /
 * k_w1 [head_dim] fp32 (1 + weight), pos [tokens] int64, inv_freq [rot / 2] fp32; the normalised, rotated new keys
 * are written to k_out (token t, kv head h at k_out + t ko_row + h head_dim) and into the ring. new_v, gate, out
 * and their strides as hsg_ring_decode's packed-layout arguments (row = token). One launch fewer than the separate
 * kernels, for ticks of one token (the single-session step). Supported: head_dim 256, rot 64, groups <= 16, the
 * workspace of hsg_ring_decode_workspace_bytes (required).
 */
int hsg_ring_decode_rope(const void* q_raw, int64_t q_row, int64_t q_head, const float* q_w1, float q_eps,
                         const void* k_raw, int64_t k_row, int64_t k_head, const float* k_w1, float k_eps,
                         const int64_t* pos, const float* inv_freq, int32_t rot, void* k_out, int64_t ko_row,
                         void* ring_k, void* ring_v, int64_t ring_rows, int32_t window, const void* new_v,
                         int64_t nv_row, int64_t nv_head, const void* gate, int64_t g_row, int64_t g_head,
                         int64_t g_group, int64_t g_off, const int64_t* ring_pos, const int64_t* slots,
                         const int64_t* starts, const int64_t* lens, const int64_t* offsets, int32_t n_rows,
                         int32_t hkv, int32_t groups, int32_t head_dim, float scale, int32_t write_ring, void* out,
                         int64_t o_row, int64_t o_head, int64_t o_group, void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * hsg_ring_decode without the workspace argument: it allocates nothing. No counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under hipGraph capture, allocation-free serving loops,
 * harnesses that forbid hipMalloc). The workspace (used by the split-K path, groups > 8) is the library's own
 * static device array of HSG_RING_DECODE_SCRATCH_BYTES, one copy per GPU, held until the process ends; its
 * device address is looked up on the first call made on each device (make that first call outside graph
 * capture). Arguments, outputs and
 * numerics are those of hsg_ring_decode, bit for bit (with the scratch as its workspace). Up to 8 query heads per kv
 * head the call runs the fused kernel, which uses no workspace, and takes any number of rows (the three-launch path of
 * at most HSG_RING_DECODE_SPLIT_UNITS rows x kv heads fits the scratch); above that it returns HSG_ERR_SHAPE when
 * hsg_ring_decode_workspace_bytes(n_rows, hkv, groups, window) exceeds the scratch (48 MiB: 122 rows at 4 kv heads,
 * G = 16, W = 512). All calls on one GPU share its scratch, so calls that overlap on one GPU (two streams, or two
 * threads) race and must be serialised by the caller; nothing left by an earlier call is read.
 */
#define HSG_RING_DECODE_SCRATCH_BYTES (48u << 20)
int hsg_ring_decode_noalloc(const void* q, int64_t q_sn, int64_t q_sl, int64_t q_sh, int64_t q_sg, void* ring_k,
                            void* ring_v, int64_t ring_rows, int32_t window, const void* new_k, int64_t nk_sn,
                            int64_t nk_sl, int64_t nk_sh, const void* new_v, int64_t nv_sn, int64_t nv_sl,
                            int64_t nv_sh, const void* gate, int64_t g_sn, int64_t g_sl, int64_t g_sh, int64_t g_sg,
                            int64_t g_off, const int64_t* ring_pos, const int64_t* slots, const int64_t* starts,
                            const int64_t* lens, const int64_t* offsets, int32_t n_rows, int32_t hkv, int32_t groups,
                            int32_t head_dim, float scale, int32_t write_ring, void* out, int64_t o_sn, int64_t o_sl,
                            int64_t o_sh, int64_t o_sg, void* stream);

/*
 * Embedding gather + RMSNorm of the first layer. Replaces embed_tokens + add_square(hidden) + rms_finish
 * (src/hs_guard/engine/slot_engine_v8.py:38,42-43; fused_kernels.py:30-72):
 *   hidden[t] = emb[ids[t]];  normed[t] = bf16((hidden * rsqrt(mean(hidden^2) + eps)) * w1)
 *   emb [vocab, width] bf16, w1 [width] fp32 (= 1 + weight), hidden/normed [tokens, width] bf16.
 * Supported: width == 1024; emb, hidden, normed and w1 16-byte aligned. Ids outside [0, vocab) read row 0 (the
 * host rejects them first).
 */
int hsg_embed_rmsnorm(const int64_t* ids, const void* emb, int64_t vocab, const float* w1, float eps,
                      void* hidden, void* normed, int32_t tokens, int32_t width, void* stream);

/*
 * Residual add + RMSNorm. Replaces add_square + sq.mean + rms_finish
 * (src/hs_guard/engine/fused_kernels.py:30-72; slot_engine_v8.py:49-55):
 *   hidden = bf16(hidden + mix) (in place; mix may be NULL: no add);
 *   normed = bf16((hidden * rsqrt(mean(hidden^2) + eps)) * w1). Supported: width == 1024; hidden, mix, normed
 *   and w1 16-byte aligned.
 */
int hsg_add_rmsnorm(void* hidden, const void* mix, const float* w1, float eps, void* normed, int32_t tokens,
                    int32_t width, void* stream);

/*
 * Gated RMSNorm of GDN outputs, per (token, head) of `width` values. Replaces gated_finish
 * (src/hs_guard/engine/fused_kernels.py:215-233) where it is not fused into the slot step (outputs of
 * hsg_gdn_chunk_prefill):
 *   out[t, h*width + c] = bf16( bf16(w[c] * bf16(x * rsqrt(mean_c(x^2) + eps))) * silu(z[t, h*width + c]) )
 *   x [tokens, x_stride], z [tokens, z_stride], out [tokens, out_stride] bf16; w [width] bf16.
 * Supported: width == 128; strides even, pointers 4-byte aligned.
 */
int hsg_gated_rmsnorm(const void* x, int64_t x_stride, const void* z, int64_t z_stride, const void* w, float eps,
                      void* out, int64_t out_stride, int32_t tokens, int32_t heads, int32_t width, void* stream);

/*
 * Causal depthwise conv + SiLU with the per-slot conv-history update. Replaces conv_silu_update
 * (src/hs_guard/engine/fused_kernels.py:126-136; kernel :94-123):
 *   qkv [tokens, qkv_stride] bf16 (first `channels` columns), pool [pool_rows, kernel_size-1, channels]
 *   bf16 (updated in place at slots[n] when lens[n] > 0), weight [channels, kernel_size] bf16,
 *   out [tokens, out_stride] bf16. Padded layout computes all L positions of every row like the reference.
 * Supported: kernel_size == 4.
 */
int hsg_conv_silu_update(const void* qkv, int64_t qkv_stride, void* pool, int64_t pool_rows, const void* weight,
                         int32_t kernel_size, const int64_t* slots, const int64_t* lens, const int64_t* offsets,
                         int32_t n_rows, int32_t L, int32_t channels, void* out, int64_t out_stride,
                         void* stream);

/*
 * Per-head RMSNorm(1+w) + partial rotate-half RoPE of q and k in one launch. Replaces square_rows +
 * mean + norm_rope x2 (src/hs_guard/engine/fused_kernels.py:237-284; slot_engine_v8.py:79-82) and the
 * rotary cos/sin of the backbone (slot_engine_v8.py:39): cos/sin = bf16(cos/sin(pos[t] * inv_freq[i])).
 *   x[t, h, :] at src + t*row + h*head;  out[t, h, :] at out + t*out_row + h*out_head (bf16).
 *   w1 [head_dim] fp32 per tensor (16-byte aligned); inv_freq [rot/2] fp32; pos [tokens] int64.
 * Supported: head_dim == 256, rot a power of two in [8, 256], q_heads + k_heads <= 32.
 */
int hsg_norm_rope(const void* q_src, int64_t q_row, int64_t q_head, int32_t q_heads, const float* q_w1,
                  float q_eps, void* q_out, int64_t q_out_row, int64_t q_out_head, const void* k_src,
                  int64_t k_row, int64_t k_head, int32_t k_heads, const float* k_w1, float k_eps, void* k_out,
                  int64_t k_out_row, int64_t k_out_head, const int64_t* pos, const float* inv_freq, int32_t rot,
                  int32_t tokens, int32_t head_dim, void* stream);

/*
 * Unfused entry points with the reference engine's own kernel contracts (the variance of each RMSNorm and the
 * rotary cos/sin are inputs, as src/hs_guard/engine/slot_engine_v8.py:42-55,74-82 computes them), so that a caller
 * composing the step as SlotStreamEngineV8 does can swap its imports (slot_engine_v8.py:6-7). Rows may have any
 * width; contiguous row-major tensors, bf16 unless stated. The streaming engine of this library runs the fused
 * forms above (hsg_add_rmsnorm, hsg_norm_rope, hsg_silu_mul, the slot step's gated epilogue) instead.
 */

/*
 * Replaces add_square (src/hs_guard/engine/fused_kernels.py:44-52; kernel :30-41), over rows x width elements:
 *   mixed non-NULL: out = bf16(residual + mixed) (one fp32 add), sq = out^2 (fp32);
 *   mixed NULL:     sq = residual^2 (out is not written).
 */
int hsg_add_square(const void* residual, const void* mixed, void* out, float* sq, int64_t rows, int32_t width,
                   void* stream);

/*
 * Replaces rms_finish (src/hs_guard/engine/fused_kernels.py:67-72; kernel :56-64):
 *   out[r, c] = bf16((x[r, c] * rsqrt(var[r] + eps)) * w1[c]);  var [rows] fp32 (the mean of x^2 over the row),
 *   w1 [width] fp32 (= 1 + weight).
 */
int hsg_rms_finish(const void* x, const float* var, const float* w1, float eps, void* out, int64_t rows,
                   int32_t width, void* stream);

/*
 * Replaces silu_mul (src/hs_guard/engine/fused_kernels.py:86-90; kernel :76-83) on two separate tensors of n
 * elements: out = bf16(bf16(silu(gate)) * up).
 */
int hsg_silu_mul_pair(const void* gate, const void* up, void* out, int64_t n, void* stream);

/*
 * Replaces gated_finish (src/hs_guard/engine/fused_kernels.py:228-233; kernel :215-225):
 *   out[r, c] = bf16(bf16(weight[c] * bf16(x[r, c] * rsqrt(var[r] + eps))) * silu(z[r, c]));
 *   var [rows] fp32, weight [width] bf16.
 */
int hsg_gated_finish(const void* x, const float* var, const void* weight, const void* z, float eps, void* out,
                     int64_t rows, int32_t width, void* stream);

/*
 * Replaces square_rows (src/hs_guard/engine/fused_kernels.py:245-249; kernel :237-242):
 *   sq[t*heads + h, c] = src[t*row_stride + h*head_stride + c]^2 (fp32), sq [tokens*heads, dim].
 */
int hsg_square_rows(const void* src, float* sq, int64_t tokens, int32_t heads, int64_t row_stride,
                    int64_t head_stride, int32_t dim, void* stream);

/*
 * Replaces norm_rope (src/hs_guard/engine/fused_kernels.py:277-284; kernel :252-274): per-head RMSNorm(1 + w) given
 * var, then rotate-half RoPE on the first `rot` dims with the given cos/sin [n_rows*lb, rot] bf16:
 *   x = bf16((src * rsqrt(var + eps)) * w1), out = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin)) (d < rot),
 *   bf16(x) beyond. Head j of token t = n*lb + l is read at src + t*row_stride + j*head_stride, its variance at
 *   var[t*heads + j], and written at out + n*out_n + (j / groups)*out_h + ((j % groups)*lb + l)*out_row: the
 *   grouped [N, heads/groups, groups*lb, dim] query layout of hsg_ring_attention (groups 1: [N, heads, lb, dim]).
 *   w1 [dim] fp32. Supported: heads % groups == 0, rot even and <= dim.
 */
int hsg_norm_rope_grouped(const void* src, const float* var, const float* w1, const void* cos, const void* sin,
                          int32_t rot, float eps, int32_t n_rows, int32_t lb, int32_t heads, int32_t groups,
                          int64_t row_stride, int64_t head_stride, int32_t dim, void* out, int64_t out_n,
                          int64_t out_h, int64_t out_row, void* stream);

/*
 * SiLU-mul of the fused gate|up projection. Replaces silu_mul (src/hs_guard/engine/fused_kernels.py:86-90):
 *   out[t, c] = bf16(bf16(silu(gu[t, c])) * gu[t, width + c]), out [tokens, width] bf16.
 * Supported: width and row_stride multiples of 8, pointers 16-byte aligned.
 */
int hsg_silu_mul(const void* gate_up, int64_t row_stride, int32_t width, void* out, int32_t tokens,
                 void* stream);

/*
 * Risk heads after the fused first projection, as the streaming engine reads them out under autocast. Replaces
 * _risk + softmax (src/hs_guard/engine/slot_engine_v7.py:44-61; slot_engine_v8.py:56; src/hs_guard/runtime.py:61-74):
 *   for role r: v = y[t, r*width : (r+1)*width] (bf16 Linear output incl. bias), LayerNorm(eps) in fp32
 *   with fp32 ln_w/ln_b [roles, width], SiLU, bf16, Linear to 3 with bf16 w2 [roles, 3, width], b2 [roles, 3],
 *   bf16 logits, softmax -> probs [roles, tokens, 3] fp32. Supported: width == 512.
 */
int hsg_risk_head(const void* y, int64_t y_stride, const float* ln_w, const float* ln_b, const void* w2,
                  const void* b2, float eps, int32_t roles, int32_t width, float* probs, int32_t tokens,
                  void* stream);

/*
 * The same heads read out entirely in fp32, as the complete-message scorer does: Classifier.readout on
 * hidden.float() outside autocast, then softmax (src/hs_guard/runtime.py:70-73,141). y [tokens, y_stride] is the
 * fp32 output of the first Linear (fp32 weights, incl. bias); ln_w, ln_b [roles, width], w2 [roles, 3, width],
 * b2 [roles, 3] fp32; nothing is rounded to bf16. Supported: width == 512.
 */
int hsg_risk_head_f32(const float* y, int64_t y_stride, const float* ln_w, const float* ln_b, const float* w2,
                      const float* b2, float eps, int32_t roles, int32_t width, float* probs, int32_t tokens,
                      void* stream);

/*
 * Ring position bookkeeping after all layers. Replaces ring_pos[slots, ring_col] = where(valid, pos, -1)
 * (src/hs_guard/engine/slot_engine_v8.py:41,57): ring_pos[slot, (start + j) % window] = start + j for
 * j < min(lens[n], lb_max); column `window` is never written (it stays -1).
 */
int hsg_ring_pos_update(int64_t* ring_pos, int64_t ring_rows, int32_t window, const int64_t* slots,
                        const int64_t* starts, const int64_t* lens, int32_t n_rows, int32_t lb_max,
                        void* stream);

/*
 * Projection GEMM on hipBLASLt with a fixed solution: D[M, N] = A[M, K] . W[N, K]^T, bf16 row-major with row
 * strides lda, ldw, ldd (elements), fp32 accumulation. Replaces the backbone's nn.Linear products
 * (src/hs_guard/engine/slot_engine_v8.py:52-53,63-65,72,78,89). algo_index: a hipBLASLt solution index (from a
 * committed plan table, so every process runs the same accumulation order), or -1 for the first of hipBLASLt's
 * heuristic candidates (16 examined, in its order) whose workspace fits workspace_bytes (torch.mm's choice when
 * that is the first). workspace: device memory for solutions that need it. Returns
 * HSG_ERR_SHAPE when the solution does not exist in this hipBLASLt, does not support the problem or needs more
 * than workspace_bytes, HSG_ERR_BLAS when hipBLASLt fails. The first call on a device creates its hipBLASLt
 * handle (make it outside graph capture); later calls are capturable.
 */
int hsg_gemm_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, void* D, int64_t ldd, int32_t M,
                  int32_t N, int32_t K, int32_t algo_index, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Up to max_count hipBLASLt heuristic candidates for the dense problem (M, N, K) of hsg_gemm_bf16, in hipBLASLt's
 * order, as solution indices (and each one's workspace bytes, when `workspace` is non-NULL), those needing more
 * than workspace_limit bytes of workspace left out. Returns the count, or -1. For generating a plan table.
 */
int hsg_gemm_candidates(int32_t M, int32_t N, int32_t K, int32_t* indices, size_t* workspace, int32_t max_count,
                        size_t workspace_limit);

/* Rows of A that hsg_gemm_bf16_skinny accepts. */
#define HSG_GEMM_SKINNY_M_MAX 8

/*
 * Skinny projection product for decode ticks, bandwidth-bound on W: D[M, N] = A[M, K] . W[N, K]^T for
 * M <= HSG_GEMM_SKINNY_M_MAX, bf16 row-major (row strides lda, ldw, ldd in elements), fp32 accumulation, one
 * rounding to bf16. Replaces the same nn.Linear products as hsg_gemm_bf16
 * (src/hs_guard/engine/slot_engine_v8.py:52-53,63-65,72,78,89) when a tick has at most 8 tokens. Each output is a
 * fixed reduction over k (per lane in k order, then a fixed tree over 64 lanes): the result depends on the inputs
 * and K only, not on M, N or timing. Requires K, lda and ldw multiples of 8 and A, W 16-byte aligned
 * (HSG_ERR_ALIGN), M <= HSG_GEMM_SKINNY_M_MAX (HSG_ERR_SHAPE). D must not overlap an operand (every workgroup reads
 * all of A while others store their columns of D). Allocates nothing; capturable.
 */
int hsg_gemm_bf16_skinny(const void* A, int64_t lda, const void* W, int64_t ldw, void* D, int64_t ldd, int32_t M,
                         int32_t N, int32_t K, void* stream);

/*
 * The MLP's down projection of a tick of at most HSG_GEMM_SKINNY_M_MAX tokens with the SiLU gate applied on the fly:
 * D[M, N] = act . W[N, K]^T with act[m, k] = bf16(bf16(silu(gate_up[m, k])) * gate_up[m, K + k]), i.e.
 * hsg_silu_mul (width K) followed by hsg_gemm_bf16_skinny, bitwise, in one launch and without act in memory.
 * Replaces silu_mul + down_proj (src/hs_guard/engine/slot_engine_v8.py:52-53; fused_kernels.py:86). ld_gu (>= 2 K) is
 * gate_up's row stride; requirements and errors as hsg_gemm_bf16_skinny.
 */
int hsg_gemm_bf16_skinny_silu(const void* gate_up, int64_t ld_gu, const void* W, int64_t ldw, void* D, int64_t ldd,
                              int32_t M, int32_t N, int32_t K, void* stream);

/*
 * The residual add + RMSNorm of a tick of at most HSG_GEMM_SKINNY_M_MAX tokens inside the product that reads it:
 * hidden_out = bf16(hidden + mix), D[M, N] = norm . W[N, K]^T with norm = bf16((hidden_out * rsqrt(mean(hidden_out^2)
 * + eps)) * w1), i.e. hsg_add_rmsnorm (w1 fp32 [K]) followed by hsg_gemm_bf16_skinny, bitwise, in one launch.
 * Replaces add_square + rms_finish + the Linear that reads the norm (src/hs_guard/engine/slot_engine_v8.py:49-52,
 * 53-55; fused_kernels.py:44,67). Supported: K == 1024 (HSG_ERR_SHAPE). hidden_out must not overlap
 * hidden or mix (every workgroup reads them; workgroup 0 writes hidden_out). Other requirements and errors as
 * hsg_gemm_bf16_skinny, with mix, w1 and hidden_out 16-byte aligned and ldm, ldo multiples of 8. bias ([N] bf16, or
 * NULL): added to the fp32 sum before its bf16 rounding, for a Linear with bias (the risk heads' first projection,
 * src/hs_guard/engine/slot_engine_v7.py:58-61, after the final norm).
 */
int hsg_gemm_bf16_skinny_addnorm(const void* hidden, int64_t ldh, const void* mix, int64_t ldm, const float* w1,
                                 float eps, void* hidden_out, int64_t ldo, const void* W, int64_t ldw, void* D,
                                 int64_t ldd, int32_t M, int32_t N, int32_t K, const void* bias, void* stream);

/* hipBLASLt's version on the current device (solution indices are valid only for the version they came from). */
int hsg_gemm_blas_version(void);

#ifdef __cplusplus
}
#endif

#endif /* HSG_H_ */
