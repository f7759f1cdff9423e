/* C ABI of the MI355X (gfx950) column sequence mixers: the delta-rule scan and sliding-window
 * causal attention of Vesper's column, as hand-written HIP kernels.
 *
 * Conventions shared by every entry point:
 *  - Pointers are device pointers to contiguous row-major tensors; sizes are element counts.
 *  - `stream` is a hipStream_t (NULL = the null stream). Work is enqueued only: no host
 *    synchronisation, no device-to-host reads and no device allocation happen inside, so every
 *    call can be captured into a HIP graph. Scratch memory, where a kernel needs it, is passed in.
 *  - Inputs are never written; outputs may alias their matching input only where stated.
 *  - `active` (optional, may be NULL) is a uint8 mask [B, T] (1 = active token). Inactive tokens
 *    still write the recurrent state and stay visible as keys; their outputs are written as 0.
 *  - Return 0 on success, otherwise a nonzero status with a message in vsp_last_error().
 *  - Results are bitwise repeatable: no atomics take part in any reduction.
 */
#ifndef VESPER_KERNELS_H
#define VESPER_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VSP_ABI_VERSION 20

/* Status codes. */
#define VSP_OK 0
#define VSP_ERR_ARG 1         /* a size, pointer or combination the kernels do not take */
#define VSP_ERR_UNSUPPORTED 2 /* a valid request this build has no kernel for */
#define VSP_ERR_LAUNCH 3      /* the HIP runtime refused the launch */

/* The message of the last failed call on this thread ("" after a success). */
const char* vsp_last_error(void);

/* VSP_ABI_VERSION of the loaded library. */
int vsp_abi_version(void);

/* Set-up, once per process before the first kernel call (later calls return at once): allocates
 * the fault record below in pinned host memory, and on the current device only takes the address
 * of the static scratch of vsp_ring_attn_noalloc_bf16 and zeroes it (another device is set up by
 * that entry's first call on it; no other device is touched). No counterpart in the reference,
 * whose kernels come from a library that needs none. */
int vsp_init(void);

/* The fault record of the bounded waits. Kernels whose waves hand work to each other through LDS
 * flags (the bf16 scan's chain) poll those flags a bounded number of times; a wait that gives up
 * sets its kernel family's bit here and the kernel writes NaN in place of its later outputs, so a
 * broken hand-over neither hangs the device nor passes as a result. vsp_fault_bits reads the
 * record without any device synchronisation (it shows the faults of kernels that have completed);
 * bit 0: the scan chain. The bits stay set until vsp_clear_faults. No counterpart in the
 * reference: its library's kernels have no inter-wave hand-over. */
unsigned vsp_fault_bits(void);
void vsp_clear_faults(void);

/* Polls a bounded wait makes before it gives up (default 2^19, seconds of waiting; a negative
 * value restores the default); returns the previous limit. Taken at each launch. For tests of the
 * fault path: a limit of 0 makes a wait whose flag is not yet set give up at once, while every
 * kernel still runs to its end. */
int vsp_set_wait_limit(int polls);

/* Which form of the bf16 scan runs at head width 64 (with or without carried inputs): 0 the
 * value-slice chains, one workgroup per 16 value columns of a head over the whole sequence; 1 the
 * segmented scan, whose workgroups each carry one head's whole state through one segment of the
 * sequence, the segments joined by their affine maps H -> X + M H; 2 (the default, and any other
 * value) by shape: the chains while B * H * 4 workgroups fit one a CU (256), the segments beyond.
 * Both compute the same scan to the bf16 tolerance; returns the previous setting. Taken at each
 * call. No counterpart in the reference (its library has one kernel); for tests and measurements
 * of both forms. */
int vsp_set_scan_segments(int form);

/* ---- delta-rule scan ------------------------------------------------------------------------
 * Per batch row b and head h, with the state H [D, D] read as H^T q, each token applies
 *     H <- (I - beta k k^T) H + beta k v^T,    o = H^T q
 * q, k, v: [B, T, H, D]; beta: [B, T, H]; state_in, state_out: [B, H, D, D] float32 (may alias).
 * No query scaling, no in-kernel key normalisation (keys arrive with L2 norm at most one).
 * Replaces the fla-core 0.5.2 calls behind vesper/kernels/delta_scan.py:122-129 (`_run`):
 * `chunk_delta_rule` for the bf16 entry (delta_scan.py:132-153) and
 * `fused_recurrent_delta_rule` for the fp32 entry (delta_scan.py:156-187).
 * D <= 256. D in {16, 32, 64, 128} (bf16) or {16, 32, 64} (fp32) runs the chunked WY/UT MFMA path
 * (64-token chunks); other widths, and T below 16, run the token-serial kernel.
 * `workspace` holds the per-chunk UT matrices of the chunked path; it needs
 * vsp_delta_scan_workspace_bytes(...) bytes (0 when the serial path runs; then it may be NULL). */
size_t vsp_delta_scan_workspace_bytes(int B, int T, int H, int D, int fp32_inputs);

/* bf16 q, k, v, beta; float32 state; bf16 o. */
int vsp_delta_scan_bf16(const void* q, const void* k, const void* v, const void* beta, const float* state_in,
                        void* o, float* state_out, void* workspace, size_t workspace_bytes,
                        const uint8_t* active, int B, int T, int H, int D, void* stream);

/* vsp_delta_scan_bf16 that also records, for the backward, the state at each 64-token chunk's
 * start: `records` receives vsp_delta_scan_records_bytes(B, T, H, D) bytes (16-byte aligned), one
 * [D x D] bf16 block a (b, h, chunk), in the order vsp_delta_scan_backward_recorded_bf16 reads.
 * Records exist for D in {32, 64} on the chunked path (T >= 16); the size is 0 otherwise and the
 * call is refused (VSP_ERR_UNSUPPORTED). The state the forward carries in fp32 is recorded rounded
 * to bf16, the precision the backward multiplies it at. No counterpart in the reference: the
 * autograd path of vesper/kernels/delta_scan.py:132-153 keeps what its backward needs itself. */
size_t vsp_delta_scan_records_bytes(int B, int T, int H, int D);
int vsp_delta_scan_record_bf16(const void* q, const void* k, const void* v, const void* beta, const float* state_in,
                               void* o, float* state_out, void* workspace, size_t workspace_bytes,
                               const uint8_t* active, void* records, size_t records_bytes, int B, int T, int H,
                               int D, void* stream);

/* float32 q, k, v, beta, state and o. */
int vsp_delta_scan_f32(const float* q, const float* k, const float* v, const float* beta, const float* state_in,
                       float* o, float* state_out, void* workspace, size_t workspace_bytes,
                       const uint8_t* active, int B, int T, int H, int D, void* stream);

/* Copy-forward fused into the scan's loads (the carry merges of vesper/column.py:779-789 and
 * vesper/loop.py:449-452, which select `where(active, fresh, carried)` for k, v and beta before
 * the scan): as vsp_delta_scan_bf16 / _f32, but where active[b, t] is 0 the token's k, v and beta
 * rows are read from k_carried, v_carried, beta_carried (same shapes and dtypes as k, v, beta)
 * instead of k, v, beta. `active` is required; the fresh rows of inactive tokens are never read. */
int vsp_delta_scan_carried_bf16(const void* q, const void* k, const void* v, const void* beta,
                                const void* k_carried, const void* v_carried, const void* beta_carried,
                                const float* state_in, void* o, float* state_out, void* workspace,
                                size_t workspace_bytes, const uint8_t* active, int B, int T, int H, int D,
                                void* stream);
int vsp_delta_scan_carried_f32(const float* q, const float* k, const float* v, const float* beta,
                               const float* k_carried, const float* v_carried, const float* beta_carried,
                               const float* state_in, float* o, float* state_out, void* workspace,
                               size_t workspace_bytes, const uint8_t* active, int B, int T, int H, int D,
                               void* stream);

/* The scan with beta given as write-strength logits: the reference's `write_strength`
 * (vesper/recurrence.py:34-88) applied in the scan's own beta loads, so beta is never written to
 * memory: beta = sigmoid(logit + ln(1 + alpha m[b, t])), exactly 0 where 1 + alpha m is 0;
 * m: [B, T] float32 or NULL (no modulator: beta = sigmoid(logit)); alpha finite and >= 0; the
 * caller holds 1 + alpha m >= 0 (the reference refuses a negative factor). beta is computed in
 * float32 and rounded to the inputs' dtype, as the reference column casts it before its scan
 * (vesper/column.py:313). Otherwise as vsp_delta_scan_bf16 / _f32, logits in beta's place and
 * dtype. */
int vsp_delta_scan_logits_bf16(const void* q, const void* k, const void* v, const void* logits, const float* m,
                               float alpha, const float* state_in, void* o, float* state_out, void* workspace,
                               size_t workspace_bytes, const uint8_t* active, int B, int T, int H, int D,
                               void* stream);
int vsp_delta_scan_logits_f32(const float* q, const float* k, const float* v, const float* logits, const float* m,
                              float alpha, const float* state_in, float* o, float* state_out, void* workspace,
                              size_t workspace_bytes, const uint8_t* active, int B, int T, int H, int D,
                              void* stream);

/* The write strength alone (vesper/recurrence.py:34-88): beta [rows, H] from logits [rows, H]
 * (same dtype) and the per-row modulator m [rows] float32 (or NULL), as above. */
int vsp_write_strength_bf16(const void* logits, const float* m, float alpha, void* beta, int rows, int H,
                            void* stream);
int vsp_write_strength_f32(const float* logits, const float* m, float alpha, float* beta, int rows, int H,
                           void* stream);

/* One decoding token per row (the contract of vesper/recurrence.py:143-163, delta_scan_step):
 * q, k, v: [B, H, D]; beta: [B, H]; state_in, state_out: [B, H, D, D] float32 (may alias, for an
 * in-place decode); o: [B, H, D]; active: [B] or NULL. */
int vsp_delta_step_f32(const float* q, const float* k, const float* v, const float* beta, const float* state_in,
                       float* state_out, float* o, const uint8_t* active, int B, int H, int D, void* stream);
int vsp_delta_step_bf16(const void* q, const void* k, const void* v, const void* beta, const float* state_in,
                        float* state_out, void* o, const uint8_t* active, int B, int H, int D, void* stream);

/* The decode step's key filter folded into the bf16 step (the looped column's per-pass decode:
 * vesper/column.py:255-289 for the key, vesper/recurrence.py:118-163 for the step): the key of each
 * (b, h) is formed from the key inputs z [B, H*D] bf16 with the K filter taps (taps [K, H*D]
 * float32, tap 0 on the token) over the history (history [B, K-1, H*D] float32, oldest first;
 * NULL when K = 1) and normalized per head, exactly as vsp_key_step_bf16 forms and rounds it, and
 * the next history is written over the history; then the step as vsp_delta_step_bf16 with that
 * key. Bitwise the two launches' results. D in {16, 32, 64, 128}, K in 1..8; z, taps, history and
 * the states 16-byte aligned; state_out may be state_in. */
int vsp_delta_step_keys_bf16(const void* q, const void* z, const void* v, const void* beta, float* history,
                             const float* taps, int K, const float* state_in, float* state_out, void* o,
                             const uint8_t* active, int B, int H, int D, void* stream);

/* The scan's backward (the gradients fla-core's chunk kernels give vesper/kernels/delta_scan.py:132-187
 * under autograd): from d_o [B, N, H, D] (the inputs' dtype) and d_state [B, H, D, D] fp32 (the
 * final state's gradient; NULL for zero), dq, dk, dv [B, N, H, D], dbeta [B, N, H] (the inputs'
 * dtype) and d_state_in [B, H, D, D] fp32 (the initial state's). active as the forward (an inactive
 * token's output gradient is ignored). D: any multiple of 16 up to 256. {16, 32, 64, 128} (bf16)
 * and {16, 32, 64} (fp32) run the tiled chunk kernels; other widths run the wide backward (the
 * forward recomputed token by token to checkpoint each chunk's starting state, then per-chunk and
 * per-value-group kernels whose partial sums are added in a fixed order). fp32 accumulation (the
 * bf16 entry multiplies on bf16 MFMA); deterministic.
 * workspace: vsp_delta_scan_backward_workspace_bytes bytes (the larger of both at D = 128), 16-byte
 * aligned. N == 0 writes nothing. */
size_t vsp_delta_scan_backward_workspace_bytes(int B, int N, int H, int D);
int vsp_delta_scan_backward_bf16(const void* q, const void* k, const void* v, const void* beta, const float* state_in,
                                 const void* d_o, const float* d_state, const uint8_t* active, void* dq, void* dk,
                                 void* dv, void* dbeta, float* d_state_in, void* workspace, size_t workspace_bytes,
                                 int B, int N, int H, int D, void* stream);
int vsp_delta_scan_backward_f32(const float* q, const float* k, const float* v, const float* beta,
                                const float* state_in, const float* d_o, const float* d_state, const uint8_t* active,
                                float* dq, float* dk, float* dv, float* dbeta, float* d_state_in, void* workspace,
                                size_t workspace_bytes, int B, int N, int H, int D, void* stream);
/* vsp_delta_scan_backward_bf16 given the forward's records (vsp_delta_scan_record_bf16 on the same
 * inputs): the states at the chunks' starts are read from them instead of being recomputed, so only
 * the state's gradient runs as a chain. D in {32, 64}; records_bytes as vsp_delta_scan_records_bytes. */
int vsp_delta_scan_backward_recorded_bf16(const void* q, const void* k, const void* v, const void* beta,
                                          const float* state_in, const void* d_o, const float* d_state,
                                          const uint8_t* active, const void* records, size_t records_bytes, void* dq,
                                          void* dk, void* dv, void* dbeta, float* d_state_in, void* workspace,
                                          size_t workspace_bytes, int B, int N, int H, int D, void* stream);

/* ---- sliding-window causal attention (prefill) -----------------------------------------------
 * q: [B, N, H, D]; keys, values: [B, M + N, HKV, D], the cache's M rows first; o: [B, N, H, D].
 * Query i sits at key index M + i and attends key indices [M + i - window + 1, M + i]; softmax in
 * fp32 with `scale` (1/sqrt(D) for the reference); query head h reads KV head h / (H / HKV).
 * D in {16, 32, 64, 128, 256}; H a multiple of HKV; active: [B, N] or NULL.
 * Replaces the fla-core 0.5.2 `parallel_attn` call of vesper/kernels/window_attn.py:27-39
 * (`window_attention`), without the zero query rows the reference pads the cache with. */
int vsp_window_attn_bf16(const void* q, const void* keys, const void* values, void* o, const uint8_t* active,
                         int B, int N, int M, int H, int HKV, int D, int window, float scale, void* stream);
int vsp_window_attn_f16(const void* q, const void* keys, const void* values, void* o, const uint8_t* active,
                        int B, int N, int M, int H, int HKV, int D, int window, float scale, void* stream);
/* The same forward, also writing lse [B, H, N] fp32: per query the log-sum-exp of its scaled scores
 * in log2 units (P = exp2(score * scale * log2(e) - lse)), +inf for an inactive query. */
int vsp_window_attn_lse_bf16(const void* q, const void* keys, const void* values, void* o, float* lse,
                             const uint8_t* active, int B, int N, int M, int H, int HKV, int D, int window,
                             float scale, void* stream);
int vsp_window_attn_lse_f16(const void* q, const void* keys, const void* values, void* o, float* lse,
                            const uint8_t* active, int B, int N, int M, int H, int HKV, int D, int window,
                            float scale, void* stream);
/* Copy-forward fused into the tile loads (the carry merges of the attention keys and values,
 * vesper/column.py:795-796, `where(active, fresh, carried)` before the call): as
 * vsp_window_attn_bf16 / _f16, but key rows M + t of a token t with active[b, t] == 0 are read from
 * row t of keys_carried / values_carried ([B, N, HKV, D]: the new rows only; cache rows are never
 * carried). `active` is required; the fresh key and value rows of inactive tokens are never read. */
int vsp_window_attn_carried_bf16(const void* q, const void* keys, const void* values, const void* keys_carried,
                                 const void* values_carried, void* o, const uint8_t* active, int B, int N, int M,
                                 int H, int HKV, int D, int window, float scale, void* stream);
int vsp_window_attn_carried_f16(const void* q, const void* keys, const void* values, const void* keys_carried,
                                const void* values_carried, void* o, const uint8_t* active, int B, int N, int M,
                                int H, int HKV, int D, int window, float scale, void* stream);
/* vsp_window_attn_* over a cache and a chunk held apart: key rows below M come from cache_keys /
 * cache_values [B, M, HKV, D] and key row M + t from keys / values [B, N, HKV, D] (the chunk's own),
 * so the kernel branch of WindowedAttention.attend (vesper/attention.py:373-383, which concatenates
 * the cache's and the chunk's keys before the fla-core call) needs no copy of either. Outputs equal
 * vsp_window_attn_* over the concatenated keys bit for bit. With M = 0 the cache pointers may be NULL. */
int vsp_window_attn_cached_bf16(const void* q, const void* cache_keys, const void* cache_values, const void* keys,
                                const void* values, void* o, const uint8_t* active, int B, int N, int M, int H,
                                int HKV, int D, int window, float scale, void* stream);
int vsp_window_attn_cached_f16(const void* q, const void* cache_keys, const void* cache_values, const void* keys,
                               const void* values, void* o, const uint8_t* active, int B, int N, int M, int H,
                               int HKV, int D, int window, float scale, void* stream);
/* The gradients (the backward of fla-core's `parallel_attn`, which autograd runs for
 * vesper/kernels/window_attn.py:27-39 under WindowedAttention.attend, vesper/attention.py:373-383):
 * from dO [B, N, H, D] and the forward's o and lse, dq [B, N, H, D], dk and dv [B, M + N, HKV, D]
 * (summed over the query heads of each KV head); workspace: B * H * N floats. Deterministic (no
 * atomics); an inactive query (lse +inf) contributes nothing and gets a zero dq. */
int vsp_window_attn_backward_bf16(const void* q, const void* keys, const void* values, const void* o,
                                  const void* dout, const float* lse, float* workspace, void* dq, void* dk,
                                  void* dv, int B, int N, int M, int H, int HKV, int D, int window, float scale,
                                  void* stream);
int vsp_window_attn_backward_f16(const void* q, const void* keys, const void* values, const void* o,
                                 const void* dout, const float* lse, float* workspace, void* dq, void* dk,
                                 void* dv, int B, int N, int M, int H, int HKV, int D, int window, float scale,
                                 void* stream);

/* ---- the attention window across chunks and the rotary embedding ---------------------------
 * The chronological window (vesper/attention.py:30-59, 142-175, `KVCache`, `kv_cache_push`): from
 * a cache of M <= window entries (cache_k, cache_v [B, M, HKV, D], cache_pos [B, M] int64, oldest
 * first) and a chunk of N (k, v [B, N, HKV, D], pos [B, N]), write the newest min(M + N, window)
 * entries, oldest first, into out_k, out_v [B, keep, HKV, D] and out_pos [B, keep] (fresh buffers;
 * the inputs are not changed). elem_bytes 2 (bf16/f16) or 4 (fp32); one launch for all three. */
int vsp_kv_cache_push(const void* cache_k, const void* cache_v, const int64_t* cache_pos, const void* k,
                      const void* v, const int64_t* pos, void* out_k, void* out_v, int64_t* out_pos, int B, int M,
                      int N, int HKV, int D, int elem_bytes, int window, void* stream);

/* Rotary position embedding (vesper/attention.py:178-217, `rotary`, as `WindowedAttention.project`
 * applies it to q and k, attention.py:292): q [B, N, H, D] and k [B, N, HKV, D] (HKV may be 0 and
 * k, k_out NULL) at int64 positions pos [B, N]; pair j of a token at position p turns by the angle
 * p * inv_freq[j] (inv_freq: [D / 2] float64 on the device, base^(-2j/D) as the host computes it),
 * in float64; cos and sin are cast to the dtype, and the rotation is computed in it with every
 * product and sum rounded to it. The outputs may be the inputs (in place). D even, <= 1024. */
int vsp_rotary_qk_bf16(const void* q, const void* k, const int64_t* pos, const double* inv_freq, void* q_out,
                       void* k_out, int B, int N, int H, int HKV, int D, void* stream);
int vsp_rotary_qk_f16(const void* q, const void* k, const int64_t* pos, const double* inv_freq, void* q_out,
                      void* k_out, int B, int N, int H, int HKV, int D, void* stream);
int vsp_rotary_qk_f32(const float* q, const float* k, const int64_t* pos, const double* inv_freq, float* q_out,
                      float* k_out, int B, int N, int H, int HKV, int D, void* stream);

/* ---- decode: one new token per row over a KV ring ------------------------------------------
 * q: [B, H, D]; k, v: [B, HKV, D] (the new token); pos: [B] int64, nonnegative;
 * ring_k, ring_v: [B, window, HKV, D]; ring_pos: [B, window] int64; ring_valid: [B, window] uint8.
 * The query at position p attends valid slots with a position in (p - window, p] and the new token
 * itself; o: [B, H, D]. With `write` nonzero the new token is then written into slot p % window
 * (keys, values, position, valid flag) in place, after every read of the call, by the same launch.
 * The contract of vesper/attention.py:298-338 (`attend_ring`, without the projections) and
 * vesper/attention.py:104-139 (`kv_ring_write`); the reference runs masked SDPA there.
 * D a multiple of 8 up to 256; at most 8 query heads per KV head; q, k, v and the ring's keys and
 * values 16-byte aligned; active: [B] or NULL (an inactive row reads zeros and still writes its
 * token). `workspace` (needed when `write` is nonzero) holds vsp_ring_attn_workspace_bytes(B)
 * bytes of per-row arrival counters: zero before the first call, and every call leaves it zero.
 * Calls that overlap in time must not share a workspace. */
size_t vsp_ring_attn_workspace_bytes(int B);
int vsp_ring_attn_bf16(const void* q, const void* k, const void* v, const int64_t* pos, void* ring_k, void* ring_v,
                       int64_t* ring_pos, uint8_t* ring_valid, void* o, const uint8_t* active, void* workspace,
                       size_t workspace_bytes, int B, int H, int HKV, int D, int window, float scale, int write,
                       void* stream);
int vsp_ring_attn_f16(const void* q, const void* k, const void* v, const int64_t* pos, void* ring_k, void* ring_v,
                      int64_t* ring_pos, uint8_t* ring_valid, void* o, const uint8_t* active, void* workspace,
                      size_t workspace_bytes, int B, int H, int HKV, int D, int window, float scale, int write,
                      void* stream);

/* The same with the ring's keys and values in float32 (ring_k, ring_v: [B, window, HKV, D] fp32,
 * 16-byte aligned), the ring the reference's CapturedDecoder allocates (vesper/decode.py:81,85 with
 * vesper/column.py:492) and attend_ring casts to the query dtype (vesper/attention.py:325): each
 * ring element is rounded to q's dtype (nearest even) as it is read, and the new token is written
 * into its slot widened to float32. q, k, v, o in bf16 (fp16 for the _f16 entry). */
int vsp_ring_attn_bf16_ring_f32(const void* q, const void* k, const void* v, const int64_t* pos, float* ring_k,
                                float* ring_v, int64_t* ring_pos, uint8_t* ring_valid, void* o, const uint8_t* active,
                                void* workspace, size_t workspace_bytes, int B, int H, int HKV, int D, int window,
                                float scale, int write, void* stream);
int vsp_ring_attn_f16_ring_f32(const void* q, const void* k, const void* v, const int64_t* pos, float* ring_k,
                               float* ring_v, int64_t* ring_pos, uint8_t* ring_valid, void* o, const uint8_t* active,
                               void* workspace, size_t workspace_bytes, int B, int H, int HKV, int D, int window,
                               float scale, int write, void* stream);

/* vsp_ring_attn_bf16 with no workspace argument and no allocation of any kind: the per-row arrival
 * counters live in a static device array of 65536 counters (256 KiB per GPU, held until the
 * process ends), whose address vsp_init takes and zeroes for the device current at set-up, and
 * this entry's first call on any other device (zeroed by a kernel on `stream`). No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). B at most 65536 (larger B is refused with
 * VSP_ERR_ARG); vsp_init must have run. Every call that writes the ring leaves the counters zero.
 * All calls on one GPU share the array: calls that overlap in time on one GPU (two streams)
 * race, so they must be ordered. */
int vsp_ring_attn_noalloc_bf16(const void* q, const void* k, const void* v, const int64_t* pos, void* ring_k,
                               void* ring_v, int64_t* ring_pos, uint8_t* ring_valid, void* o,
                               const uint8_t* active, int B, int H, int HKV, int D, int window, float scale,
                               int write, void* stream);

/* ---- the causal key filter and key normalization (before the scan) --------------------------
 * z: [B, N, D] key inputs (bf16, f16 or fp32); history: [B, K-1, D] fp32, the K-1 inputs before
 * the chunk, oldest first (may be NULL when K == 1); taps: [K, D] fp32, tap 0 on the current token.
 * keys: [B, N, D] = [B, N, heads, D / heads] in z's dtype:
 *   u[t, j] = sum_{r < K} taps[r, j] * z[t - r, j] (rows before the chunk from the history), then
 *   per head normalize_keys(u) = s / max(||s||, 1), s = u / max(max |u|, 1e-6).
 * The contract of vesper/column.py:255-289 (`RecurrentSublayer.keys`; the next history, the newest
 * K-1 inputs, is the caller's) as vesper/kernels/keys.py:28-32 (`fused_keys`, forward) computes it
 * on CUDA. K in 1..8; head width D / heads a power of two in 8..512; one batch row of z at most
 * 2 GiB; z, history, taps and keys 16-byte aligned. */
int vsp_key_filter_bf16(const void* z, const float* history, const float* taps, void* keys, int B, int N, int D,
                        int heads, int K, void* stream);
int vsp_key_filter_f16(const void* z, const float* history, const float* taps, void* keys, int B, int N, int D,
                       int heads, int K, void* stream);
int vsp_key_filter_f32(const float* z, const float* history, const float* taps, float* keys, int B, int N, int D,
                       int heads, int K, void* stream);
/* The whole key step of RecurrentSublayer.keys (vesper/column.py:255-289, which returns the keys
 * and the next history): the keys as vsp_key_filter_*, optionally
 * - with the copy-forward fused into the filter's loads (the carry merge of the key inputs before
 *   the filter, vesper/column.py:779-782, `where(active, z, z_carried)`): token t's input row (as
 *   the current token and in the halo of later ones) is z_carried's row t where active[b, t] == 0;
 *   z_carried ([B, N, D], z's dtype) and active go together or are both NULL;
 * - writing the next history, the newest K - 1 inputs of (history, the chunk as read) in float32,
 *   into history_out [B, K-1, D] (NULL: not written; it must not overlap history, or it is history
 *   itself for a chunk of at most 16 tokens with bf16/fp16 z, 8 with fp32 z: the in-place update
 *   of a decode step).
 * The rows of z for inactive tokens are never read. */
int vsp_key_step_bf16(const void* z, const void* z_carried, const uint8_t* active, const float* history,
                      const float* taps, void* keys, float* history_out, int B, int N, int D, int heads, int K,
                      void* stream);
int vsp_key_step_f16(const void* z, const void* z_carried, const uint8_t* active, const float* history,
                     const float* taps, void* keys, float* history_out, int B, int N, int D, int heads, int K,
                     void* stream);
int vsp_key_step_f32(const float* z, const float* z_carried, const uint8_t* active, const float* history,
                     const float* taps, float* keys, float* history_out, int B, int N, int D, int heads, int K,
                     void* stream);

/* normalize_keys (vesper/recurrence.py:91-115) on `rows` rows of any width, x and y [rows, width]
 * contiguous in one dtype: y = s / max(||s||, 1), s = x / max(max |x|, 1e-6), float32 arithmetic
 * (the peak division correctly rounded, so the peak component becomes exactly 1), rounded to the
 * dtype. The row form for widths the key filter does not take (above 512, or not a power of two),
 * up to the reference's 65536-wide rows (tests/test_recurrence_review.py:61-64). The backward
 * gives grad_x from grad_y with the peak held constant (recurrence.py:103-105). One wave a row;
 * deterministic. rows == 0 or width == 0 writes nothing. */
int vsp_normalize_keys_bf16(const void* x, void* y, int64_t rows, int width, void* stream);
int vsp_normalize_keys_f16(const void* x, void* y, int64_t rows, int width, void* stream);
int vsp_normalize_keys_f32(const float* x, float* y, int64_t rows, int width, void* stream);
int vsp_normalize_keys_backward_bf16(const void* x, const void* grad_y, void* grad_x, int64_t rows, int width,
                                     void* stream);
int vsp_normalize_keys_backward_f16(const void* x, const void* grad_y, void* grad_x, int64_t rows, int width,
                                    void* stream);
int vsp_normalize_keys_backward_f32(const float* x, const float* grad_y, float* grad_x, int64_t rows, int width,
                                    void* stream);

/* The key filter's backward (vesper/kernels/keys.py:46-78, `_FusedKeys.backward`, on CUDA
 * vesper/kernels/keys_triton.py:56-177): from grad_keys [B, N, D] (z's dtype), with the
 * normalization's peak held constant (vesper/recurrence.py:103-105),
 *   grad_z [B, N, D] (z's dtype), grad_taps [K, D] fp32, and grad_history [B, K-1, D] fp32 (skipped
 *   when NULL). Deterministic: no atomics, the taps' partial sums added in a fixed order.
 * Same shape limits as the forward; workspace of vsp_key_filter_backward_workspace_bytes bytes
 * (16-byte aligned, contents ignored). B == 0 or N == 0 writes zero gradients. */
size_t vsp_key_filter_backward_workspace_bytes(int B, int N, int D, int K);
int vsp_key_filter_backward_bf16(const void* z, const float* history, const float* taps, const void* grad_keys,
                                 void* grad_z, float* grad_taps, float* grad_history, void* workspace,
                                 size_t workspace_bytes, int B, int N, int D, int heads, int K, void* stream);
int vsp_key_filter_backward_f16(const void* z, const float* history, const float* taps, const void* grad_keys,
                                void* grad_z, float* grad_taps, float* grad_history, void* workspace,
                                size_t workspace_bytes, int B, int N, int D, int heads, int K, void* stream);
int vsp_key_filter_backward_f32(const float* z, const float* history, const float* taps, const float* grad_keys,
                                float* grad_z, float* grad_taps, float* grad_history, void* workspace,
                                size_t workspace_bytes, int B, int N, int D, int heads, int K, void* stream);

/* ---- the sublayers' pre-normalization of the looped column -----------------------------------
 * RMSNorm (vesper/column.py:146-188): out = x / sqrt(mean(x^2) + 1e-6) * gain per row of `d`
 * floats, computed scale-safely as the reference does (each row divided by its peak magnitude
 * floored at 1e-3 first); x: [rows, d] float32, gain: [d] float32 or NULL (all ones), out:
 * [rows, d] bf16, the projections' operand. d a multiple of 8 in 8..2048; x, gain, out 16-byte
 * aligned. */
int vsp_rms_norm_bf16(const float* x, const float* gain, void* out, int rows, int d, void* stream);
/* The same norm of s = x + residual (residual [rows, d] bf16, added in float32 as the column's
 * residual add does: vesper/column.py:779-796), with s also written to sum_out ([rows, d] float32,
 * or NULL; it must not overlap x): the add and the norm in one launch, bitwise the two launches'.
 * x, residual, sum_out, gain and out 16-byte aligned. */
int vsp_add_rms_norm_bf16(const float* x, const void* residual, float* sum_out, const float* gain, void* out, int rows,
                          int d, void* stream);

/* The decode step's projection of that normalized stream, fused (the looped column's per-pass
 * projections, vesper/column.py:192-260 and vesper/attention.py:269-292, for a decode step of M
 * single-token rows): s = x + residual (float32; residual [M, d] bf16 or NULL) is written to
 * sum_out ([M, d] float32, or NULL; it must not overlap x), z = RMSNorm(s, gain) in bf16 exactly as
 * vsp_rms_norm_bf16 computes it, and for each of the nblk (1..4) weight blocks
 * out_j = z W_j [:, :used_j] (bf16, [M, used_j] contiguous, fp32 accumulation), W_j [d, cols] the
 * block's weight passed transposed: weights_t [nblk, cols, d] bf16. Block sigmoid_block (or -1 for
 * none) is stored as the logistic of its bf16-rounded product (the write strength). d a multiple
 * of 32 in 32..2048; 1 <= used_j <= cols; x, residual, sum_out, gain and weights_t 16-byte
 * aligned, the outputs 4-byte aligned. Blocks j with bit j of rotate_mask set are rotated as they
 * are stored, as vsp_rotary_qk_bf16 rotates them (heads of rotary_dk columns, token m at
 * positions[m] (int64 [M]), inv_freq the float64 [rotary_dk / 2] table): bitwise the separate
 * launch's q and k; used_j a multiple of rotary_dk. */
int vsp_decode_proj_bf16(const float* x, const void* residual, float* sum_out, const float* gain,
                         const void* weights_t, int nblk, int cols, int d, int M, int used0, int used1, int used2,
                         int used3, void* out0, void* out1, void* out2, void* out3, int sigmoid_block,
                         const int64_t* positions, const double* inv_freq, int rotate_mask, int rotary_dk,
                         void* stream);

/* The same stacked projections for a prefill (the looped column's per-pass projections of M
 * tokens' normalized input, vesper/column.py:192-260 and vesper/attention.py:269-292): for each of
 * the nblk (1..4) weight blocks out_j = z W_j [:, :used_j] (bf16, [M, used_j] contiguous, fp32
 * accumulation), z [M, d] bf16, W_j [d, cols] the block's weight passed transposed: weights_t
 * [nblk, cols, d] bf16. Only the used columns are computed. Block sigmoid_block (or -1) is stored
 * as the logistic of its bf16-rounded product, as vsp_decode_proj_bf16 stores it. d a multiple of
 * 64 in 64..16384, 1 <= used_j <= cols, z and each weight block under 4 GiB (with a 256-row
 * margin), z, weights_t and the outputs 16-byte aligned (the outputs may be NULL when M is 0). */
int vsp_project_bf16(const void* z, const void* weights_t, int nblk, int cols, int d, int M, int used0, int used1,
                     int used2, int used3, void* out0, void* out1, void* out2, void* out3, int sigmoid_block,
                     void* stream);

/* ---- copy-forward bookkeeping of the looped column ------------------------------------------
 * Replaces the row-wise `where` selects of vesper/loop.py:523-537 (`_merge`: tokens halting now
 * freeze their fresh projections into the carried ones) and vesper/loop.py:441-452 (a halted
 * token's hidden state carried forward): for each of `count` (0..8) tensors of `rows` rows of
 * row_bytes[i] bytes, dst[i][r] = src[i][r] where flags[i][r] != 0, in place, one launch; the
 * rows whose flag is 0 are neither read nor written. src, dst, row_bytes, flags are host arrays of
 * `count` entries; the device buffers hold rows * row_bytes[i] bytes each. */
int vsp_copy_rows_where(int count, const void* const* src, void* const* dst, const size_t* row_bytes,
                        const uint8_t* const* flags, int rows, void* stream);

/* The pass loop's halting bookkeeping for one pass (vesper/loop.py:441-452; the pass count of the
 * loop's LoopResult): over count tokens (bool bytes), halts = active & exits (exits NULL: every
 * active token halts, the last pass), n_iters += active (int32, in place), next = active & !halts.
 * One launch for the five elementwise steps; halts and next must not be active. */
int vsp_halt_step(const uint8_t* active, const uint8_t* exits, int* n_iters, uint8_t* halts, uint8_t* next, int count,
                  void* stream);

/* The residual stream after a pass's attention for the rows still in the loop (vesper/loop.py:452
 * with the column's residual add): x[r] = x1[r] + a[r] (x1, x float32 [rows, d]; a bf16 [rows, d],
 * added in float32) where flags[r] != 0, every row when flags is NULL; other rows of x are left
 * as they are. d a multiple of 8; x1, a, x 16-byte aligned; x must not overlap x1 or a. */
int vsp_residual_rows_where(const float* x1, const void* a, float* x, const uint8_t* flags, int rows, int d,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VESPER_KERNELS_H */
