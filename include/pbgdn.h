/*
 * pbgdn.h - C ABI of the MI355X (gfx950) Gated DeltaNet operator.
 *
 * Two entry points carry the compute, each the device-side replacement of one
 * kernel of the reference module pseudobrain/gated_deltanet.py:
 *
 *   pbgdn_chunk_fwd      chunkwise prefill; replaces the fla custom op
 *                        `pseudobrain::gated_delta_chunk` (_fla_chunk_op,
 *                        gated_deltanet.py:200-216) behind delta_rule_fla
 *                        (gated_deltanet.py:280-285), and computes the same
 *                        recurrence as delta_rule_chunked (gated_deltanet.py:110-165).
 *   pbgdn_recurrent_fwd  per-token recurrence (decode steps, T <= SEQUENTIAL_MAX);
 *                        replaces delta_rule_sequential (gated_deltanet.py:93-107);
 *                        pbgdn_recurrent_verify_fwd is its speculative-verify
 *                        form (the state after every token kept in a slot).
 *
 * Two more carry the layer-side work on either side of the recurrence:
 *
 *   pbgdn_prologue_fwd   short convolution + SiLU, q/k L2 norm, decay/beta
 *                        gates (GatedDeltaNetLayer.forward, gated_deltanet.py:415-429,
 *                        short_convolution :314-338, l2_normalize :59-70);
 *   pbgdn_epilogue_fwd   per-head RMSNorm x o_norm x SiLU(gate) (:439-441);
 *   pbgdn_prologue_varlen_fwd  the prologue over packed sequences, each with
 *                        its own tail in a pool of slots (the serving form).
 *
 * and one fuses all three for the decode step (one token per sequence):
 *
 *   pbgdn_decode_layer_fwd  projection row -> conv, norms, gates -> recurrent
 *                        step -> RMSNorm/gate output, conv tail and state
 *                        updated in place in their slot pools.
 *
 * Conventions (all entry points):
 *   - every pointer is device memory owned by the caller; nothing is allocated
 *     (scratch memory comes in as a caller-provided workspace);
 *   - tensors are dense row-major in the reference layouts:
 *       q, k  [B, T, Hk, K]     v, o  [B, T, Hv, V]     g, beta  [B, T, Hv]
 *       states [N, Hv, K, V] in state_dtype (F32, BF16 or F16; serving caches
 *       may keep the state in the model's dtype), S stored [d_k, d_v] per head;
 *   - GQA: value head h reads query/key head h / (Hv / Hk)
 *     (repeat_interleave, gated_deltanet.py:422-424); Hk == Hv is the
 *     reference's already-repeated layout;
 *   - g is the log decay (<= 0), float32; beta float32 or the q/k/v dtype;
 *   - arithmetic: the state and every accumulation are float32 inside the
 *     kernels; a 16-bit state is widened when it is read and rounded to
 *     nearest even when it is written;
 *   - launches are asynchronous on `stream` (a hipStream_t; NULL = the null
 *     stream); no host synchronisation; safe to call from several threads.
 *     Nothing a call computes depends on earlier calls: the library keeps
 *     only per-device facts it queries once (compute units, XCDs, kernel LDS
 *     limits, the no-allocation scratch address), and the decode steps' cache
 *     policy is the caller's state_policy argument;
 *   - return 0 (PBGDN_OK) or a PBGDN_ERR_* code; no exception crosses the ABI.
 */
#ifndef PBGDN_H_
#define PBGDN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PBGDN_ABI_VERSION 14

/* element types */
#define PBGDN_F32 0
#define PBGDN_BF16 1
#define PBGDN_F16 2

/* status codes */
#define PBGDN_OK 0
#define PBGDN_ERR_INVALID_ARGUMENT 1 /* a null pointer, a bad size or dtype code */
#define PBGDN_ERR_UNSUPPORTED 2      /* valid, but a head width / chunk this library has no kernel for */
#define PBGDN_ERR_LAUNCH 3           /* the HIP launch failed (hipGetLastError) */
#define PBGDN_ERR_SCRATCH 4          /* more workspace than pbgdn_chunk_fwd_noalloc's scratch holds */

/* Cache policy of a decode step's state (pbgdn_recurrent_fwd at T = 1,
 * pbgdn_decode_layer_fwd), named by the caller:
 *   PBGDN_STATE_STREAM    the state comes from HBM and goes back past the
 *                         last-level cache (non-temporal): a model whose
 *                         layers each keep a pool steps a different pool every
 *                         call, so no state is still cached when it is read
 *                         again (float32 state, B = 64, Qwen3-Next heads: 69%
 *                         of 8 TB/s, against 61% with cacheable accesses);
 *   PBGDN_STATE_RESIDENT  the caller steps the same pool again before much
 *                         else passes through the 256 MB last-level cache (one
 *                         layer stepped in a loop): cacheable accesses keep it
 *                         there (83% of 8 TB/s, against 71% streamed); taken
 *                         only when the call moves at most 192 MiB of state,
 *                         larger calls stream.
 * The policy sets cache bits only: results are the same bit for bit. */
#define PBGDN_STATE_STREAM 0
#define PBGDN_STATE_RESIDENT 1

/* Version of this ABI (PBGDN_ABI_VERSION). */
int pbgdn_abi_version(void);

/* Static text for a status code. */
const char *pbgdn_status_string(int status);

/*
 * Chunkwise prefill (chunk = 64 tokens).
 *
 * Reference: _fla_chunk_op (pseudobrain/gated_deltanet.py:200-216) and
 * delta_rule_chunked (gated_deltanet.py:110-165); the semantics are those of
 * gated_delta_rule(q, k, v, g, beta, scale, h0) (gated_deltanet.py:300-308)
 * with cu_seqlens varlen packing added.
 *
 *   q, k        [B, T, Hk, K]   dtype in_dtype (F32, BF16 or F16)
 *   v           [B, T, Hv, V]   dtype in_dtype
 *   g           [B, T, Hv]      float32 log decay
 *   beta        [B, T, Hv]      dtype beta_dtype (F32 or in_dtype)
 *   h0          [N, Hv, K, V]   initial states in state_dtype, or NULL for zeros
 *   cu_seqlens  [N + 1] int32 sequence boundaries into the T axis (B must be
 *               1, cu_seqlens[0] == 0, cu_seqlens[N] == T, nondecreasing), or
 *               NULL: then N = B sequences of T tokens each
 *   o           [B, T, Hv, V]   dtype out_dtype (F32 or in_dtype; another
 *               type is PBGDN_ERR_UNSUPPORTED), written
 *   ht          [N, Hv, K, V]   final states in state_dtype, written (may be
 *               NULL; may equal h0 for an in-place state update)
 *   state_dtype element type of h0 and ht (F32, BF16 or F16)
 *   state_idx   NULL, or [N] int32 state slot of each sequence: then h0 and ht
 *               are pools of num_states slots [num_states, Hv, K, V] (either
 *               may be NULL, and they may be the same pool), sequence n starts
 *               from slot state_idx[n] of h0 and its final state goes to slot
 *               state_idx[n] of ht; a slot outside [0, num_states) starts from
 *               zeros and keeps no final state; the slots of one call must be
 *               distinct (vLLM's per-request state slots,
 *               serving/pb27_vllm/pb27_vllm/universal_models.py:147-165)
 *   has_initial_state NULL, or [N] uint8: 0 starts sequence n from zeros
 *               instead of h0 (a new request whose slot holds stale data)
 *   num_states  slots in the pools (ignored when state_idx is NULL)
 *   num_seqs    N (must equal B when cu_seqlens is NULL)
 *   scale       query scale (the reference passes K ** -0.5)
 *   chunk       must be 64 (CHUNK, gated_deltanet.py:49)
 *   workspace   device scratch of at least pbgdn_chunk_workspace_size(B, T,
 *               Hv, num_seqs, in_dtype) bytes, 16-byte aligned: per-chunk intermediates
 *               (Tb, Q K^T o D, decays) passed from the first kernel of the
 *               call to the second; its contents need no initialisation and
 *               are dead when the call's work on `stream` completes
 *
 * Supported: K in {64, 128} with V a multiple of 16, and K = 256 with in_dtype
 * BF16 or F16 and V a multiple of 32 (keys 128 < K <= 256 zero-padded to 256
 * by the caller; the padded keys add nothing); Hv a multiple of Hk.
 * Ranges: the products run on fp16/bf16 MFMA operands with fp32 accumulation;
 * a chunk whose intermediate V - gamma K S leaves the fp16 range is scaled by
 * a power of two internally. With in_dtype F32, q and k enter as fp16
 * (|q|, |k| < 65504), the state as an fp16 high/low pair, and U = Tb X (the
 * WY product that carries the state update) is formed from fp16 high/low
 * pairs of Tb and X (final-state error ~3e-4 where single fp16 operands gave
 * 7-9e-4); the call first
 * computes on the device the power of two that brings max |v| and max |h0|
 * (over the states it reads) within 1024, runs on the scaled v and h0 and
 * scales o and ht back, exactly (the recurrence is linear in v and h0), so
 * any finite float32 v and h0 are in range.
 */
int pbgdn_chunk_fwd(const void *q, const void *k, const void *v, int in_dtype,
                    const float *g, const void *beta, int beta_dtype,
                    const void *h0, void *ht, int state_dtype,
                    const int32_t *state_idx, const uint8_t *has_initial_state,
                    int num_states, const int32_t *cu_seqlens, int num_seqs,
                    void *o, int out_dtype, int B, int T, int Hk, int Hv,
                    int K, int V, float scale, int chunk, void *workspace,
                    size_t workspace_bytes, void *stream);

/*
 * The layer core of a prefill: pbgdn_chunk_fwd followed by the epilogue of
 * pbgdn_epilogue_fwd, hs = o rsqrt(mean(o^2) + eps) o_norm SiLU(gate) per
 * (token, value head). Reference: GatedDeltaNetLayer.forward,
 * gated_deltanet.py:437-441 (gated_delta_rule, then the norm and gate).
 *
 *   q .. num_seqs, B .. stream   as pbgdn_chunk_fwd
 *   gate        [B, T, gate_stride] rows, value head h at columns h V .. h V + V - 1
 *               (a column slice of the projection), dtype gate_dtype;
 *               gate_stride >= Hv V, a multiple of 8
 *   o_norm      [V] float32; eps >= 0
 *   hs          [B, T, Hv V] dtype hs_dtype, written
 *   o           [B, T, Hv, V] in in_dtype: the operator's output when the
 *               epilogue runs as a pass of its own (written then), else unused
 *
 * When the wide scan takes the call (in_dtype BF16 or F16, K = V = 128, N x
 * Hv at least half the device's CUs, gate_dtype == in_dtype, hs_dtype F32 or
 * in_dtype), the scan applies the epilogue to each chunk's output in
 * registers (fp32, before any rounding) and writes hs: o is not touched (it
 * may be NULL) and the epilogue pass, with its read of o, is saved. Otherwise
 * o is written in in_dtype and the epilogue runs after it on the same stream.
 * pbgdn_chunk_layer_fuses tells the two apart before the call. V must be 64
 * or 128 (the epilogue's widths).
 */
int pbgdn_chunk_layer_fwd(const void *q, const void *k, const void *v,
                          int in_dtype, const float *g, const void *beta,
                          int beta_dtype, const void *h0, void *ht,
                          int state_dtype, const int32_t *state_idx,
                          const uint8_t *has_initial_state, int num_states,
                          const int32_t *cu_seqlens, int num_seqs,
                          const void *gate, long gate_stride, int gate_dtype,
                          const float *o_norm, float eps, void *hs,
                          int hs_dtype, void *o, int B, int T, int Hk, int Hv,
                          int K, int V, float scale, int chunk,
                          void *workspace, size_t workspace_bytes,
                          void *stream);

/*
 * Bytes of workspace pbgdn_chunk_fwd needs for a call with these sizes
 * (B * T tokens in num_seqs sequences, Hv value heads) and input dtype: 13 KiB
 * per 64-token chunk and value head for 16-bit inputs, 19 KiB for float32
 * (the low part of Tb as well), plus 4 KiB (float32 inputs' range scale).
 * 0 for invalid sizes or dtype. No reference counterpart: the reference
 * materialises the same per-chunk tensors (gated_deltanet.py:143-157) with
 * torch allocations.
 */
size_t pbgdn_chunk_workspace_size(int B, int T, int Hv, int num_seqs, int in_dtype);

/* Bytes of device scratch each GPU holds for pbgdn_chunk_fwd_noalloc (64 MiB). */
#define PBGDN_NOALLOC_SCRATCH_BYTES (64u << 20)

/*
 * pbgdn_chunk_fwd without a workspace argument and without any allocation:
 * the prefill's workspace records live in a device array of
 * PBGDN_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on
 * until the process ends. No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, allocation-free serving
 * loops, harnesses that forbid hipMalloc).
 *
 * Arguments, results and kernels are those of pbgdn_chunk_fwd; `stream` must
 * belong to the current device (PBGDN_ERR_INVALID_ARGUMENT otherwise). A call
 * whose pbgdn_chunk_workspace_size(B, T, Hv, num_seqs, in_dtype) exceeds
 * PBGDN_NOALLOC_SCRATCH_BYTES returns PBGDN_ERR_SCRATCH and launches nothing
 * (e.g. at Hv = 32 about 9,900 tokens in one sequence; at Hv = 16 twice that).
 * Every call on one GPU shares that GPU's array: calls whose work overlaps on
 * one GPU (other streams, other threads) race and must be serialised by the
 * caller. The array keeps the last call's contents; nothing in it needs
 * clearing (each call writes every record it reads).
 */
int pbgdn_chunk_fwd_noalloc(const void *q, const void *k, const void *v,
                            int in_dtype, const float *g, const void *beta,
                            int beta_dtype, const void *h0, void *ht,
                            int state_dtype, const int32_t *state_idx,
                            const uint8_t *has_initial_state, int num_states,
                            const int32_t *cu_seqlens, int num_seqs, void *o,
                            int out_dtype, int B, int T, int Hk, int Hv, int K,
                            int V, float scale, int chunk, void *stream);

/*
 * 1 when pbgdn_chunk_layer_fwd with these arguments applies the epilogue
 * inside the scan (its o argument then unused and allowed to be NULL), 0 when
 * it writes o and runs the epilogue as a second pass (o required), on the
 * current device; -1 for arguments pbgdn_chunk_layer_fwd would reject as
 * invalid dtypes or widths. Lets a caller allocate o only when it is written.
 * No reference counterpart (the reference always materialises o).
 */
int pbgdn_chunk_layer_fuses(int in_dtype, int gate_dtype, int hs_dtype, long gate_stride, int num_seqs, int Hv,
                            int K, int V);

/*
 * Fused recurrent steps: for each token, in one pass over the state,
 *   S <- exp(g) S;  u = beta (v - S^T k);  S <- S + k u^T;  o = S^T (q scale).
 *
 * Reference: delta_rule_sequential (pseudobrain/gated_deltanet.py:93-107),
 * the kernel gated_delta_rule selects for T <= SEQUENTIAL_MAX (:291-297) and
 * for one-token decode.
 *
 *   q, k        [B, T, Hk, K]   dtype in_dtype
 *   v           [B, T, Hv, V]   dtype in_dtype
 *   g, beta     [B, T, Hv]      g float32, beta beta_dtype
 *   state_in    [S, Hv, K, V]   states read (S = num_states), state_dtype
 *   state_out   [S, Hv, K, V]   states written, state_dtype; may equal state_in
 *               (in-place update: each state is read whole before it is written;
 *               the slots of one call must be distinct)
 *   state_idx   [B] int32 state slot of each sequence, or NULL for slot b;
 *               a slot outside [0, num_states) (e.g. -1 padding) is skipped:
 *               no state is touched and that sequence's o is written as zeros
 *   num_states  S (must be >= B when state_idx is NULL)
 *   state_dtype F32, BF16 or F16 (both state tensors); they must be aligned
 *               to 4 elements; q, k, v to 16 bytes, g and beta to 4 bytes
 *   o           [B, T, Hv, V]   dtype out_dtype
 *   state_policy PBGDN_STATE_STREAM or PBGDN_STATE_RESIDENT (above): the
 *               state's cache policy for a one-token step; calls of more than
 *               one token read and write each state once and ignore it
 *
 * Supported: K in {32, 64, 128, 256}, V in {32, 64, 128, 256}.
 */
int pbgdn_recurrent_fwd(const void *q, const void *k, const void *v,
                        int in_dtype, const float *g, const void *beta,
                        int beta_dtype, const void *state_in,
                        void *state_out, int state_dtype,
                        const int32_t *state_idx,
                        int num_states, void *o, int out_dtype, int B, int T,
                        int Hk, int Hv, int K, int V, float scale,
                        int state_policy, void *stream);

/*
 * Speculative verify: the recurrent steps of pbgdn_recurrent_fwd over the T
 * tokens of each sequence (the accepted token and T-1 draft tokens), writing
 * the state after every token to its own slot, so that the state after the
 * last accepted token can be kept (vLLM keeps conv-1+num_spec rows of the
 * conv state and a slot per draft token of the recurrent state,
 * serving/pb27_vllm/pb27_vllm/universal_models.py:147-165).
 * No reference counterpart: the reference's serving path delegates it to vLLM.
 *
 *   state_in         [S, Hv, K, V] states read, state_dtype
 *   states           [S, Hv, K, V] states written, state_dtype (may equal
 *                    state_in)
 *   state_idx        [B] int32 slot of each sequence's starting state, or
 *                    NULL for slot b; a slot outside [0, S) gives zero output
 *                    and writes nothing
 *   token_state_idx  [B, T] int32 slot that receives the state after token t
 *                    of sequence b; a slot outside [0, S) is skipped. The
 *                    starting states are read whole before anything is
 *                    written; the slots a call writes must be distinct and
 *                    must not be another sequence's starting slot
 *   q, k, v, g, beta, o, scale, state_dtype: as pbgdn_recurrent_fwd
 */
int pbgdn_recurrent_verify_fwd(const void *q, const void *k, const void *v,
                               int in_dtype, const float *g, const void *beta,
                               int beta_dtype, const void *state_in,
                               void *states, int state_dtype,
                               const int32_t *state_idx,
                               const int32_t *token_state_idx, int num_states,
                               void *o, int out_dtype, int B, int T, int Hk,
                               int Hv, int K, int V, float scale, void *stream);

/*
 * Layer prologue: from the input projection of a GatedDeltaNetLayer to the
 * operator's inputs, in one pass (gated_deltanet.py:415-429):
 *   y = SiLU(causal depthwise conv of tail ++ qkv)            (:314-338)
 *   q, k = l2_normalize(y[q], y[k]) per key head, mode 'max' or 'hf' (:59-70)
 *   v = y[v]
 *   g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)   (:425-427)
 * The GQA repeat (:422-424) is not materialised: the operator maps heads.
 *
 *   qkv         [B, T, 2 Hk K + Hv V] rows of qkv_stride elements, in_dtype
 *               (the [q | k | v] columns of the projection)
 *   decay       [B, T, 2 Hv] rows of decay_stride elements, in_dtype
 *               (the [a | b] columns of the projection)
 *   tail        [B, conv-1, 2 Hk K + Hv V] tail_dtype: the last conv-1 inputs
 *               before qkv (NULL when conv <= 1); cast to in_dtype before the
 *               convolution, as the reference does
 *   tail_out    same shape: the last conv-1 inputs of tail ++ qkv; may be
 *               `tail` (NULL when conv <= 1)
 *   conv_weight [2 Hk K + Hv V, conv] float32, tap conv-1 on the current input
 *               (NULL when conv == 0: SiLU only)
 *   a_log, dt_bias [Hv] float32
 *   q, k        [B, T, Hk, K] out_dtype      v [B, T, Hv, V] out_dtype
 *   g, beta     [B, T, Hv] float32
 *   l2_mode     0 'max' (x / max(|x|, 1e-6)), 1 'hf' (x rsqrt(|x|^2 + 1e-6))
 *
 * Supported: K in {64, 128}; V a multiple of 8; conv in 0..4. qkv, q, k, v,
 * tail and tail_out 16-byte aligned; qkv_stride a multiple of 8.
 */
int pbgdn_prologue_fwd(const void *qkv, long qkv_stride, const void *decay,
                       long decay_stride, int in_dtype, const void *tail,
                       void *tail_out, int tail_dtype, const float *conv_weight,
                       int conv, const float *a_log, const float *dt_bias,
                       void *q, void *k, void *v, int out_dtype, float *g,
                       float *beta, int B, int T, int Hk, int Hv, int K, int V,
                       int l2_mode, void *stream);

/*
 * Layer epilogue (gated_deltanet.py:439-441), one pass:
 *   out = o rsqrt(mean_V(o^2) + eps) o_norm SiLU(gate)   per (token, value head)
 *
 *   o           [B, T, Hv, V] o_dtype (the operator's output)
 *   gate        [B, T, Hv V] rows of gate_stride elements, gate_dtype (the
 *               output-gate columns of the projection)
 *   o_norm      [V] float32
 *   eps         the per-head RMSNorm epsilon (the reference's norm_eps, 1e-5)
 *   out         [B, T, Hv V] out_dtype (the reference's hs before the out
 *               projection, in the hidden dtype)
 *
 * Supported: V in {64, 128}. o, gate, out 16-byte aligned; gate_stride a
 * multiple of 8.
 */
int pbgdn_epilogue_fwd(const void *o, int o_dtype, const void *gate,
                       long gate_stride, int gate_dtype, const float *o_norm,
                       float eps, void *out, int out_dtype, int B, int T,
                       int Hv, int V, void *stream);

/*
 * Layer prologue over packed sequences: pbgdn_prologue_fwd with B = 1 and N
 * sequences packed along T by cu_seqlens [N + 1], each convolving against its
 * own carried tail, kept in a pool of slots as a serving cache keeps conv
 * states. No reference counterpart as one call (the reference's layer works
 * on [B, T] batches with a tail per batch row, short_convolution,
 * gated_deltanet.py:314-338); the per-sequence arithmetic is that one.
 *
 *   qkv, decay, in_dtype, conv_weight, conv, a_log, dt_bias, q, k, v,
 *   out_dtype, g, beta, Hk, Hv, K, V, l2_mode: as pbgdn_prologue_fwd, B = 1
 *   tail        pool of tails, tail_dtype: row j (0 = oldest) of channel c of
 *               slot s at element s * tail_slot_stride + j * tail_row_stride
 *               + c * tail_chan_stride ([S, conv-1, C] and the channel-major
 *               [S, C, conv-1] both work); NULL when conv <= 1
 *   cu_seqlens  [N + 1] int32, nondecreasing from 0 to T (a bound outside
 *               [0, T] is clamped, never followed out of the buffer)
 *   tail_out    pool the new tails go to, same layout; may be `tail` (every
 *               old tail element is read before the new one is written)
 *   slot_idx    [N] int32 slot of each sequence, or NULL for slot n; a slot
 *               outside [0, num_slots) starts from a zero tail and keeps no
 *               new one; the slots of one call must be distinct
 *   has_initial_state [N] uint8, or NULL: 0 starts sequence n from a zero tail
 *
 * Supported: as pbgdn_prologue_fwd; N <= 65535.
 */
int pbgdn_prologue_varlen_fwd(const void *qkv, long qkv_stride,
                              const void *decay, long decay_stride,
                              int in_dtype, const int32_t *cu_seqlens,
                              int num_seqs, const void *tail, void *tail_out,
                              int tail_dtype, long tail_slot_stride,
                              long tail_row_stride, long tail_chan_stride,
                              const int32_t *slot_idx,
                              const uint8_t *has_initial_state, int num_slots,
                              const float *conv_weight, int conv,
                              const float *a_log, const float *dt_bias,
                              void *q, void *k, void *v, int out_dtype,
                              float *g, float *beta, int T, int Hk, int Hv,
                              int K, int V, int l2_mode, void *stream);

/*
 * Backward of pbgdn_chunk_fwd for [B, T] batches: the gradients the
 * reference's pseudobrain::gated_delta_chunk_backward returns
 * (gated_deltanet.py:230-277), given the gradients of o and of the final
 * state. It recomputes what it needs from the forward's inputs (no saved
 * intermediates): the state at every 64-token chunk start by a forward pass,
 * the state adjoint at every chunk end by a reverse pass, then each chunk's
 * gradients; all arithmetic float32.
 *
 *   q, k, v, in_dtype, g, beta, beta_dtype, h0, B, T, Hk, Hv, K, V, scale:
 *               as pbgdn_chunk_fwd without cu_seqlens (h0 [B, Hv, K, V]
 *               float32, or NULL for zeros)
 *   dout        [B, T, Hv, V] do_dtype: the gradient of o; do_dtype must be
 *               in_dtype (the reference casts it to q's dtype)
 *   dht         [B, Hv, K, V] float32 or NULL (zeros): the gradient of the
 *               final state
 *   dq, dk      [B, T, Hk, K] in_dtype (GQA: summed over the Hv/Hk value
 *               heads of each key head)
 *   dv          [B, T, Hv, V] in_dtype
 *   dg          [B, T, Hv] float32
 *   dbeta       [B, T, Hv] beta_dtype
 *   dh0         [B, Hv, K, V] float32, or NULL when not wanted
 *   workspace   device scratch of pbgdn_chunk_bwd_workspace_size(B, T, Hk,
 *               Hv, K, V) bytes, 16-byte aligned, no initialisation needed
 *               (per chunk: its start state, end adjoint, T, the dO terms)
 *
 * Supported: K, V in {64, 128}; at most 65,535 chunks per sequence and
 * 32,767 batch rows.
 */
int pbgdn_chunk_bwd(const void *q, const void *k, const void *v, int in_dtype,
                    const float *g, const void *beta, int beta_dtype,
                    const float *h0, const void *dout, int do_dtype,
                    const float *dht, void *dq, void *dk, void *dv, float *dg,
                    void *dbeta, float *dh0, void *workspace,
                    size_t workspace_bytes, int B, int T, int Hk, int Hv,
                    int K, int V, float scale, void *stream);

/* Workspace bytes pbgdn_chunk_bwd needs for these sizes. */
size_t pbgdn_chunk_bwd_workspace_size(int B, int T, int Hk, int Hv, int K,
                                      int V);

/*
 * Fused decode step of a GatedDeltaNetLayer: one token per sequence, from the
 * input projection to the layer output, in one launch (GatedDeltaNetLayer.forward
 * at T = 1, gated_deltanet.py:415-441: short_convolution :314-338,
 * l2_normalize :59-70, the gates :425-427, delta_rule_sequential :93-107, the
 * epilogue :439-441). q, k and v stay float32 between the convolution and the
 * recurrence, as on the reference's sequential path. No reference counterpart
 * as one call: the reference runs these as separate torch steps.
 *
 *   z           [B, z_stride] in_dtype rows of the projection, the columns
 *               [q | k | v | gate | a | b] (2 Hk K + 2 Hv V + 2 Hv of them)
 *   conv_state  pool of conv tails, conv_dtype: row j (0 = oldest) of channel c
 *               of slot s at element s * conv_slot_stride + j * conv_row_stride
 *               + c * conv_chan_stride (so [S, conv-1, C] and vLLM's
 *               channel-major [S, C, conv-1] both work); the tail shifts by one
 *               row in place; NULL when conv <= 1
 *   conv_weight [2 Hk K + Hv V, conv] float32 (NULL when conv == 0)
 *   a_log, dt_bias [Hv] float32; l2_mode as pbgdn_prologue_fwd
 *   state       pool [S, Hv, K, V] state_dtype, updated in place (aligned to
 *               4 elements)
 *   state_idx   [B] int32 slot of each sequence in both pools, or NULL for
 *               slot b; a slot outside [0, num_states) touches no pool and its
 *               output is zeros; the slots of one call must be distinct
 *   o_norm      [V] float32; eps the RMSNorm epsilon (the reference's 1e-5)
 *   hs          [B, Hv V] out_dtype, written
 *   scale       query scale (K ** -0.5)
 *   state_policy PBGDN_STATE_STREAM or PBGDN_STATE_RESIDENT (above)
 *
 * Supported: K, V in {64, 128}; conv 0..4; Hv a multiple of Hk, at most 8 Hk.
 */
int pbgdn_decode_layer_fwd(const void *z, long z_stride, int in_dtype,
                           void *conv_state, int conv_dtype,
                           long conv_slot_stride, long conv_row_stride,
                           long conv_chan_stride, const float *conv_weight,
                           int conv, const float *a_log, const float *dt_bias,
                           int l2_mode, void *state, int state_dtype,
                           const int32_t *state_idx, int num_states,
                           const float *o_norm, float eps, void *hs,
                           int out_dtype, int B, int Hk, int Hv, int K, int V,
                           float scale, int state_policy, void *stream);

/*
 * The residuals that pseudobrain::gated_delta_chunk returns beside o and the
 * final state (gated_deltanet.py:200-217, `_fla_chunk_op`: fla's gc and A for
 * 64-token chunks, which its backward op takes back at :230-249), from the
 * operator's own inputs:
 *
 *   gc  [B, T, Hv] float32: the inclusive cumulative sum of g within each
 *       64-token chunk, in token order
 *   a   [B, T, Hv, 64] a_dtype: row t of the chunk of token t of
 *       T = (I + strict_lower(beta_t (k_t . k_s) exp(gc_t - gc_s)))^-1, the
 *       `solve` of delta_rule_chunked (:141-149), in float32 arithmetic
 *
 * k [B, T, Hk, K] in k_dtype (value head h reads key head h / (Hv / Hk)), g
 * [B, T, Hv] float32, beta [B, T, Hv] in beta_dtype. Either output may be
 * NULL. Any K >= 1.
 */
int pbgdn_chunk_residuals(const void *k, int k_dtype, const float *g,
                          const void *beta, int beta_dtype, float *gc, void *a,
                          int a_dtype, int B, int T, int Hk, int Hv, int K,
                          void *stream);

/*
 * The inverse of gc: g_t = gc_t - gc_{t-1} within each 64-token chunk (gc_t
 * at a chunk's first token), [B, T, Hv] float32, gc and g distinct. What
 * pseudobrain::gated_delta_chunk_backward's callers hold is gc (:230-249);
 * pbgdn_chunk_bwd takes g. Each g_t comes back to within the rounding of the
 * cumulative sum it was added to.
 */
int pbgdn_chunk_decumulate(const float *gc, float *g, int B, int T, int Hv,
                           void *stream);

/*
 * Streaming copy of `bytes` from src to dst on `stream`: 16-byte non-temporal
 * buffer loads and stores, four pieces in flight per thread, 16 workgroups of
 * 256 threads per compute unit of the current device. No counterpart in the
 * reference: a measurement aid, the read + write bandwidth this GPU sustains
 * for a plain stream, against which the decode step's state traffic is
 * reported. bytes a multiple of 16, at most 2 GiB - 16; src and dst 16-byte
 * aligned and either equal (a pass in place: every piece is read before the
 * same thread writes it back) or not overlapping.
 */
int pbgdn_stream_probe(const void *src, void *dst, int64_t bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PBGDN_H_ */
