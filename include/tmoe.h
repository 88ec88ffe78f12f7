/*
 * tmoe.h — C ABI of libtmoe, the MI355X (gfx950) MoE-layer hot path.
 *
 * Conventions
 *   - Every pointer argument named x/out/ids/weights/... is a DEVICE pointer
 *     unless stated otherwise; sizes are plain ints.  bf16 tensors are passed as
 *     void* holding IEEE bfloat16 bit patterns, row-major, contiguous.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - Calls are asynchronous on `stream`; the return value reports argument
 *     validation and launch errors only (0 = TMOE_OK, negative = tmoe_status).
 *     Conditions the device detects (an expert id outside [0, E]) are recorded
 *     in the workspace and reported by tmoe_workspace_status().
 *   - Nothing here allocates device memory.  Callers pass a workspace of at
 *     least tmoe_workspace_bytes(...) bytes, ZERO-FILLED before its first use
 *     and not written by the caller afterwards: the kernels return its counters
 *     to zero and keep a call counter (epoch) in it.  Calls that share one
 *     workspace must be ordered (same stream, or joined with events).
 *   - T > 1 (dispatch and the prefill paths): T*k <= 524288.
 *   - Expert weights are reached through a device "expert table":
 *       bf16 table  uint64_t[E][2] = { gate_up [2I, H], down [H, I] } base pointers
 *       int4 table  uint64_t[E][4] = { gate_up packed [2I, H/2] u8, gate_up scales
 *                                      [2I, H/G] bf16, down packed [H, I/2] u8,
 *                                      down scales [H, I/G] bf16 }
 *     so expert ids never leave the device (no per-layer host sync, the
 *     reference's `top_k_index[0].tolist()` at tarfa/engine/fused_int4.py:166).
 *
 * Reference citations are into syncroot/tarfa (tarfa/...) and the transformers
 * 5.15.0 Qwen3.5-MoE modelling file it calls (transformers/...).
 */
#ifndef TMOE_H
#define TMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TMOE_ABI_VERSION 2

enum tmoe_status {
  TMOE_OK = 0,
  TMOE_ERR_NULL = -1,       /* a required pointer is NULL                          */
  TMOE_ERR_SHAPE = -2,      /* unsupported or inconsistent sizes                   */
  TMOE_ERR_ALIGN = -3,      /* a pointer is not 16-byte aligned                    */
  TMOE_ERR_WORKSPACE = -4,  /* workspace smaller than tmoe_workspace_bytes()       */
  TMOE_ERR_HIP = -5,        /* a HIP runtime call or kernel launch failed          */
  TMOE_ERR_EXPERT_ID = -6,  /* device saw an expert id outside [0, E] (sentinel E is skipped) */
  TMOE_ERR_TIMEOUT = -7,    /* a kernel's bounded dependency wait expired (results invalid)   */
  TMOE_ERR_SCRATCH = -8,    /* the call needs more than TMOE_STATIC_SCRATCH_BYTES (no-alloc entry point) */
};

/* ABI version of the loaded library (TMOE_ABI_VERSION at build time). */
int tmoe_abi_version(void);

/* Static text for a status code. */
const char* tmoe_strerror(int status);

/* Workspace bytes needed by any entry point below for T tokens at this shape
 * (Is = shared-expert intermediate size, 0 = no shared expert). */
size_t tmoe_workspace_bytes(int T, int H, int E, int I, int k, int Is);

/* Synchronise `stream`, then return and clear the device-side status the
 * kernels recorded in `workspace` (TMOE_OK, TMOE_ERR_EXPERT_ID or TMOE_ERR_TIMEOUT). */
int tmoe_workspace_status(void* workspace, void* stream);

/* ---------------------------------------------------------------- seeded data
 * Counter-based generator (splitmix64 output function over key + (i+1)*golden,
 * Irwin-Hall n=4 normal).  Stands in for the reference's seeded torch.randn
 * (tarfa/engine/moe_kernel.py:129-139) so any expert can be regenerated on the
 * host bit-identically.
 *   fill_bf16: dst[i] = bf16(fp32(c16(h_{start+i})) * scale)        (weights, activations)
 *   fill_f32 : dst[i] = fp32(double(c32(h_{2(start+i)}, h_{2(start+i)+1})) * scale)  (logits)
 */
int tmoe_fill_bf16(void* dst, uint64_t n, uint64_t key, float scale, uint64_t start, void* stream);
int tmoe_fill_f32(float* dst, uint64_t n, uint64_t key, double scale, uint64_t start, void* stream);

/* ---------------------------------------------------------------- router (a1)
 * Replaces Qwen3_5MoeTopKRouter.forward (transformers/.../modeling_qwen3_5_moe.py:768-776)
 * with fp32 logits: logits = x . router_w^T in fp32 (or `logits_in` when not NULL,
 * then x/router_w may be NULL), softmax in fp32, top-k by logit descending with
 * ties to the lower expert index, renormalised in fp32, weights cast to bf16.
 * ids_out [T,k] int64, weights_out [T,k] bf16, logits_out [T,E] fp32 (optional),
 * heat [E] uint32 (optional): heat[e] += 1 per selection (residency ledger).
 */
int tmoe_router_topk(const void* x, const void* router_w, const float* logits_in, int T, int H,
                     int E, int k, int64_t* ids_out, void* weights_out, float* logits_out,
                     uint32_t* heat, void* stream);

/* The boundary's re-truncation of a routing that carries more experts than the engine runs
 * (tarfa/engine/fused_int4.py:157-160, JTOPK at :17): per token keep the j largest of its k
 * bf16 weights (equal weights keep the lower slot first), gather their ids, and renormalise
 * in bf16: w'_r = bf16(w_r / bf16(sum of the kept weights)), the sum in fp32 in the kept
 * (descending) order.  ids [T,k] int64, weights [T,k] bf16 -> ids_out [T,j], weights_out [T,j];
 * 1 <= j <= k <= 16.
 */
int tmoe_topk_renorm_bf16(const int64_t* ids, const void* weights, int T, int k, int j,
                          int64_t* ids_out, void* weights_out, void* stream);

/* ---------------------------------------------------------------- dispatch (a3)
 * Token -> expert permutation of the reference's prefill
 * (tarfa/engine/fused_int4.py:228-229, 241): rows grouped by ascending expert id,
 * within an expert in (slot, token) order.  offsets [E+1] int32, perm [T*k] int32
 * with perm[r] = t*k + slot (entries past offsets[E] are unused); inv [T*k] int32
 * with inv[t*k + slot] = r (-1 for skipped ids).  Ids outside [0, E) are skipped.
 */
int tmoe_dispatch(const int64_t* ids, int T, int k, int E, int32_t* offsets, int32_t* perm,
                  int32_t* inv, void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- experts.forward (a2-a7)
 * Drop-in for the routed-compute step `experts.forward(hidden_states, top_k_index,
 * top_k_weights)` that the reference installs with types.MethodType
 * (tarfa/engine/fused_int4.py:155-262; same boundary channel.py:44-61).
 * x [T,H] bf16, ids [T,k] int64 (sentinel E skipped), weights [T,k] bf16, out [T,H] bf16.
 *   T == 1: per routed expert in router order, bf16(F.linear(bf16(silu(g))*u, Wd)),
 *           acc = bf16(acc + bf16(w_j * d_j))                (fused_int4.py:192-194)
 *   T  > 1: per token bf16 adds in ascending expert id (index_add_, fused_int4.py:239-244);
 *           2 <= T <= 16 with H, I multiples of 128 (bf16) streams each expert hit once
 *           (small-batch kernels), larger T runs dispatch and the grouped GEMM
 */
int tmoe_experts_forward_bf16(const void* x, int T, const int64_t* ids, const void* weights,
                              const uint64_t* expert_table, int H, int E, int I, int k, void* out,
                              void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- whole MoE block (a1-a8)
 * Replaces Qwen3_5MoeSparseMoeBlock.forward (transformers/.../modeling_qwen3_5_moe.py:787-798)
 * with the experts step above: router (fp32 logits), routed experts, shared expert
 * bf16(sigmoid(bf16(x.w_sg)) * down(bf16(silu(bf16(gate x))) * bf16(up x))), and
 * out = bf16(routed + shared).  router_w may be NULL when logits_in [T,E] fp32 is given;
 * the four shared pointers may all be NULL (Is = 0) for a layer without a shared expert.
 * ids_out / weights_out (optional) receive the routing; heat as in tmoe_router_topk.
 */
int tmoe_moe_block_bf16(const void* x, int T, const void* router_w, const float* logits_in,
                        const uint64_t* expert_table, const void* sh_gate, const void* sh_up,
                        const void* sh_down, const void* sh_gate_w, int H, int E, int I, int k,
                        int Is, void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                        void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- int4 format (a9)
 * Packed int4 rows with bf16 group scales, the group-scaled form of the reference's
 * format (tarfa/engine/channel_q4.py:10-14 dequant_int4, moe_kernel.py:110-114):
 *   packed [N, K/2] uint8: byte b holds column 2b (low nibble) and 2b+1 (high nibble),
 *          value = nibble - 8;   scales [N, K/G] bf16;
 *   dequant  w = bf16((nibble - 8) * scale[n, k / G])
 * tmoe_quantize_int4 (the reference has no quantiser; its int4 files come from
 * outside the repository, channel_q4.py:6):
 *   scale = bf16(max |w| over the group / 7)   (fp32 division, round to nearest even)
 *   q = clamp(rint(w / scale), -8, 7), q = 0 where scale == 0
 * w [N, K] bf16.  K a multiple of 8 and of G; G even, at most 2048.
 * tmoe_dequant_int4_bf16 materialises the bf16 matrix (debug / bit-exact checks);
 * packed must be 4-byte and out 16-byte aligned.
 */
int tmoe_quantize_int4(const void* w, int N, int K, int G, void* packed, void* scales, void* stream);
int tmoe_dequant_int4_bf16(const void* packed, const void* scales, int N, int K, int G, void* out,
                           void* stream);

/* ---------------------------------------------------------------- int4 fast mode (a10)
 * Labelled fast mode of the reference's decode (tarfa/engine/fused_int4.py:206-219 ->
 * moe_kernel.py:90-104 moe_ffn), with group-128 scales.  Expert table
 * uint64_t[E][4] (see above), entries 16-byte aligned.  Is == I or 0.
 *   T == 1 (H and I multiples of 512): per routed expert in router order, fp32
 *   gate/up dot products (int4 x bf16, fp32 accumulation, group scale applied per
 *   group), act = bf16(silu(g) * u) computed in fp32, fp32 down dot products; then
 *   y = y + w_j * d_j in fp32 (separately rounded products and sums), out = bf16(y).
 *   T > 1 (H and I multiples of 128): the reference's int4 prefill
 *   (fused_int4.py:247-260): each weight is dequantised to bf16((n - 8) * s), bit-exact
 *   with tmoe_dequant_int4_bf16, inside the grouped GEMM, and the result is the exact-BF16
 *   prefill of tmoe_experts_forward_bf16 on those dequantised weights.
 * tmoe_moe_block_int4 adds the router and the shared expert, which stays exact bf16
 * as in tmoe_moe_block_bf16: out = bf16(bf16(y) + bf16(gate * shared)).
 * Arguments otherwise as tmoe_experts_forward_bf16 / tmoe_moe_block_bf16.
 */
int tmoe_experts_forward_int4(const void* x, int T, const int64_t* ids, const void* weights,
                              const uint64_t* expert_table_q4, int H, int E, int I, int k, void* out,
                              void* workspace, size_t ws_bytes, void* stream);
int tmoe_moe_block_int4(const void* x, int T, const void* router_w, const float* logits_in,
                        const uint64_t* expert_table_q4, const void* sh_gate, const void* sh_up,
                        const void* sh_down, const void* sh_gate_w, int H, int E, int I, int k,
                        int Is, void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                        void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- the reference's int4 files
 * The int4 layout of the reference's own per-layer files (tarfa/engine/channel_q4.py:18,
 * 28-38; moe_kernel.py:10-14): the same packed nibbles, but ONE fp16 scale per weight row
 * (G = K), dequantised by the reference as fp16((nibble - 8) * s[n])
 * (channel_q4.py:10-14 dequant_int4).
 * tmoe_dequant_int4_f16: that dequantisation, bit for bit: fp16 scales [N, K/G], fp16 out
 *   [N, K], G = K for the reference's per-row layout (any even G dividing K accepted).
 *   packed 4-byte and out 16-byte aligned.
 * tmoe_experts_forward_int4_f16rows / tmoe_moe_block_int4_f16rows: the int4 entry points
 *   above with expert table uint64_t[E][4] = { gate_up packed [2I, H/2] u8, gate_up scales
 *   [2I] fp16, down packed [H, I/2] u8, down scales [H] fp16 } (16-byte aligned).
 *   T == 1: as the reference's moe_ffn (moe_kernel.py:90-104): per row, the fp32 sum of
 *   (nibble - 8) * x times fp32(s); act = bf16(silu(g) * u) in fp32; fp32 down rows; fp32
 *   router-order weighted sum; one bf16 cast.  T > 1: the exact-BF16 prefill on the weights
 *   bf16((nibble - 8) * fp32(s)), the exact product rounded once (the reference's own int4
 *   prefill multiplies in the model dtype, fused_int4.py:257-258).
 */
int tmoe_dequant_int4_f16(const void* packed, const void* scales, int N, int K, int G, void* out, void* stream);
int tmoe_experts_forward_int4_f16rows(const void* x, int T, const int64_t* ids, const void* weights,
                                      const uint64_t* expert_table_q4r, int H, int E, int I, int k, void* out,
                                      void* workspace, size_t ws_bytes, void* stream);
int tmoe_moe_block_int4_f16rows(const void* x, int T, const void* router_w, const float* logits_in,
                                const uint64_t* expert_table_q4r, const void* sh_gate, const void* sh_up,
                                const void* sh_down, const void* sh_gate_w, int H, int E, int I, int k, int Is,
                                void* out, int64_t* ids_out, void* weights_out, uint32_t* heat, void* workspace,
                                size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- the MoE sublayer
 * The steps on either side of the block in a Qwen3.5-MoE decoder layer
 * (transformers/models/qwen3_5_moe/modeling_qwen3_5_moe.py:870-875): h is the hidden
 * state before the post-attention RMSNorm (:801-818) and
 *   x   = bf16(h * (1 / sqrt(mean(h^2) + eps)) * (1 + ln_w))   (fp32 arithmetic)
 *   out = bf16(h + moe_block(x))
 * with moe_block exactly tmoe_moe_block_bf16 / _int4 on x.  ln_w [H] bf16 (the
 * zero-centred weight: the scale is 1 + ln_w); eps >= 0; out must not alias h.
 * Batch 1 on the fused decode kernel forms x in each of its tasks and adds h in its
 * combine (no extra launch); T > 1 normalises once (workspace) and adds h in the
 * prefill combine.  Arguments otherwise as tmoe_moe_block_bf16 / _int4.
 */
int tmoe_moe_layer_bf16(const void* h, int T, const void* ln_w, float eps, const void* router_w,
                        const float* logits_in, const uint64_t* expert_table, const void* sh_gate,
                        const void* sh_up, const void* sh_down, const void* sh_gate_w, int H, int E, int I,
                        int k, int Is, void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                        void* workspace, size_t ws_bytes, void* stream);
int tmoe_moe_layer_int4(const void* h, int T, const void* ln_w, float eps, const void* router_w,
                        const float* logits_in, const uint64_t* expert_table_q4, const void* sh_gate,
                        const void* sh_up, const void* sh_down, const void* sh_gate_w, int H, int E, int I,
                        int k, int Is, void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                        void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- allocation-free block
 * No counterpart in the reference.  For callers that cannot allocate device memory or
 * pass a workspace (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): tmoe_moe_block_bf16 with the workspace replaced by a static
 * device array inside the library, TMOE_STATIC_SCRATCH_BYTES per GPU, held by each GPU
 * the library runs on until the process ends.  Nothing is allocated by the call.
 *   - Calls needing a larger workspace than the static one (tmoe_workspace_bytes(T, ...)
 *     > TMOE_STATIC_SCRATCH_BYTES; at H=2560, E=256, I=Is=1024, k=8 that is T > 219)
 *     return TMOE_ERR_SCRATCH before any launch.
 *   - `status`: a caller-owned device uint32 (4-byte aligned, required) into which the
 *     kernels OR device-detected conditions: 1 = an expert id outside [0, E] (cannot come
 *     from the router itself), 2 = a bounded wait expired (results invalid).  The caller
 *     zeroes it and reads it at its own synchronisation points.
 *   - `stream` must belong to the current device (else TMOE_ERR_HIP); the scratch is that
 *     device's copy.
 *   - Every call on one GPU shares that GPU's scratch: calls that overlap in time on one
 *     GPU (other streams, other threads) race and must be ordered by the caller.
 * Arguments otherwise as tmoe_moe_block_bf16; results bit-identical to it.
 */
#define TMOE_STATIC_SCRATCH_BYTES (16u << 20)
int tmoe_moe_block_bf16_noalloc(const void* x, int T, const void* router_w, const float* logits_in,
                                const uint64_t* expert_table, const void* sh_gate, const void* sh_up,
                                const void* sh_down, const void* sh_gate_w, int H, int E, int I, int k, int Is,
                                void* out, int64_t* ids_out, void* weights_out, uint32_t* heat, uint32_t* status,
                                void* stream);

/* ---------------------------------------------------------------- route telemetry (a13)
 * The reference's per-layer route-reuse counters (tarfa/engine/fused_int4.py:71-95
 * _record_route / routing_telemetry), kept on the device so decode never synchronises
 * the host for telemetry.  `state` is a zero-filled device buffer of
 * tmoe_route_telemetry_bytes(L, k, E) bytes (8-byte aligned); one tmoe_route_record call
 * per token records ids [L, k] int64 (each layer's routing, e.g. the ids_out of its
 * tmoe_moe_block_* call).  Per layer: ids outside [0, E) are dropped (the sentinel E
 * included); a step without a valid id records nothing; otherwise steps += 1,
 * uses += number of valid ids, reuse_w += |set(ids) & union of the last w recorded
 * sets| for w = 1, 2, 4, 8, 16, distinct += newly seen experts.  The state begins with
 * uint64 counters[L][8] = {steps, uses, reuse_1, reuse_2, reuse_4, reuse_8, reuse_16,
 * distinct}.  Heat counters per (layer, expert) are the `heat` argument of the block
 * entry points.
 */
size_t tmoe_route_telemetry_bytes(int L, int k, int E);
int tmoe_route_record(const int64_t* ids, int L, int k, int E, void* state, size_t state_bytes,
                      void* stream);

/* ---------------------------------------------------------------- debug timeline
 * No counterpart in the reference (its decode is timed by wall clock around the whole call,
 * tarfa/engine/fused_int4.py:164, 203-204).  While set, every batch-1 call that runs the
 * fused decode kernel records, in the device buffer `buf` (8-byte aligned), the
 * s_memrealtime stamps (100 MHz) of each of its tasks: 16 header words {tasks, blocks,
 * router, shared up, shared down, gate/up per slot, down per slot, k, ...}, then per task
 * {start, routing known, loads returned, end, HW_ID, XCC_ID, ticket, 0}, then per wave
 * {entry, exit}, all uint64.  A launch whose records do not fit in `bytes` records nothing;
 * each launch overwrites the last.  buf = NULL turns it off.  Process-wide; for profiling,
 * not for concurrent use.
 */
int tmoe_debug_decode_trace(void* buf, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* TMOE_H */
