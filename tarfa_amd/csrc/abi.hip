// extern "C" entry points: argument validation, workspace carving, launches.
#include <stdlib.h>

#include <mutex>

#include "tmoe_device.h"
#include "tmoe_ws.h"
#include "tmoe_decode.h"

namespace tmoe {
int decode_launch(DecodeParams& p, bool run_router, hipStream_t s);
int decode_fused_launch(DecodeParams& p, bool run_router, hipStream_t s);
int launch_router_logits(const uint16_t* x, const uint16_t* wg, int T, int H, int E, float* logits, hipStream_t s);
int launch_router_topk(const float* logits, int T, int E, int k, int64_t* ids64, uint16_t* wb, int32_t* ids32,
                       float* wf, uint32_t* heat, hipStream_t s);
int prefill_launch(const uint16_t* x, int T, const int32_t* ids32, const int64_t* ids64, const float* wf,
                   const uint16_t* wb, const uint64_t* table, const uint16_t* sh_gate, const uint16_t* sh_up,
                   const uint16_t* sh_down, const float* gs, int H, int E, int I, int k, int Is, uint16_t* out,
                   void* ws, hipStream_t s, int q4, const uint16_t* resid, uint32_t* err);
int launch_router_topk_gate(const float* logits, int T, int E, int k, int64_t* ids64, uint16_t* wb, int32_t* ids32,
                            float* wf, uint32_t* heat, const uint16_t* x, const uint16_t* w_sg, int H, float* gs,
                            hipStream_t s);
int rmsnorm_launch(const uint16_t* h, const uint16_t* w, float eps, int T, int H, uint16_t* x, hipStream_t s);
int residual_add_launch(const uint16_t* h, uint16_t* y, size_t n, hipStream_t s);
bool sb_supported(int T, int H, int I, int Is, int k, int q4);
int sb_launch(const uint16_t* x, int T, const int32_t* ids32, const int64_t* ids64, const float* wf,
              const uint16_t* wb, const uint64_t* table, const uint16_t* sh_gate, const uint16_t* sh_up,
              const uint16_t* sh_down, const uint16_t* sh_gate_w, int H, int E, int I, int k, int Is,
              uint16_t* out, void* ws, hipStream_t s, const uint16_t* resid, uint32_t* err, int sh_pre);
int sb_router_launch(const uint16_t* x, const uint16_t* wg, int T, int H, int E, int I, int k, int Is,
                     const uint16_t* sh_gate, const uint16_t* sh_up, const uint16_t* sh_gate_w, int64_t* ids64,
                     uint16_t* wb, uint32_t* heat, void* ws, hipStream_t s, int* sh_pre);
}  // namespace tmoe


using namespace tmoe;

// Batch-1 path: the fused persistent kernel unless TMOE_DECODE_UNFUSED=1 (the
// three-launch path, kept for comparison) or the shape has no fused variant.
static int decode(DecodeParams& p, bool run_router, hipStream_t s) {
  static const bool unfused = [] {
    const char* v = getenv("TMOE_DECODE_UNFUSED");
    return v && v[0] == '1';
  }();
  if (!unfused) {
    const int st = decode_fused_launch(p, run_router, s);
    if (st != TMOE_ERR_SHAPE) return st;
  }
  return decode_launch(p, run_router, s);
}

// 2 <= T <= 16 (bf16 experts): the two-launch small-batch path unless TMOE_SMALLBATCH=0
// (the grouped-GEMM path, kept for comparison) or the shape has no small-batch variant.
static bool small_batch(int T, int H, int I, int Is, int k, int q4) {
  static const bool off = [] {
    const char* v = getenv("TMOE_SMALLBATCH");
    return v && v[0] == '0';
  }();
  return !off && sb_supported(T, H, I, Is, k, q4);
}

static bool misaligned(const void* p) { return ((uintptr_t)p & 15u) != 0; }

static int check_shape(int T, int H, int E, int I, int k, int Is) {
  // The bounds are the ones the fixed-size decode hand-off area is sized for.
  if (T < 1 || E < 1 || E > kMaxExperts || k < 1 || k > kMaxTopK || k > E) return TMOE_ERR_SHAPE;
  if (H < 8 || H > kMaxDim || H % 8) return TMOE_ERR_SHAPE;
  if (I < 8 || I > kMaxDim || I % 8) return TMOE_ERR_SHAPE;
  if (Is < 0 || Is > kMaxDim || Is % 8) return TMOE_ERR_SHAPE;
  return TMOE_OK;
}

extern "C" int tmoe_abi_version(void) { return TMOE_ABI_VERSION; }

extern "C" const char* tmoe_strerror(int status) {
  switch (status) {
    case TMOE_OK: return "ok";
    case TMOE_ERR_NULL: return "a required pointer is NULL";
    case TMOE_ERR_SHAPE: return "unsupported or inconsistent sizes";
    case TMOE_ERR_ALIGN: return "a pointer is not 16-byte aligned";
    case TMOE_ERR_WORKSPACE: return "workspace smaller than tmoe_workspace_bytes()";
    case TMOE_ERR_HIP: return "HIP runtime call or kernel launch failed";
    case TMOE_ERR_EXPERT_ID: return "expert id outside [0, num_experts] seen on the device";
    case TMOE_ERR_TIMEOUT: return "a bounded device-side dependency wait expired";
    case TMOE_ERR_SCRATCH: return "the call needs more scratch than the library's static scratch holds";
    default: return "unknown tmoe status";
  }
}

extern "C" size_t tmoe_workspace_bytes(int T, int H, int E, int I, int k, int Is) {
  if (check_shape(T, H, E, I, k, Is)) return 0;
  return ws_layout(T, H, E, I, k, Is).total;
}

extern "C" int tmoe_workspace_status(void* workspace, void* stream) {
  if (!workspace) return TMOE_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  uint32_t flags = 0;
  if (hipMemcpyAsync(&flags, workspace, sizeof(flags), hipMemcpyDeviceToHost, s) != hipSuccess) return TMOE_ERR_HIP;
  if (hipStreamSynchronize(s) != hipSuccess) return TMOE_ERR_HIP;
  if (!flags) return TMOE_OK;
  const uint32_t zero = 0;
  if (hipMemcpy(workspace, &zero, sizeof(zero), hipMemcpyHostToDevice) != hipSuccess) return TMOE_ERR_HIP;
  return (flags & kErrTimeout) ? TMOE_ERR_TIMEOUT : TMOE_ERR_EXPERT_ID;
}

static void bind_ws(DecodeParams& p, void* ws, const Ws& L) {
  p.status = ws_ptr<uint32_t>(ws, L.status);
  p.err = p.status + kStatusError;
  p.logits_ws = ws_ptr<float>(ws, L.logits);
  p.ids_ws = ws_ptr<int32_t>(ws, L.ids);
  p.w_ws = ws_ptr<float>(ws, L.wts);
  p.gs_ws = ws_ptr<float>(ws, L.gs);
  p.act_ws = ws_ptr<uint16_t>(ws, L.act);
  p.sact_ws = ws_ptr<uint16_t>(ws, L.act) + (size_t)p.k * p.I;
  p.sh_ws = ws_ptr<uint16_t>(ws, L.sh);
  p.sync = ws_ptr<uint32_t>(ws, L.sync);
  p.lg64 = ws_ptr<uint64_t>(ws, L.tagged);
  p.lg_stride = logit_stride(p.E);
  p.act64 = p.lg64 + (size_t)kLogitReplicas * p.lg_stride;
  p.dq64 = p.act64 + ((size_t)p.k * p.I + p.Is) / 2;
  p.handoff = ws_ptr<void>(ws, L.tagged);
  p.handoff_words = kHandoffWords;
}


// Int4 modes (q4 = 1: group-128 bf16 scales; q4 = 2: the reference's per-row fp16 scales):
// T == 1 needs H and I multiples of 512, T > 1 multiples of 128; table entries 16-byte aligned.
static int experts_forward(const void* x, int T, const int64_t* ids, const void* weights,
                           const uint64_t* expert_table, int H, int E, int I, int k, void* out, void* workspace,
                           size_t ws_bytes, hipStream_t s, int q4) {
  if (int st = check_shape(T, H, E, I, k, 0)) return st;
  if (!x || !ids || !weights || !expert_table || !out || !workspace) return TMOE_ERR_NULL;
  if (misaligned(x) || misaligned(workspace)) return TMOE_ERR_ALIGN;
  if (q4 && (T == 1 ? (H % 512 || I % 512) : (H % 128 || I % 128))) return TMOE_ERR_SHAPE;
  const Ws L = ws_layout(T, H, E, I, k, 0);
  if (ws_bytes < L.total) return TMOE_ERR_WORKSPACE;
  if (T == 1) {
    DecodeParams p{};
    p.x = (const uint16_t*)x;
    p.table = expert_table;
    p.q4 = q4;
    p.ids_in = ids;
    p.w_in = (const uint16_t*)weights;
    p.H = H; p.E = E; p.I = I; p.k = k; p.Is = 0;
    p.out = (uint16_t*)out;
    bind_ws(p, workspace, L);
    return q4 ? decode_fused_launch(p, false, s) : decode(p, false, s);
  }
  if (small_batch(T, H, I, 0, k, q4))
    return sb_launch((const uint16_t*)x, T, nullptr, ids, nullptr, (const uint16_t*)weights, expert_table, nullptr,
                     nullptr, nullptr, nullptr, H, E, I, k, 0, (uint16_t*)out, workspace, s, nullptr, nullptr, 0);
  return prefill_launch((const uint16_t*)x, T, nullptr, ids, nullptr, (const uint16_t*)weights, expert_table,
                        nullptr, nullptr, nullptr, nullptr, H, E, I, k, 0, (uint16_t*)out, workspace, s, q4, nullptr,
                        nullptr);
}

extern "C" int tmoe_experts_forward_bf16(const void* x, int T, const int64_t* ids, const void* weights,
                                         const uint64_t* expert_table, int H, int E, int I, int k, void* out,
                                         void* workspace, size_t ws_bytes, void* stream) {
  return experts_forward(x, T, ids, weights, expert_table, H, E, I, k, out, workspace, ws_bytes, (hipStream_t)stream,
                         0);
}

extern "C" int tmoe_experts_forward_int4(const void* x, int T, const int64_t* ids, const void* weights,
                                         const uint64_t* expert_table_q4, int H, int E, int I, int k, void* out,
                                         void* workspace, size_t ws_bytes, void* stream) {
  return experts_forward(x, T, ids, weights, expert_table_q4, H, E, I, k, out, workspace, ws_bytes,
                         (hipStream_t)stream, 1);
}

extern "C" int tmoe_experts_forward_int4_f16rows(const void* x, int T, const int64_t* ids, const void* weights,
                                                 const uint64_t* expert_table_q4r, int H, int E, int I, int k,
                                                 void* out, void* workspace, size_t ws_bytes, void* stream) {
  return experts_forward(x, T, ids, weights, expert_table_q4r, H, E, I, k, out, workspace, ws_bytes,
                         (hipStream_t)stream, 2);
}

// ln_w non-null: x is the hidden state h before the layer's RMSNorm; the block runs on
// bf16(rmsnorm(h) * (1 + ln_w)) and out = bf16(h + block output).
static int moe_block(const void* x, int T, const void* router_w, const float* logits_in, const uint64_t* expert_table,
                     const void* sh_gate, const void* sh_up, const void* sh_down, const void* sh_gate_w, int H, int E,
                     int I, int k, int Is, void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                     void* workspace, size_t ws_bytes, hipStream_t s, int q4, const void* ln_w = nullptr,
                     float ln_eps = 0.f, uint32_t* err = nullptr) {
  const bool has_sh = sh_gate || sh_up || sh_down || sh_gate_w;
  if (has_sh && (!sh_gate || !sh_up || !sh_down || !sh_gate_w || Is < 8)) return TMOE_ERR_NULL;
  if (!has_sh) Is = 0;
  if (int st = check_shape(T, H, E, I, k, Is)) return st;
  if (!x || !expert_table || !out || !workspace || (!router_w && !logits_in)) return TMOE_ERR_NULL;
  if (ln_w && (misaligned(ln_w) || misaligned(out))) return TMOE_ERR_ALIGN;
  if (ln_w && (out == x || !(ln_eps >= 0.f))) return TMOE_ERR_SHAPE;
  if (misaligned(x) || misaligned(workspace) || (router_w && misaligned(router_w)) ||
      (has_sh && (misaligned(sh_gate) || misaligned(sh_up) || misaligned(sh_down) || misaligned(sh_gate_w))))
    return TMOE_ERR_ALIGN;
  if (q4 && ((T == 1 ? (H % 512 || I % 512) : (H % 128 || I % 128)) || (Is && Is != I))) return TMOE_ERR_SHAPE;
  const Ws L = ws_layout(T, H, E, I, k, Is);
  if (ws_bytes < L.total) return TMOE_ERR_WORKSPACE;
  if (T == 1) {
    DecodeParams p{};
    p.x = (const uint16_t*)x;
    p.router_w = logits_in ? nullptr : (const uint16_t*)router_w;
    p.logits_in = logits_in;
    p.table = expert_table;
    p.q4 = q4;
    p.sh_gate = (const uint16_t*)sh_gate;
    p.sh_up = (const uint16_t*)sh_up;
    p.sh_down = (const uint16_t*)sh_down;
    p.sh_gate_w = (const uint16_t*)sh_gate_w;
    p.H = H; p.E = E; p.I = I; p.k = k; p.Is = Is;
    p.out = (uint16_t*)out;
    p.ids_out = ids_out;
    p.w_out = (uint16_t*)weights_out;
    p.heat = heat;
    bind_ws(p, workspace, L);
    if (err) p.err = err;
    if (!ln_w) return q4 ? decode_fused_launch(p, true, s) : decode(p, true, s);
    // The fused kernel forms the normalised input in every task and adds the residual in
    // its combine; other shapes normalise first and add the residual after.
    p.ln_w = (const uint16_t*)ln_w;
    p.ln_eps = ln_eps;
    p.resid = (const uint16_t*)x;
    const int st = decode_fused_launch(p, true, s);
    if (st != TMOE_ERR_SHAPE || q4) return st;
    uint16_t* xn = ws_ptr<uint16_t>(workspace, L.xn);
    if (int st2 = rmsnorm_launch((const uint16_t*)x, (const uint16_t*)ln_w, ln_eps, 1, H, xn, s)) return st2;
    p.x = xn;
    p.ln_w = nullptr;
    p.resid = nullptr;
    if (int st2 = decode(p, true, s)) return st2;
    return residual_add_launch((const uint16_t*)x, (uint16_t*)out, (size_t)H, s);
  }
  // T > 1: router, shared gate, then the prefill experts path with the shared expert as an extra group.
  const void* h = x;
  if (ln_w) {
    uint16_t* xn = ws_ptr<uint16_t>(workspace, L.xn);
    if (int st = rmsnorm_launch((const uint16_t*)h, (const uint16_t*)ln_w, ln_eps, T, H, xn, s)) return st;
    x = xn;
  }
  float* logits = ws_ptr<float>(workspace, L.logits);
  int32_t* ids32 = ws_ptr<int32_t>(workspace, L.ids);
  float* wf = ws_ptr<float>(workspace, L.wts);
  float* gs = ws_ptr<float>(workspace, L.gs);
  if (small_batch(T, H, I, Is, k, q4)) {
    // Router (logits and top-k in one launch, with the shared expert's gate/up beside it), then
    // the small-batch experts; the shared gate is computed inside.
    int sh_pre = 0;
    if (logits_in) {
      if (int st = launch_router_topk(logits_in, T, E, k, ids_out, (uint16_t*)weights_out, ids32, wf, heat, s))
        return st;
    } else if (int st = sb_router_launch((const uint16_t*)x, (const uint16_t*)router_w, T, H, E, I, k, Is,
                                         (const uint16_t*)sh_gate, (const uint16_t*)sh_up, (const uint16_t*)sh_gate_w,
                                         ids_out, (uint16_t*)weights_out, heat, workspace, s, &sh_pre)) {
      return st;
    }
    return sb_launch((const uint16_t*)x, T, ids32, nullptr, wf, nullptr, expert_table, (const uint16_t*)sh_gate,
                     (const uint16_t*)sh_up, (const uint16_t*)sh_down, (const uint16_t*)sh_gate_w, H, E, I, k, Is,
                     (uint16_t*)out, workspace, s, ln_w ? (const uint16_t*)h : nullptr, err, sh_pre);
  }
  const float* lg = logits_in;
  if (!lg) {
    if (int st = launch_router_logits((const uint16_t*)x, (const uint16_t*)router_w, T, H, E, logits, s)) return st;
    lg = logits;
  }
  // Top-k and, with a shared expert, its gate in the same launch.
  if (has_sh) {
    if (int st = launch_router_topk_gate(lg, T, E, k, ids_out, (uint16_t*)weights_out, ids32, wf, heat,
                                         (const uint16_t*)x, (const uint16_t*)sh_gate_w, H, gs, s))
      return st;
  } else if (int st = launch_router_topk(lg, T, E, k, ids_out, (uint16_t*)weights_out, ids32, wf, heat, s)) {
    return st;
  }
  return prefill_launch((const uint16_t*)x, T, ids32, nullptr, wf, nullptr, expert_table, (const uint16_t*)sh_gate,
                        (const uint16_t*)sh_up, (const uint16_t*)sh_down, has_sh ? gs : nullptr, H, E, I, k, Is,
                        (uint16_t*)out, workspace, s, q4, ln_w ? (const uint16_t*)h : nullptr, err);
}

extern "C" int tmoe_moe_block_bf16(const void* x, int T, const void* router_w, const float* logits_in,
                                   const uint64_t* expert_table, const void* sh_gate, const void* sh_up,
                                   const void* sh_down, const void* sh_gate_w, int H, int E, int I, int k, int Is,
                                   void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                                   void* workspace, size_t ws_bytes, void* stream) {
  return moe_block(x, T, router_w, logits_in, expert_table, sh_gate, sh_up, sh_down, sh_gate_w, H, E, I, k, Is, out,
                   ids_out, weights_out, heat, workspace, ws_bytes, (hipStream_t)stream, 0);
}

extern "C" int tmoe_moe_block_int4(const void* x, int T, const void* router_w, const float* logits_in,
                                   const uint64_t* expert_table_q4, const void* sh_gate, const void* sh_up,
                                   const void* sh_down, const void* sh_gate_w, int H, int E, int I, int k, int Is,
                                   void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                                   void* workspace, size_t ws_bytes, void* stream) {
  return moe_block(x, T, router_w, logits_in, expert_table_q4, sh_gate, sh_up, sh_down, sh_gate_w, H, E, I, k, Is,
                   out, ids_out, weights_out, heat, workspace, ws_bytes, (hipStream_t)stream, 1);
}

extern "C" int tmoe_moe_block_int4_f16rows(const void* x, int T, const void* router_w, const float* logits_in,
                                           const uint64_t* expert_table_q4r, const void* sh_gate, const void* sh_up,
                                           const void* sh_down, const void* sh_gate_w, int H, int E, int I, int k,
                                           int Is, void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                                           void* workspace, size_t ws_bytes, void* stream) {
  return moe_block(x, T, router_w, logits_in, expert_table_q4r, sh_gate, sh_up, sh_down, sh_gate_w, H, E, I, k, Is,
                   out, ids_out, weights_out, heat, workspace, ws_bytes, (hipStream_t)stream, 2);
}

// The MoE sublayer of a decoder layer: out = bf16(h + block(bf16(rmsnorm(h) * (1 + ln_w)))).
extern "C" int tmoe_moe_layer_bf16(const void* h, int T, const void* ln_w, float eps, const void* router_w,
                                   const float* logits_in, const uint64_t* expert_table, const void* sh_gate,
                                   const void* sh_up, const void* sh_down, const void* sh_gate_w, int H, int E, int I,
                                   int k, int Is, void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                                   void* workspace, size_t ws_bytes, void* stream) {
  if (!ln_w) return TMOE_ERR_NULL;
  return moe_block(h, T, router_w, logits_in, expert_table, sh_gate, sh_up, sh_down, sh_gate_w, H, E, I, k, Is, out,
                   ids_out, weights_out, heat, workspace, ws_bytes, (hipStream_t)stream, 0, ln_w, eps);
}

extern "C" int tmoe_moe_layer_int4(const void* h, int T, const void* ln_w, float eps, const void* router_w,
                                   const float* logits_in, const uint64_t* expert_table_q4, const void* sh_gate,
                                   const void* sh_up, const void* sh_down, const void* sh_gate_w, int H, int E, int I,
                                   int k, int Is, void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                                   void* workspace, size_t ws_bytes, void* stream) {
  if (!ln_w) return TMOE_ERR_NULL;
  return moe_block(h, T, router_w, logits_in, expert_table_q4, sh_gate, sh_up, sh_down, sh_gate_w, H, E, I, k, Is,
                   out, ids_out, weights_out, heat, workspace, ws_bytes, (hipStream_t)stream, 1, ln_w, eps);
}

// ---------------------------------------------------------------- allocation-free block
// The workspace of tmoe_moe_block_bf16_noalloc is this file-scope device array; each GPU
// holds its own copy (at its own address) for the life of the process.  Host code never
// names it as memory: the first call on a device, with that device current, looks up
// that device's copy with hipGetSymbolAddress and keeps the pointer, and only that
// pointer reaches the kernels.  The array is zero when the code object loads, and every
// call leaves what the next one needs at zero (sync counters) or harmless (tagged
// hand-off words carry the epoch of the call that wrote them), as with a caller's
// workspace; the T-dependent regions are written before they are read within a call.
static __device__ __align__(256) unsigned char scratch[TMOE_STATIC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};
}  // namespace

// This device's copy of the scratch array, or nullptr if the lookup fails.
static void* device_scratch(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch[dev] = ptr;
  }
  return g_scratch[dev];
}

extern "C" int tmoe_moe_block_bf16_noalloc(const void* x, int T, const void* router_w, const float* logits_in,
                                           const uint64_t* expert_table, const void* sh_gate, const void* sh_up,
                                           const void* sh_down, const void* sh_gate_w, int H, int E, int I, int k,
                                           int Is, void* out, int64_t* ids_out, void* weights_out, uint32_t* heat,
                                           uint32_t* status, void* stream) {
  if (!status) return TMOE_ERR_NULL;
  if ((uintptr_t)status & 3u) return TMOE_ERR_ALIGN;
  const int has_sh = sh_gate || sh_up || sh_down || sh_gate_w;
  if (int st = check_shape(T, H, E, I, k, has_sh ? Is : 0)) return st;
  if (ws_layout(T, H, E, I, k, has_sh ? Is : 0).total > (size_t)TMOE_STATIC_SCRATCH_BYTES) return TMOE_ERR_SCRATCH;
  hipStream_t s = (hipStream_t)stream;
  int dev = -1, sdev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TMOE_ERR_HIP;
  if (s && (hipStreamGetDevice(s, &sdev) != hipSuccess || sdev != dev)) return TMOE_ERR_HIP;
  void* ws = device_scratch(dev);
  if (!ws) return TMOE_ERR_HIP;
  return moe_block(x, T, router_w, logits_in, expert_table, sh_gate, sh_up, sh_down, sh_gate_w, H, E, I, k, Is, out,
                   ids_out, weights_out, heat, ws, (size_t)TMOE_STATIC_SCRATCH_BYTES, s, 0, nullptr, 0.f, status);
}
