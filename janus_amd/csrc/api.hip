// Pipelines behind the experts and block entry points, workspace layouts, and the error channel.
//
// experts (fused_moe, janus/moe_w4a16.py:122-140):   align -> gate_up -> down (weighted slots) -> combine
// block   (Qwen3_5MoeSparseMoeBlock.forward):        route -> align -> gate_up (+ shared) -> down (+ shared, combine)
//                                                     -> combine (fp32 slot sum, one rounding)
// Every launch goes on the caller's stream; counts stay on the device (grids are sized for the worst case and idle
// workgroups exit), so a caller can capture the whole sequence in a HIP graph.
#include <stdarg.h>

#include <atomic>

#include "align.h"
#include "gemm.h"
#include "norm.h"
#include "router.h"

namespace janus {

namespace {
thread_local char g_error[512] = "";
constexpr int kStageEvents = 6;
thread_local hipEvent_t g_events[kStageEvents] = {};
thread_local int g_nevents = 0;

// Stage boundaries of the pipelines: 0 start (before route), 1 before align, 2 before gate_up, 3 before down,
// 4 before the combine, 5 end.
void mark(int i, hipStream_t stream) {
  if (i < g_nevents && g_events[i]) (void)hipEventRecord(g_events[i], stream);
}
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

// One status word per device: every GPU the library runs on holds its own copy of this variable, at its own address.
__device__ int g_status_word;

int* device_status_word() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int*> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  int* p = cache[dev].load(std::memory_order_acquire);
  if (!p) {
    if (hipGetSymbolAddress(reinterpret_cast<void**>(&p), HIP_SYMBOL(g_status_word)) != hipSuccess) return nullptr;
    cache[dev].store(p, std::memory_order_release);
  }
  return p;
}

namespace {
__global__ void read_status_kernel(int* __restrict__ status, int32_t* __restrict__ out, int clear) {
  out[0] = *status;
  if (clear) *status = 0;
}
}  // namespace

namespace {

struct ExpertsWorkspace {
  AlignWorkspace align;
  int* sorted_ids;  // [P] permuted assignment ids, sentinel A
  int4* chunks;     // [C]
  int* num_chunks;  // [1]
  uint16_t* h;      // [P, I]
  uint16_t* h_sh;   // [T, I_s]
  int16_t* slots;    // [T, nslots, H] weighted expert outputs: int16 codes (slot format of gemm.h)
  float* slot_scale;  // [T, nslots, H / kSlotBlock] their block scales
  int* sched;       // [nsched] counters of the persistent GEMM launch, cleared by align
  int P, C, nslots, nsched;
  int chunk_rows;  // chunk_rows_for the call
};

// plan_block > 0: the permuted rows follow a caller's tile plan padded to that block (align() at that block size).
ExpertsWorkspace carve_experts(Carver& c, int T, int top_k, int E, int H, int I, int I_s, int plan_block = 0) {
  ExpertsWorkspace w;
  const int A = T * top_k;
  w.P = plan_block > 0 ? ceil_div(A + E * (plan_block - 1), plan_block) * plan_block : A + E * (kRowPad - 1);
  w.chunk_rows = chunk_rows_for(A, E);
  w.C = ceil_div(A, w.chunk_rows) + E;
  w.align = carve_align(c, A, E);
  w.sorted_ids = c.take<int>(w.P);
  w.chunks = c.take<int4>(w.C);
  w.num_chunks = c.take<int>(1);
  w.nsched = sched_words(w.C, I_s > 0 ? ceil_div(T, w.chunk_rows) : 0);
  w.sched = c.take<int>(w.nsched);
  w.h = c.take<uint16_t>((size_t)w.P * I);
  w.h_sh = c.take<uint16_t>((size_t)T * I_s);
  w.nslots = top_k + (I_s > 0 ? 1 : 0);
  w.slots = c.take<int16_t>((size_t)T * w.nslots * H);
  w.slot_scale = c.take<float>((size_t)T * w.nslots * (H / kSlotBlock));
  return w;
}

int check_expert_sizes(const char* who, int T, int H, int I, int E, int top_k, int I_s = 0) {
  JANUS_REQUIRE(T >= 0 && H > 0 && H % 128 == 0 && I > 0 && I % 128 == 0 && E > 0 && E <= kMaxExperts && top_k > 0 &&
                    top_k <= E && (long)T * top_k < (1l << 30),
                JANUS_MOE_EINVAL,
                "%s: unsupported sizes T=%d H=%d I=%d E=%d top_k=%d (need H %% 128 == 0, I %% 128 == 0, E <= %d, "
                "top_k <= E)", who, T, H, I, E, top_k, kMaxExperts);
  // The GEMMs address activation rows with 32-bit byte offsets from the buffer base: x rows (T x H bf16), the routed
  // h rows (P = T*top_k + E*(kRowPad-1) padded rows x I) and the shared-expert h rows (T x I_s).
  const long P = (long)T * top_k + (long)E * (kRowPad - 1);
  JANUS_REQUIRE((long)T * H * 2 < (1l << 31) && P * I * 2 < (1l << 31) && (long)T * I_s * 2 < (1l << 31),
                JANUS_MOE_EINVAL,
                "%s: T=%d H=%d I=%d I_s=%d E=%d top_k=%d: an activation buffer (T*H, (T*top_k + 15*E)*I or T*I_s bf16 "
                "values) reaches 2 GiB", who, T, H, I, I_s, E, top_k);
  return JANUS_MOE_OK;
}

// The serving epilogue of run_experts: instead of writing the MoE output, add it to the residual x_res in place and
// write the next layer's normed input n_out (0 where valid[t] == 0).
struct ServeEpilogue {
  uint16_t* x_res;
  const uint16_t* norm_w;
  float eps;
  const uint8_t* valid;
  uint16_t* n_out;
};

// Runs align + the two grouped GEMMs + the combine; routing (idx, weights) already on the device.
template <typename IdxT>
int run_experts(const uint16_t* x, const IdxT* idx, const float* route_w, const int32_t* guq, const uint16_t* gus,
                const int32_t* dq, const uint16_t* ds, const int32_t* sguq, const uint16_t* sgus, const int32_t* sdq,
                const uint16_t* sds, const float* gamma, int T, int H, int I, int I_s, int E, int top_k, uint16_t* out,
                const ExpertsWorkspace& w, hipStream_t stream, int codec = 0, const float* gu_global = nullptr,
                const float* dn_global = nullptr, const uint8_t* valid = nullptr,
                const ServeEpilogue* serve = nullptr, const int64_t* check_ids = nullptr,
                const float* sgu_global = nullptr, const float* sdn_global = nullptr,
                const int64_t* plan_sorted_ids = nullptr, const int64_t* plan_expert_ids = nullptr,
                int plan_block = 0) {
  const int A = T * top_k;
  int* status = device_status_word();
  JANUS_REQUIRE(status, JANUS_MOE_ELAUNCH, "the device status word of this library could not be resolved");
  mark(1, stream);
  // check_ids: the caller's own top-k ids (the experts entries). An id outside [0, E) is dropped by align, reported in
  // the status word, and its slot skipped by the combine. The block path routes padding tokens to id E on purpose.
  int rc = plan_sorted_ids
               ? launch_plan_chunks(plan_sorted_ids, plan_expert_ids, w.P / plan_block, plan_block, A, E, w.sorted_ids,
                                    w.chunks, w.C, w.chunk_rows, w.num_chunks, w.sched, w.nsched, stream)
               : launch_align<IdxT, int>(idx, A, E, kRowPad, w.align, w.sorted_ids, w.P, nullptr, 0, nullptr, w.chunks,
                                         w.chunk_rows, w.num_chunks, w.sched, w.nsched, check_ids ? status : nullptr,
                                         stream);
  if (rc) return rc;
  const bool shared = I_s > 0;
  GemmParams p = {};
  p.sorted_ids = w.sorted_ids;
  p.topk = top_k;
  p.A = A;
  p.T = T;
  p.chunks = w.chunks;
  p.num_chunks = w.num_chunks;
  p.codec = codec;
  p.max_chunks = w.C;
  p.n_shared_chunks = shared ? ceil_div(T, w.chunk_rows) : 0;
  p.chunk_rows = w.chunk_rows;
  // gate_up
  p.a = x;
  p.a_bytes = (uint32_t)((size_t)T * H * 2);
  p.q = guq;
  p.s = gus;
  p.gsc = gu_global;
  p.N = 2 * I;
  p.K = H;
  p.q_sh = sguq;
  p.s_sh = sgus;
  p.gsc_sh = sgu_global;
  p.N_sh = 2 * I_s;
  p.K_sh = H;
  p.nslab = ceil_div(I > I_s ? I : I_s, 128);
  p.h = w.h;
  p.h_sh = w.h_sh;
  // down: weighted expert outputs into the slots
  GemmParams d = p;
  d.a = w.h;
  d.a_sh = w.h_sh;
  d.a_bytes = (uint32_t)((size_t)w.P * I * 2);
  d.a_sh_bytes = (uint32_t)((size_t)T * I_s * 2);
  d.q = dq;
  d.s = ds;
  d.gsc = dn_global;
  d.N = H;
  d.K = I;
  d.q_sh = sdq;
  d.s_sh = sds;
  d.gsc_sh = sdn_global;
  d.N_sh = H;
  d.K_sh = I_s;
  d.nslab = ceil_div(H, 256);
  d.slots = w.slots;
  d.slot_scale = w.slot_scale;
  d.nslots = w.nslots;
  d.route_w = route_w;
  d.gamma = gamma;
  mark(2, stream);
  rc = launch_experts_fused(p, d, w.sched, status, stream);  // both GEMMs, one persistent launch
  if (rc == kNotFused) {
    rc = launch_gate_up(p, stream);
    if (rc) return rc;
    mark(3, stream);
    rc = launch_down(d, stream);
  } else {
    mark(3, stream);
  }
  if (rc) return rc;
  mark(4, stream);
  if (serve)  // the combine folded into the next residual add + norm; `out` is not written
    rc = launch_combine_add_rmsnorm(w.slots, w.slot_scale, w.nslots, valid, serve->x_res, serve->norm_w, serve->eps,
                                    serve->valid, T, H, serve->n_out, stream);
  else
    rc = launch_combine(w.slots, w.slot_scale, w.nslots, out, T, H, valid, check_ids, top_k, E, stream);
  mark(5, stream);
  return rc;
}

struct BlockWorkspace {
  RouteWorkspace route;
  int32_t* topk_idx;
  float* topk_w;
  float* gamma;
  ExpertsWorkspace experts;
};

BlockWorkspace carve_block(Carver& c, int T, int H, int I, int E, int top_k, int I_s) {
  BlockWorkspace b;
  b.route = carve_route(c, T, H, E);
  b.topk_idx = c.take<int32_t>((size_t)T * top_k);
  b.topk_w = c.take<float>((size_t)T * top_k);
  b.gamma = c.take<float>(T);
  b.experts = carve_experts(c, T, top_k, E, H, I, I_s);
  return b;
}

}  // namespace
}  // namespace janus

using namespace janus;

extern "C" const char* janus_moe_last_error(void) { return g_error; }
extern "C" int janus_moe_abi_version(void) { return 1; }

extern "C" int janus_moe_profile_events(void* const* events, int count) {
  JANUS_REQUIRE(count >= 0 && count <= kStageEvents && (count == 0 || events), JANUS_MOE_EINVAL,
                "janus_moe_profile_events: count=%d (at most %d)", count, kStageEvents);
  for (int i = 0; i < kStageEvents; ++i) g_events[i] = i < count ? static_cast<hipEvent_t>(events[i]) : nullptr;
  g_nevents = count;
  return JANUS_MOE_OK;
}

extern "C" int janus_moe_device_status(int32_t* out, int clear, janus_stream_t stream) {
  JANUS_REQUIRE(out, JANUS_MOE_EINVAL, "janus_moe_device_status: null pointer");
  int* status = device_status_word();
  JANUS_REQUIRE(status, JANUS_MOE_ELAUNCH, "janus_moe_device_status: the device status word could not be resolved");
  hipLaunchKernelGGL(read_status_kernel, dim3(1), dim3(1), 0, (hipStream_t)stream, status, out, clear);
  JANUS_LAUNCH_CHECK("janus_moe_device_status");
  return JANUS_MOE_OK;
}

extern "C" size_t janus_moe_experts_workspace_bytes(int S, int top_k, int E, int H, int I) {
  if (S < 0 || top_k <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
  Carver c(nullptr);
  carve_experts(c, S, top_k, E, H, I, 0);
  return align_up(c.used, 256);
}

extern "C" int janus_moe_experts(const uint16_t* x, const int64_t* top_k_index, const float* top_k_weights,
                                 const int32_t* gate_up_q, const uint16_t* gate_up_s, const int32_t* down_q,
                                 const uint16_t* down_s, int S, int H, int I, int E, int top_k, uint16_t* out, void* ws,
                                 size_t ws_bytes, janus_stream_t stream) {
  int rc = check_expert_sizes("janus_moe_experts", S, H, I, E, top_k);
  if (rc) return rc;
  if (S == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(x && top_k_index && top_k_weights && gate_up_q && gate_up_s && down_q && down_s && out,
                JANUS_MOE_EINVAL, "janus_moe_experts: null pointer");
  const size_t need = janus_moe_experts_workspace_bytes(S, top_k, E, H, I);
  JANUS_REQUIRE(ws && ws_bytes >= need, JANUS_MOE_EWORKSPACE, "janus_moe_experts: workspace %zu < %zu bytes", ws_bytes,
                need);
  Carver c(ws);
  ExpertsWorkspace w = carve_experts(c, S, top_k, E, H, I, 0);
  mark(0, (hipStream_t)stream);
  return run_experts<int64_t>(x, top_k_index, top_k_weights, gate_up_q, gate_up_s, down_q, down_s, nullptr, nullptr,
                              nullptr, nullptr, nullptr, S, H, I, 0, E, top_k, out, w, (hipStream_t)stream, 0, nullptr,
                              nullptr, nullptr, nullptr, top_k_index);
}

extern "C" int janus_moe_experts_nvfp4(const uint16_t* x, const int64_t* top_k_index, const float* top_k_weights,
                                       const uint8_t* gate_up, const uint8_t* gate_up_scale, const float* gate_up_global,
                                       const uint8_t* down, const uint8_t* down_scale, const float* down_global, int S,
                                       int H, int I, int E, int top_k, uint16_t* out, void* ws, size_t ws_bytes,
                                       janus_stream_t stream) {
  int rc = check_expert_sizes("janus_moe_experts_nvfp4", S, H, I, E, top_k);
  if (rc) return rc;
  if (S == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(x && top_k_index && top_k_weights && gate_up && gate_up_scale && gate_up_global && down &&
                    down_scale && down_global && out,
                JANUS_MOE_EINVAL, "janus_moe_experts_nvfp4: null pointer");
  const size_t need = janus_moe_experts_workspace_bytes(S, top_k, E, H, I);
  JANUS_REQUIRE(ws && ws_bytes >= need, JANUS_MOE_EWORKSPACE, "janus_moe_experts_nvfp4: workspace %zu < %zu bytes",
                ws_bytes, need);
  Carver c(ws);
  ExpertsWorkspace w = carve_experts(c, S, top_k, E, H, I, 0);
  mark(0, (hipStream_t)stream);
  return run_experts<int64_t>(x, top_k_index, top_k_weights, reinterpret_cast<const int32_t*>(gate_up),
                              reinterpret_cast<const uint16_t*>(gate_up_scale),
                              reinterpret_cast<const int32_t*>(down), reinterpret_cast<const uint16_t*>(down_scale),
                              nullptr, nullptr, nullptr, nullptr, nullptr, S, H, I, 0, E, top_k, out, w,
                              (hipStream_t)stream, /*codec=*/1, gate_up_global, down_global, nullptr, nullptr,
                              top_k_index);
}

extern "C" size_t janus_moe_experts_planned_workspace_bytes(int S, int top_k, int E, int H, int I, int block) {
  if (S < 0 || top_k <= 0 || E <= 0 || H <= 0 || I <= 0 || block <= 0) return 0;
  Carver c(nullptr);
  carve_experts(c, S, top_k, E, H, I, 0, block);
  return align_up(c.used, 256);
}

extern "C" int janus_moe_experts_planned(int codec, const uint16_t* x, const int64_t* top_k_index,
                                         const float* top_k_weights, const void* gate_up, const void* gate_up_scale,
                                         const float* gate_up_global, const void* down, const void* down_scale,
                                         const float* down_global, const int64_t* plan_sorted_ids,
                                         const int64_t* plan_expert_ids, int block, int S, int H, int I, int E,
                                         int top_k, uint16_t* out, void* ws, size_t ws_bytes, janus_stream_t stream) {
  int rc = check_expert_sizes("janus_moe_experts_planned", S, H, I, E, top_k);
  if (rc) return rc;
  JANUS_REQUIRE(codec == 0 || codec == 1, JANUS_MOE_EINVAL, "janus_moe_experts_planned: codec %d (0 int4, 1 NVFP4)",
                codec);
  JANUS_REQUIRE(block > 0 && block <= 1024, JANUS_MOE_EINVAL, "janus_moe_experts_planned: block=%d", block);
  const long tiles = ((long)S * top_k + (long)E * (block - 1) + block - 1) / block;
  JANUS_REQUIRE(tiles * block * (long)I * 2 < (1l << 31), JANUS_MOE_EINVAL,
                "janus_moe_experts_planned: the plan's rows (%ld x I=%d bf16) reach 2 GiB", tiles * block, I);
  if (S == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(x && top_k_index && top_k_weights && gate_up && gate_up_scale && down && down_scale && out &&
                    plan_sorted_ids && plan_expert_ids && (codec == 0 || (gate_up_global && down_global)),
                JANUS_MOE_EINVAL, "janus_moe_experts_planned: null pointer");
  const size_t need = janus_moe_experts_planned_workspace_bytes(S, top_k, E, H, I, block);
  JANUS_REQUIRE(ws && ws_bytes >= need, JANUS_MOE_EWORKSPACE, "janus_moe_experts_planned: workspace %zu < %zu bytes",
                ws_bytes, need);
  Carver c(ws);
  ExpertsWorkspace w = carve_experts(c, S, top_k, E, H, I, 0, block);
  mark(0, (hipStream_t)stream);
  return run_experts<int64_t>(x, top_k_index, top_k_weights, static_cast<const int32_t*>(gate_up),
                              static_cast<const uint16_t*>(gate_up_scale), static_cast<const int32_t*>(down),
                              static_cast<const uint16_t*>(down_scale), nullptr, nullptr, nullptr, nullptr, nullptr,
                              S, H, I, 0, E, top_k, out, w, (hipStream_t)stream, codec, gate_up_global, down_global,
                              nullptr, nullptr, top_k_index, nullptr, nullptr, plan_sorted_ids, plan_expert_ids, block);
}

extern "C" int janus_moe_dequant_nvfp4(const uint8_t* packed, const uint8_t* scale, const float* global, long rows,
                                       int K, uint16_t* out, janus_stream_t stream) {
  JANUS_REQUIRE(rows >= 0 && K > 0 && K % 16 == 0, JANUS_MOE_EINVAL,
                "janus_moe_dequant_nvfp4: rows=%ld K=%d (need K %% 16 == 0)", rows, K);
  if (rows == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(packed && scale && global && out, JANUS_MOE_EINVAL, "janus_moe_dequant_nvfp4: null pointer");
  return launch_dequant_nvfp4(packed, scale, global, rows, K, out, (hipStream_t)stream);
}

extern "C" size_t janus_moe_block_workspace_bytes(int T, int H, int I, int E, int top_k, int I_s) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || top_k <= 0 || I_s < 0) return 0;
  Carver c(nullptr);
  carve_block(c, T, H, I, E, top_k, I_s);
  return align_up(c.used, 256);
}

extern "C" int janus_moe_block_forward(const janus_moe_block_weights* wt, const uint16_t* x, int T, uint16_t* out,
                                       int32_t* topk_idx, float* topk_w, void* ws, size_t ws_bytes,
                                       janus_stream_t stream) {
  return janus_moe_block_forward_masked(wt, x, nullptr, T, out, topk_idx, topk_w, ws, ws_bytes, stream);
}

namespace {
// Either codec's block weights, as the pipeline reads them: weight and scale pointers untyped (int4 words and bf16
// scales, or NVFP4 bytes and e4m3 scales), plus the NVFP4 global scales per weight row (null for int4).
struct BlockView {
  int H, I, E, top_k, I_s, codec;
  const float* router_w;
  const void* router_prep;
  const float* router_bias;
  const void *gate_up, *gate_up_scale, *down, *down_scale;
  const float *gate_up_global, *down_global;
  const void *sh_gate_up, *sh_gate_up_scale, *sh_down, *sh_down_scale;
  const float *sh_gate_up_global, *sh_down_global;
  const uint16_t* sh_gate_w;
};

BlockView view_of(const janus_moe_block_weights* w) {
  return BlockView{w->H, w->I, w->E, w->top_k, w->I_s, 0, w->router_w, w->router_prep, w->router_bias,
                   w->gate_up_q, w->gate_up_s, w->down_q, w->down_s, nullptr, nullptr,
                   w->sh_gate_up_q, w->sh_gate_up_s, w->sh_down_q, w->sh_down_s, nullptr, nullptr, w->sh_gate_w};
}

BlockView view_of(const janus_moe_block_weights_nvfp4* w) {
  return BlockView{w->H, w->I, w->E, w->top_k, w->I_s, 1, w->router_w, w->router_prep, w->router_bias,
                   w->gate_up, w->gate_up_scale, w->down, w->down_scale, w->gate_up_global, w->down_global,
                   w->sh_gate_up, w->sh_gate_up_scale, w->sh_down, w->sh_down_scale, w->sh_gate_up_global,
                   w->sh_down_global, w->sh_gate_w};
}

// The block forward behind the block entries: x is the MoE input; serve null writes the layer output to out.
int block_forward(const BlockView* wt, const uint16_t* x, const uint8_t* valid, int T, uint16_t* out,
                  int32_t* topk_idx, float* topk_w, void* ws, size_t ws_bytes, hipStream_t stream,
                  const ServeEpilogue* serve) {
  const int H = wt->H, I = wt->I, E = wt->E, k = wt->top_k, I_s = wt->I_s;
  const bool nv = wt->codec == 1;
  int rc = check_expert_sizes("janus_moe_block_forward", T, H, I, E, k, I_s > 0 ? I_s : 0);
  if (rc) return rc;
  rc = check_route_sizes(T, H, E, k);
  if (rc) return rc;
  JANUS_REQUIRE(I_s >= 0 && I_s % 128 == 0, JANUS_MOE_EINVAL, "janus_moe_block_forward: I_s=%d must be a multiple of 128",
                I_s);
  if (T == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(x && (out || serve) && wt->router_w && wt->router_prep && wt->gate_up && wt->gate_up_scale &&
                    wt->down && wt->down_scale && (!nv || (wt->gate_up_global && wt->down_global)) &&
                    (I_s == 0 || (wt->sh_gate_up && wt->sh_gate_up_scale && wt->sh_down && wt->sh_down_scale &&
                                  (!nv || (wt->sh_gate_up_global && wt->sh_down_global)))),
                JANUS_MOE_EINVAL, "janus_moe_block_forward%s: null pointer", nv ? "_nvfp4" : "");
  const size_t need = janus_moe_block_workspace_bytes(T, H, I, E, k, I_s);
  JANUS_REQUIRE(ws && ws_bytes >= need, JANUS_MOE_EWORKSPACE, "janus_moe_block_forward: workspace %zu < %zu bytes",
                ws_bytes, need);
  Carver c(ws);
  BlockWorkspace b = carve_block(c, T, H, I, E, k, I_s);
  int32_t* idx = topk_idx ? topk_idx : b.topk_idx;
  float* rw = topk_w ? topk_w : b.topk_w;
  const bool gated = I_s > 0 && wt->sh_gate_w;
  mark(0, stream);
  rc = launch_route(x, wt->router_w, wt->router_prep, wt->router_bias, gated ? wt->sh_gate_w : nullptr, T, H, E, k,
                    valid, idx, rw, b.gamma, b.route, stream);
  if (rc) return rc;
  auto words = [](const void* p) { return static_cast<const int32_t*>(p); };
  auto halves = [](const void* p) { return static_cast<const uint16_t*>(p); };
  return run_experts<int>(x, idx, rw, words(wt->gate_up), halves(wt->gate_up_scale), words(wt->down),
                          halves(wt->down_scale), words(wt->sh_gate_up), halves(wt->sh_gate_up_scale),
                          words(wt->sh_down), halves(wt->sh_down_scale), gated ? b.gamma : nullptr, T, H, I, I_s, E, k,
                          out, b.experts, stream, wt->codec, wt->gate_up_global, wt->down_global, valid, serve,
                          nullptr, wt->sh_gate_up_global, wt->sh_down_global);
}
}  // namespace

extern "C" int janus_moe_block_forward_masked(const janus_moe_block_weights* wt, const uint16_t* x,
                                              const uint8_t* valid, int T, uint16_t* out, int32_t* topk_idx,
                                              float* topk_w, void* ws, size_t ws_bytes, janus_stream_t stream) {
  JANUS_REQUIRE(wt, JANUS_MOE_EINVAL, "janus_moe_block_forward: null weights");
  const BlockView v = view_of(wt);
  return block_forward(&v, x, valid, T, out, topk_idx, topk_w, ws, ws_bytes, (hipStream_t)stream, nullptr);
}

extern "C" int janus_moe_block_forward_nvfp4(const janus_moe_block_weights_nvfp4* wt, const uint16_t* x,
                                             const uint8_t* valid, int T, uint16_t* out, int32_t* topk_idx,
                                             float* topk_w, void* ws, size_t ws_bytes, janus_stream_t stream) {
  JANUS_REQUIRE(wt, JANUS_MOE_EINVAL, "janus_moe_block_forward_nvfp4: null weights");
  const BlockView v = view_of(wt);
  return block_forward(&v, x, valid, T, out, topk_idx, topk_w, ws, ws_bytes, (hipStream_t)stream, nullptr);
}

namespace {
// The scratch of janus_moe_block_forward_noalloc: a file-scope device array, one copy per GPU the library runs on,
// held until the process ends. In host code `scratch` names a host-side stand-in, not device memory: the device
// address comes from hipGetSymbolAddress, once per device with that device current, and only that address is used.
__device__ __align__(256) unsigned char scratch[JANUS_MOE_NOALLOC_SCRATCH_BYTES];

void* scratch_address() {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  void* p = cache[dev].load(std::memory_order_acquire);
  if (!p) {
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    cache[dev].store(p, std::memory_order_release);
  }
  return p;
}
}  // namespace

extern "C" int janus_moe_block_forward_noalloc(const janus_moe_block_weights* wt, const uint16_t* x,
                                               const uint8_t* valid, int T, uint16_t* out, int32_t* topk_idx,
                                               float* topk_w, janus_stream_t stream) {
  JANUS_REQUIRE(wt, JANUS_MOE_EINVAL, "janus_moe_block_forward_noalloc: null weights");
  const size_t need = janus_moe_block_workspace_bytes(T, wt->H, wt->I, wt->E, wt->top_k, wt->I_s);
  JANUS_REQUIRE(need <= JANUS_MOE_NOALLOC_SCRATCH_BYTES, JANUS_MOE_EWORKSPACE,
                "janus_moe_block_forward_noalloc: T=%d needs %zu bytes of scratch; the static array holds %zu (use "
                "janus_moe_block_forward_masked with a workspace)", T, need, (size_t)JANUS_MOE_NOALLOC_SCRATCH_BYTES);
  void* ws = scratch_address();
  JANUS_REQUIRE(ws, JANUS_MOE_ELAUNCH, "janus_moe_block_forward_noalloc: hipGetSymbolAddress of the scratch failed");
  const BlockView v = view_of(wt);
  return block_forward(&v, x, valid, T, out, topk_idx, topk_w, ws, JANUS_MOE_NOALLOC_SCRATCH_BYTES,
                       (hipStream_t)stream, nullptr);
}

extern "C" int janus_moe_block_forward_serve(const janus_moe_block_weights* wt, const uint16_t* x,
                                             const uint16_t* h_attn, const uint16_t* post_norm_w, float post_eps,
                                             const uint16_t* next_norm_w, float next_eps, const uint8_t* valid,
                                             const uint8_t* next_valid, int T, uint16_t* x_out, uint16_t* h_out,
                                             int32_t* topk_idx, float* topk_w, void* ws, size_t ws_bytes,
                                             janus_stream_t stream) {
  JANUS_REQUIRE(wt, JANUS_MOE_EINVAL, "janus_moe_block_forward_serve: null weights");
  int rc = check_norm_sizes(T, wt->H);
  if (rc) return rc;
  JANUS_REQUIRE(post_eps >= 0.f && next_eps >= 0.f, JANUS_MOE_EINVAL, "janus_moe_block_forward_serve: negative eps");
  if (T == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(x && post_norm_w && next_norm_w && x_out && h_out, JANUS_MOE_EINVAL,
                "janus_moe_block_forward_serve: null pointer");
  JANUS_REQUIRE(h_out != x && h_out != x_out, JANUS_MOE_EINVAL,
                "janus_moe_block_forward_serve: h_out must not alias x or x_out");
  const hipStream_t s = (hipStream_t)stream;
  // x_out = x + h_attn, h_out = the post-attention norm of it: the MoE's input
  rc = launch_add_rmsnorm(x, h_attn, post_norm_w, post_eps, nullptr, T, wt->H, x_out, h_out, s);
  if (rc) return rc;
  const ServeEpilogue serve = {x_out, next_norm_w, next_eps, next_valid, h_out};
  const BlockView v = view_of(wt);
  return block_forward(&v, h_out, valid, T, nullptr, topk_idx, topk_w, ws, ws_bytes, s, &serve);
}

extern "C" int janus_moe_dequant(const int32_t* q, const uint16_t* s, long rows, int K, uint16_t* out,
                                 janus_stream_t stream) {
  JANUS_REQUIRE(rows >= 0 && K > 0 && K % 128 == 0, JANUS_MOE_EINVAL, "janus_moe_dequant: rows=%ld K=%d (need K %% 128 == 0)",
                rows, K);
  if (rows == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(q && s && out, JANUS_MOE_EINVAL, "janus_moe_dequant: null pointer");
  return launch_dequant(q, s, rows, K, out, (hipStream_t)stream);
}
