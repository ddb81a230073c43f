// Router on gfx950: the softmax / top-k / renormalise of Qwen3_5MoeTopKRouter.forward
// (transformers models/qwen3_5_moe/modeling_qwen3_5_moe.py:768-776) with a bit-exact selection rule:
//   logit(t, e) = fp32 round-to-nearest-even of the exact dot product x[t] . w[e] (+ bias[e] in fp32);
//   the top_k largest logits, ties to the lower expert id, in descending slot order.
//
// Two launches, no host sync:
//   router_logits  approximate logits for every (token, expert): bf16 MFMA over a two-plane split of the fp32 weight
//                  (w = hi + mid + r, |r| <= 2^-16 |w|), fp32 accumulation, split over k in 512-wide slices.
//   router_select  one wave per token: the candidate set {e : approx_e >= approx_(k) - 2 delta_t} provably contains the
//                  top_k, where delta_t >= |approx - exact| (Cauchy-Schwarz on the split residual plus a 2^-12 relative
//                  allowance for fp32 accumulation). Only candidates in a cluster of approximate values closer than
//                  2 delta that reaches into the top_k need their exact logit: an fp64 dot product whose error bound
//                  decides the fp32 rounding, or, within that bound of a rounding midpoint, a double-double sum.
#include "router.h"

namespace janus {
namespace {

constexpr int kSlice = 512;      // k per router_logits workgroup
constexpr int kSelThreads = 256; // 4 tokens per select workgroup
constexpr int kMaxJ = 16;        // experts per lane (E <= 1024)
constexpr int kMaxHv = 8;        // 16-byte x vectors per lane (H <= 4096)

struct RouterPrep {
  uint16_t* hi;      // [E, H] bf16
  uint16_t* mid;     // [E, H] bf16
  double* wnorm;     // [E] ||w_e||_2
  double* resnorm;   // [E] ||w_e - hi_e - mid_e||_2
  double* meta;      // [0] max_e resnorm, [1] max_e wnorm
};

RouterPrep carve_prep(Carver& c, int E, int H) {
  RouterPrep p;
  p.hi = c.take<uint16_t>((size_t)E * H);
  p.mid = c.take<uint16_t>((size_t)E * H);
  p.wnorm = c.take<double>(E);
  p.resnorm = c.take<double>(E);
  p.meta = c.take<double>(2);
  return p;
}

// Orders this wave's LDS traffic: a wave's LDS operations execute in program order, so keeping the compiler from
// moving accesses across this point is enough for lanes to see each other's writes.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_down(v, off);
  return __shfl(v, 0);
}
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_down(v, off);
  return __shfl(v, 0);
}

// ---- prepare: split rows, norms -------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) router_split_kernel(const float* __restrict__ w, int E, int H, RouterPrep p) {
  const int e = blockIdx.x;
  __shared__ double red[2][256];
  double r2 = 0.0, w2 = 0.0;
  for (int h = threadIdx.x; h < H; h += 256) {
    const float v = w[(long)e * H + h];
    const __bf16 hi = static_cast<__bf16>(v);
    const float r1 = v - static_cast<float>(hi);
    const __bf16 mid = static_cast<__bf16>(r1);
    const float r2f = r1 - static_cast<float>(mid);
    p.hi[(long)e * H + h] = __builtin_bit_cast(uint16_t, hi);
    p.mid[(long)e * H + h] = __builtin_bit_cast(uint16_t, mid);
    r2 += (double)r2f * (double)r2f;
    w2 += (double)v * (double)v;
  }
  red[0][threadIdx.x] = r2;
  red[1][threadIdx.x] = w2;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      red[0][threadIdx.x] += red[0][threadIdx.x + s];
      red[1][threadIdx.x] += red[1][threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    p.wnorm[e] = sqrt(red[1][0]);
    p.resnorm[e] = sqrt(red[0][0]);
  }
}

__global__ void __launch_bounds__(256) router_meta_kernel(int E, RouterPrep p) {
  __shared__ double red[2][256];
  double r = 0.0, w = 0.0;
  for (int e = threadIdx.x; e < E; e += 256) {
    r = fmax(r, p.resnorm[e]);
    w = fmax(w, p.wnorm[e]);
  }
  red[0][threadIdx.x] = r;
  red[1][threadIdx.x] = w;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      red[0][threadIdx.x] = fmax(red[0][threadIdx.x], red[0][threadIdx.x + s]);
      red[1][threadIdx.x] = fmax(red[1][threadIdx.x], red[1][threadIdx.x + s]);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    p.meta[0] = red[0][0];
    p.meta[1] = red[1][0];
  }
}

// ---- approximate logits ---------------------------------------------------------------------------------------
// grid (ceil(T/64), ceil(E/64), ceil(H/512)); wave w: experts blockIdx.y*64 + 16w .. +15, tokens blockIdx.x*64 .. +63.
__global__ void __launch_bounds__(256) router_logits_kernel(const uint16_t* __restrict__ x, RouterPrep p, int T, int H,
                                                            int E, int Epad, float* __restrict__ partial) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, nl = lane & 15;
  const int e = blockIdx.y * 64 + wave * 16 + nl;
  const int t0 = blockIdx.x * 64;
  const int k0 = blockIdx.z * kSlice, k1 = min(H, k0 + kSlice);
  const bool e_ok = e < E;
  const uint16_t* hrow = p.hi + (long)(e_ok ? e : 0) * H;
  const uint16_t* mrow = p.mid + (long)(e_ok ? e : 0) * H;
  const uint16_t* xrow[4];
  bool t_ok[4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int t = t0 + tb * 16 + nl;
    t_ok[tb] = t < T;
    xrow[tb] = x + (long)(t_ok[tb] ? t : 0) * H;
  }
  f32x4 acc[4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) acc[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16x8 zero8 = {};
  // four k-steps per iteration: their 24 fragment loads are all in flight before the first MFMA
  constexpr int kU = 4;
  for (int k = k0; k < k1; k += 32 * kU) {
    bf16x8 a_hi[kU], a_mid[kU], b[kU][4];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int kk = k + 32 * u + 8 * g;
      const bool k_ok = kk < k1;
      a_hi[u] = (e_ok && k_ok) ? *reinterpret_cast<const bf16x8*>(hrow + kk) : zero8;
      a_mid[u] = (e_ok && k_ok) ? *reinterpret_cast<const bf16x8*>(mrow + kk) : zero8;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
        b[u][tb] = (t_ok[tb] && k_ok) ? *reinterpret_cast<const bf16x8*>(xrow[tb] + kk) : zero8;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        acc[tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi[u], b[u][tb], acc[tb], 0, 0, 0);
        acc[tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_mid[u], b[u][tb], acc[tb], 0, 0, 0);
      }
  }
  // lane holds experts blockIdx.y*64 + 16*wave + 4g + i of token t0 + 16tb + nl
  const int ebase = blockIdx.y * 64 + wave * 16 + 4 * g;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int t = t0 + tb * 16 + nl;
    if (t < T)
      *reinterpret_cast<float4*>(partial + ((long)blockIdx.z * T + t) * Epad + ebase) =
          make_float4(acc[tb][0], acc[tb][1], acc[tb][2], acc[tb][3]);
  }
}

// ---- exact logits ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void two_sum(double a, double b, double& s, double& e) {
  s = a + b;
  const double bb = s - a;
  e = (a - (s - bb)) + (b - bb);
}

// Neighbouring fp32 values of a finite r (integer steps on the bit pattern).
__device__ __forceinline__ float f32_next_up(float r) {
  if (r == 0.0f) return __uint_as_float(1u);
  const uint32_t b = __float_as_uint(r);
  return __uint_as_float(r > 0.0f ? b + 1u : b - 1u);
}
__device__ __forceinline__ float f32_next_down(float r) { return -f32_next_up(-r); }

// fp32 nearest-even rounding of hi + lo (|lo| <= ulp(hi)/2): differs from float(hi) only when hi is exactly an fp32
// midpoint, where the sign of lo decides.
__device__ float round_dd_to_f32(double hi, double lo) {
  const float r = (float)hi;
  const double rd = (double)r;
  if (rd == hi || lo == 0.0) return r;
  const float n = hi > rd ? f32_next_up(r) : f32_next_down(r);
  const double mid = 0.5 * (rd + (double)n);
  if (hi != mid) return r;
  return ((lo > 0.0) == (hi > rd)) ? n : r;
}

// Wave-cooperative exact logit of (x of this lane, expert row wrow). xv: the lane's x vectors (8 bf16 each at
// h = 512 j + 8 lane). Returns the correctly rounded fp32 dot product in every lane.
__device__ float exact_logit(const uint4 (&xv)[kMaxHv], int nhv, int H, const float* __restrict__ wrow, double bound) {
  const int lane = threadIdx.x & 63;
  double acc = 0.0;
  int nterms = 0;
  float wv[kMaxHv][8];
#pragma unroll
  for (int j = 0; j < kMaxHv; ++j) {
    if (j >= nhv) break;
    const int h0 = 512 * j + 8 * lane;
    if (h0 < H) {
      const float4 a = *reinterpret_cast<const float4*>(wrow + h0);
      const float4 b = *reinterpret_cast<const float4*>(wrow + h0 + 4);
      wv[j][0] = a.x; wv[j][1] = a.y; wv[j][2] = a.z; wv[j][3] = a.w;
      wv[j][4] = b.x; wv[j][5] = b.y; wv[j][6] = b.z; wv[j][7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) wv[j][i] = 0.f;
    }
  }
#pragma unroll
  for (int j = 0; j < kMaxHv; ++j) {
    if (j >= nhv) break;
    const uint32_t words[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float xf = __uint_as_float(i & 1 ? (words[i / 2] & 0xFFFF0000u) : (words[i / 2] << 16));
      acc = fma((double)xf, (double)wv[j][i], acc);
    }
    nterms += 8;
  }
  const double v = wave_sum_f64(acc);
  // |v - exact| <= (terms per lane + tree depth) * 2^-53 * sum|x w| <= that * ||x|| ||w||
  const double err = (double)(nterms + 6) * 0x1p-53 * bound;
  const float r = (float)v;
  const double rd = (double)r;
  const double dn = 0.5 * (rd + (double)f32_next_down(r));
  const double up = 0.5 * (rd + (double)f32_next_up(r));
  if (v - dn > err && up - v > err) return r;
  // Within the bound of a rounding midpoint: double-double accumulation.
  double hi = 0.0, lo = 0.0;
#pragma unroll
  for (int j = 0; j < kMaxHv; ++j) {
    if (j >= nhv) break;
    const uint32_t words[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float xf = __uint_as_float(i & 1 ? (words[i / 2] & 0xFFFF0000u) : (words[i / 2] << 16));
      double s, e;
      two_sum(hi, (double)xf * (double)wv[j][i], s, e);
      hi = s;
      lo += e;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const double h2 = __shfl_down(hi, off), l2 = __shfl_down(lo, off);
    double s, e;
    two_sum(hi, h2, s, e);
    lo = lo + l2 + e;
    hi = s;
  }
  double s, e;
  two_sum(hi, lo, s, e);
  const float out = round_dd_to_f32(s, e);
  return __shfl(out, 0);
}

// ---- selection -----------------------------------------------------------------------------------------------
struct Cand {
  float v;
  int e;
};

__device__ __forceinline__ bool better(float va, int ea, float vb, int eb) { return va > vb || (va == vb && ea < eb); }

// Sorts cand[0..n) (value descending, id ascending) into out[0..n) by rank counting.
__device__ void rank_sort(const Cand* cand, Cand* out, int n) {
  const int lane = threadIdx.x & 63;
  for (int i = lane; i < n; i += 64) {
    const Cand ci = cand[i];
    int r = 0;
    for (int j = 0; j < n; ++j) r += better(cand[j].v, cand[j].e, ci.v, ci.e);
    out[r] = ci;
  }
}

__global__ void __launch_bounds__(kSelThreads) router_select_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ w, RouterPrep p, const float* __restrict__ bias,
    const uint16_t* __restrict__ wsg, int T, int H, int E, int Epad, int nslice, int top_k,
    const float* __restrict__ partial, int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    float* __restrict__ gamma) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  Cand* cand = reinterpret_cast<Cand*>(smem) + (size_t)wave * 2 * E;
  Cand* sorted = cand + E;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;  // a whole wave; no workgroup barriers below

  // x row in registers, norm, shared gate
  const int nhv = (H + 511) / 512;
  uint4 xv[kMaxHv];
  float ss = 0.f, gdot = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxHv; ++j) {
    xv[j] = make_uint4(0, 0, 0, 0);
    if (j < nhv) {
      const int h0 = 512 * j + 8 * lane;
      if (h0 < H) {
        xv[j] = *reinterpret_cast<const uint4*>(x + (long)t * H + h0);
        const uint32_t words[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
        uint4 gw = wsg ? *reinterpret_cast<const uint4*>(wsg + h0) : make_uint4(0, 0, 0, 0);
        const uint32_t gws[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xf = __uint_as_float(i & 1 ? (words[i / 2] & 0xFFFF0000u) : (words[i / 2] << 16));
          const float gf = __uint_as_float(i & 1 ? (gws[i / 2] & 0xFFFF0000u) : (gws[i / 2] << 16));
          ss = fmaf(xf, xf, ss);
          gdot = fmaf(xf, gf, gdot);
        }
      }
    }
  }
  ss = wave_sum_f32(ss);
  if (wsg) {
    gdot = wave_sum_f32(gdot);
    if (lane == 0 && gamma) gamma[t] = 1.0f / (1.0f + __expf(-gdot));
  }
  const double xnorm = sqrt((double)ss) * (1.0 + 1e-5);
  const double delta = xnorm * (p.meta[0] + 0x1p-12 * p.meta[1]) + 1e-30;

  // approximate logits: lane holds experts lane + 64 j
  const int nj = (E + 63) / 64;
  float av[kMaxJ];
#pragma unroll
  for (int j = 0; j < kMaxJ; ++j) {
    av[j] = -__builtin_inff();
    const int e = lane + 64 * j;
    if (j < nj && e < E) {
      float s = 0.f;
#pragma unroll
      for (int z = 0; z < kMaxHv; ++z)
        if (z < nslice) s += partial[((long)z * T + t) * Epad + e];
      if (bias) s += bias[e];
      av[j] = s;
    }
  }
  // k-th largest approximate value (ties to the lower id)
  uint32_t taken = 0;
  float vk = 0.f;
  for (int r = 0; r < top_k; ++r) {
    float bv = -__builtin_inff();
    int be = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kMaxJ; ++j) {
      const int e = lane + 64 * j;
      if (j < nj && e < E && !((taken >> j) & 1) && better(av[j], e, bv, be)) {
        bv = av[j];
        be = e;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oe = __shfl_xor(be, off);
      if (better(ov, oe, bv, be)) {
        bv = ov;
        be = oe;
      }
    }
    if ((be & 63) == lane) taken |= 1u << (be >> 6);
    vk = bv;
  }
  // bias rounding and the split / accumulation allowance
  const float d2 = (float)(2.0 * delta) + (bias ? 4.0f * __builtin_fabsf(vk) * 0x1p-24f : 0.f);
  const float theta = vk - d2;
  // candidates in LDS
  int nc = 0;
#pragma unroll
  for (int j = 0; j < kMaxJ; ++j) {
    const int e = lane + 64 * j;
    const bool pred = j < nj && e < E && av[j] >= theta;
    const uint64_t m = ballot(pred);
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    if (pred) cand[nc + __popcll(m & below)] = Cand{av[j], e};
    nc += __popcll(m);
  }
  wave_sync();
  rank_sort(cand, sorted, nc);
  wave_sync();
  // which candidates need their exact logit: members of a cluster (adjacent gaps < d2) that reaches into the top_k.
  // Flags for all candidates first (in cand[].e, free after the sort), from approximate values only.
  if (lane == 0) {
    int s = 0;
    for (int i = 0; i < nc; ++i) {
      if (i > 0 && sorted[i - 1].v - sorted[i].v >= d2) s = i;  // s: start of i's cluster
      int e2 = i;
      while (e2 + 1 < nc && sorted[e2].v - sorted[e2 + 1].v < d2) ++e2;
      cand[i].e = (e2 > s || (i > s)) && (s < top_k);
    }
  }
  wave_sync();
  for (int i = 0; i < nc; ++i) {
    if (cand[i].e) {  // wave-uniform
      const int e = sorted[i].e;
      float l = exact_logit(xv, nhv, H, w + (long)e * H, xnorm * p.wnorm[e] * (1.0 + 1e-6));
      if (bias) l = l + bias[e];
      if (lane == 0) sorted[i].v = l;
    }
  }
  wave_sync();
  rank_sort(sorted, cand, nc);
  wave_sync();
  // renormalised softmax over the top_k
  float v = -__builtin_inff();
  int e = 0;
  if (lane < top_k) {
    v = cand[lane].v;
    e = cand[lane].e;
  }
  const float vmax = __shfl(v, 0);
  const float ex = lane < top_k ? expf(v - vmax) : 0.f;
  const float den = wave_sum_f32(ex);
  if (lane < top_k) {
    topk_idx[(long)t * top_k + lane] = e;
    topk_w[(long)t * top_k + lane] = ex / den;
  }
}

}  // namespace

size_t router_prep_bytes(int E, int H) {
  Carver c(nullptr);
  carve_prep(c, E, H);
  return align_up(c.used, 256);
}

size_t route_workspace_bytes(int T, int H, int E) {
  Carver c(nullptr);
  carve_route(c, T, H, E);
  return align_up(c.used, 256);
}

RouteWorkspace carve_route(Carver& c, int T, int H, int E) {
  RouteWorkspace r;
  const int nslice = ceil_div(H, kSlice);
  const int Epad = ceil_div(E, 64) * 64;
  r.partial = c.take<float>((size_t)nslice * (T > 0 ? T : 1) * Epad);
  return r;
}

int launch_route(const uint16_t* x, const float* w, const void* prep, const float* bias, const uint16_t* wsg, int T,
                 int H, int E, int top_k, int32_t* topk_idx, float* topk_w, float* gamma, const RouteWorkspace& ws,
                 hipStream_t stream) {
  if (T == 0) return JANUS_MOE_OK;
  Carver pc(const_cast<void*>(prep));
  RouterPrep p = carve_prep(pc, E, H);
  const int nslice = ceil_div(H, kSlice);
  const int Epad = ceil_div(E, 64) * 64;
  hipLaunchKernelGGL(router_logits_kernel, dim3(ceil_div(T, 64), Epad / 64, nslice), dim3(256), 0, stream, x, p, T, H,
                     E, Epad, ws.partial);
  JANUS_LAUNCH_CHECK("router_logits");
  const size_t smem = (size_t)4 * 2 * E * sizeof(Cand);
  hipLaunchKernelGGL(router_select_kernel, dim3(ceil_div(T, 4)), dim3(kSelThreads), smem, stream, x, w, p, bias, wsg, T,
                     H, E, Epad, nslice, top_k, ws.partial, topk_idx, topk_w, gamma);
  JANUS_LAUNCH_CHECK("router_select");
  return JANUS_MOE_OK;
}

int check_route_sizes(int T, int H, int E, int top_k) {
  JANUS_REQUIRE(T >= 0 && H > 0 && H % 32 == 0 && H <= 512 * kMaxHv && E > 0 && E <= 64 * kMaxJ && E % 4 == 0 &&
                    top_k > 0 && top_k <= 64 && top_k <= E,
                JANUS_MOE_EINVAL, "router: unsupported sizes T=%d H=%d E=%d top_k=%d (need H %% 32 == 0, H <= %d, "
                "E %% 4 == 0, E <= %d, top_k <= min(64, E))", T, H, E, top_k, 512 * kMaxHv, 64 * kMaxJ);
  return JANUS_MOE_OK;
}

}  // namespace janus

using namespace janus;

extern "C" size_t janus_moe_router_prep_bytes(int E, int H) {
  if (E <= 0 || H <= 0) return 0;
  return router_prep_bytes(E, H);
}

extern "C" int janus_moe_router_prepare(const float* w_router, int E, int H, void* prep, size_t prep_bytes,
                                        janus_stream_t stream) {
  JANUS_REQUIRE(E > 0 && H > 0 && H % 8 == 0, JANUS_MOE_EINVAL, "janus_moe_router_prepare: bad sizes E=%d H=%d", E, H);
  JANUS_REQUIRE(w_router && prep, JANUS_MOE_EINVAL, "janus_moe_router_prepare: null pointer");
  JANUS_REQUIRE(prep_bytes >= router_prep_bytes(E, H), JANUS_MOE_EWORKSPACE,
                "janus_moe_router_prepare: prep buffer %zu < %zu bytes", prep_bytes, router_prep_bytes(E, H));
  Carver pc(prep);
  RouterPrep p = carve_prep(pc, E, H);
  hipLaunchKernelGGL(router_split_kernel, dim3(E), dim3(256), 0, (hipStream_t)stream, w_router, E, H, p);
  JANUS_LAUNCH_CHECK("router_split");
  hipLaunchKernelGGL(router_meta_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, E, p);
  JANUS_LAUNCH_CHECK("router_meta");
  return JANUS_MOE_OK;
}

extern "C" size_t janus_moe_route_workspace_bytes(int T, int H, int E) {
  if (T < 0 || H <= 0 || E <= 0) return 0;
  return route_workspace_bytes(T, H, E);
}

extern "C" int janus_moe_route(const uint16_t* x, const float* w_router, const void* prep, const float* bias,
                               const uint16_t* w_shared_gate, int T, int H, int E, int top_k, int32_t* topk_idx,
                               float* topk_w, float* gamma, void* ws, size_t ws_bytes, janus_stream_t stream) {
  int rc = check_route_sizes(T, H, E, top_k);
  if (rc) return rc;
  JANUS_REQUIRE(T == 0 || (x && w_router && prep && topk_idx && topk_w), JANUS_MOE_EINVAL, "janus_moe_route: null pointer");
  const size_t need = route_workspace_bytes(T, H, E);
  JANUS_REQUIRE(ws && ws_bytes >= need, JANUS_MOE_EWORKSPACE, "janus_moe_route: workspace %zu < %zu bytes", ws_bytes,
                need);
  Carver c(ws);
  RouteWorkspace r = carve_route(c, T, H, E);
  return launch_route(x, w_router, prep, bias, w_shared_gate, T, H, E, top_k, topk_idx, topk_w, gamma, r,
                      (hipStream_t)stream);
}
