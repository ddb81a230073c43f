// Router on gfx950: the softmax / top-k / renormalise of Qwen3_5MoeTopKRouter.forward
// (transformers models/qwen3_5_moe/modeling_qwen3_5_moe.py:768-776) with a bit-exact selection rule:
//   logit(t, e) = fp32 round-to-nearest-even of the exact dot product x[t] . w[e] (+ bias[e] in fp32);
//   the top_k largest logits, ties to the lower expert id, in descending slot order.
//
// Two launches, no host sync:
//   router_logits  approximate logits for every (token, expert): bf16 MFMA over a two-plane split of the fp32 weight
//                  (w = hi + mid + r, |r| <= 2^-16 |w|), fp32 accumulation, split over k in 512-wide slices.
//   router_select  one wave per token: the candidate set {e : approx_e >= approx_(k) - 2 delta_t} provably contains the
//                  top_k, where delta_t >= |approx - exact| (Cauchy-Schwarz on the split residual plus a 2^-17 relative
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
// grid (ceil(T/64), Epad/64, ceil(H/512)); wave w: experts blockIdx.y*64 + 16w .. +15, tokens blockIdx.x*64 .. +63 of
// the k slice blockIdx.z. The slice of the 64 x rows sits in LDS (shared by the 4 waves); each wave streams its 16
// expert rows of both planes from global memory, kAhead k-steps ahead.
//
// Rounding. Every bf16 x bf16 product is exact in fp32. Each k-step of 32 forms a fresh block sum of the 32 hi-plane
// products (one MFMA from zero) that VALU adds to the running fp32 hi sum; the mid plane (|mid| <= 2^-9 |w|)
// accumulates in its own MFMA chain over the slice, and the slice's partial is hi sum + mid sum. A hi product passes
// through at most 31 roundings in its block, 16 block additions, the final addition and up to 8 slice additions (in
// router_select): 56 roundings of at most 2^-23 relative each (truncating arithmetic assumed), 2^-17.2 of sum |x w|;
// a mid product through at most 512 + 1 + 8, which is 521 * 2^-23 * 2^-9 < 2^-22 of sum |x w|. Together within the
// 2^-17 allowance the selection uses, with sum |x w| <= ||x|| ||w||.
constexpr int kSteps = kSlice / 32;  // k-steps per slice
constexpr int kAhead = 8;            // weight fragment loads in flight per wave
constexpr int kTileT = 64;           // tokens per workgroup
constexpr int kXRowBytes = kSlice * 2;

__global__ void __launch_bounds__(256, 2) router_logits_kernel(const uint16_t* __restrict__ x, RouterPrep p, int T, int H,
                                                            int E, int Epad, float* __restrict__ partial) {
  __shared__ __attribute__((aligned(16))) unsigned char xs[kTileT * kXRowBytes];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, nl = lane & 15;
  const int t0 = blockIdx.x * kTileT;
  const int k0 = blockIdx.z * kSlice, klen = min(H - k0, kSlice);

  // x tile: 64 rows x 64 16-byte chunks, chunk c of row r stored at chunk position c ^ (r & 15). Buffer loads write it
  // straight into LDS (lane l of a load fills position l of the row); a chunk past the slice or a row past T is given
  // an offset beyond the buffer, which the hardware returns as zeros.
  const __amdgpu_buffer_rsrc_t xrsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), (short)0, (int)((long)T * H * 2), 0x00020000);
#pragma unroll
  for (int i = 0; i < kTileT / 4; ++i) {
    const int row = wave * (kTileT / 4) + i, t = t0 + row, c = lane ^ (row & 15);
    const uint32_t off = (t < T && c * 8 < klen) ? (uint32_t)(((long)t * H + k0 + c * 8) * 2) : 0x80000000u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xrsrc, (__attribute__((address_space(3))) void*)(xs + row * kXRowBytes),
                                             16, off, 0, 0, 0);
  }
  const int e = blockIdx.y * 64 + wave * 16 + nl;
  const bool e_ok = e < E;
  const uint16_t* hrow = p.hi + (long)(e_ok ? e : 0) * H + k0 + 8 * g;
  const uint16_t* mrow = p.mid + (long)(e_ok ? e : 0) * H + k0 + 8 * g;
  u32x4 wh[kAhead], wm[kAhead];
  // Loads without a branch, so that all of them are in flight together: an expert past E reads expert 0's row (its
  // column of partial is padding, never selected), a step past the slice re-reads step 0 (the x tile is zero there,
  // and finite weights times zero add nothing).
  auto load_w = [&](int slot, int step) __attribute__((always_inline)) {
    const int st = 32 * step < klen ? step : 0;
    wh[slot] = *reinterpret_cast<const u32x4*>(hrow + 32 * st);
    wm[slot] = *reinterpret_cast<const u32x4*>(mrow + 32 * st);
  };
#pragma unroll
  for (int s = 0; s < kAhead; ++s) load_w(s, s);
  __syncthreads();

  f32x4 acc[4], accm[4];  // hi-plane running sums (fresh block per step), mid-plane MFMA chains
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) acc[tb] = accm[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int slot = s % kAhead;
    const bf16x8 hf = __builtin_bit_cast(bf16x8, wh[slot]);
    const bf16x8 mf = __builtin_bit_cast(bf16x8, wm[slot]);
    if (s + kAhead < kSteps) load_w(slot, s + kAhead);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const int row = 16 * tb + nl;
      const bf16x8 xf = *reinterpret_cast<const bf16x8*>(xs + row * kXRowBytes + (((4 * s + g) ^ nl) * 16));
      const f32x4 b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hf, xf, zero4, 0, 0, 0);
      accm[tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mf, xf, accm[tb], 0, 0, 0);
      acc[tb] += b;
      asm volatile("" : "+v"(acc[tb]));  // add now: left alone, the compiler keeps every step's block sum live
    }
  }
  // lane holds experts blockIdx.y*64 + 16*wave + 4g + i of token t0 + 16tb + nl
  const int ebase = blockIdx.y * 64 + wave * 16 + 4 * g;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int t = t0 + tb * 16 + nl;
    if (t < T)
      *reinterpret_cast<float4*>(partial + ((long)blockIdx.z * T + t) * Epad + ebase) =
          make_float4(acc[tb][0] + accm[tb][0], acc[tb][1] + accm[tb][1], acc[tb][2] + accm[tb][2],
                      acc[tb][3] + accm[tb][3]);
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

// Wave-cooperative exact logits of this lane's x (8 bf16 at h = 512 j + 8 lane) against the rows ids[0..n) of w
// (wave-uniform, n <= kExactBatch). The loads of all n rows are in flight together. out[c]: the correctly rounded fp32
// dot product, in every lane. bound[c] >= ||x|| ||w_c||.
constexpr int kExactBatch = 4;  // array size; rows per batch: exact_batch(NHV)
constexpr int exact_batch(int nhv) { return nhv <= 2 ? 4 : nhv == 4 ? 2 : 1; }

template <int NHV>
struct XRow {
  uint4 v[NHV];
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
template <int NHV>
__device__ __forceinline__ float xval(const XRow<NHV>& x, int j, int i) {
  const uint32_t wd = i < 2 ? x.v[j].x : i < 4 ? x.v[j].y : i < 6 ? x.v[j].z : x.v[j].w;
  return (i & 1) ? bf16_hi(wd) : bf16_lo(wd);
}
template <int NHV>
__device__ __forceinline__ void load_wrow(const float* __restrict__ wrow, int H, bool ok, float (&wv)[NHV][8]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < NHV; ++j) {
    const int h0 = 512 * j + 8 * lane;
    if (ok && h0 < H) {
      const float4 a = *reinterpret_cast<const float4*>(wrow + h0);
      const float4 b = *reinterpret_cast<const float4*>(wrow + h0 + 4);
      wv[j][0] = a.x; wv[j][1] = a.y; wv[j][2] = a.z; wv[j][3] = a.w;
      wv[j][4] = b.x; wv[j][5] = b.y; wv[j][6] = b.z; wv[j][7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) wv[j][i] = 0.f;
    }
  }
}

// The exact logit when an fp64 sum lies within its error bound of an fp32 rounding midpoint: double-double
// accumulation of the same products. Rare; kept out of line so the common path keeps its registers.
template <int NHV>
__device__ __noinline__ float exact_logit_dd(XRow<NHV> x, const float* __restrict__ wrow, int H) {
  float wv[NHV][8];
  load_wrow<NHV>(wrow, H, true, wv);
  double hi = 0.0, lo = 0.0;
#pragma unroll
  for (int j = 0; j < NHV; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      double s2, e2;
      two_sum(hi, (double)xval(x, j, i) * (double)wv[j][i], s2, e2);
      hi = s2;
      lo += e2;
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const double h2 = __shfl_down(hi, off), l2 = __shfl_down(lo, off);
    double s2, e2;
    two_sum(hi, h2, s2, e2);
    lo = lo + l2 + e2;
    hi = s2;
  }
  double s2, e2;
  two_sum(hi, lo, s2, e2);
  return __shfl(round_dd_to_f32(s2, e2), 0);
}

template <int NHV>
__device__ void exact_logits(const XRow<NHV>& x, int H, const float* __restrict__ w, const int (&ids)[kExactBatch],
                             int n, const double (&bound)[kExactBatch], float (&out)[kExactBatch]) {
  float wv[kExactBatch][NHV][8];
#pragma unroll
  for (int c = 0; c < kExactBatch; ++c)
    if (c < exact_batch(NHV)) load_wrow<NHV>(w + (long)ids[c] * H, H, c < n, wv[c]);
  double v[kExactBatch];
#pragma unroll
  for (int c = 0; c < exact_batch(NHV); ++c) {
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < NHV; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = fma((double)xval(x, j, i), (double)wv[c][j][i], acc);
    v[c] = acc;
    __builtin_amdgcn_sched_barrier(0);  // one row's fp64 operands live at a time
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
    for (int c = 0; c < exact_batch(NHV); ++c) v[c] += __shfl_xor(v[c], off);
#pragma unroll
  for (int c = 0; c < exact_batch(NHV); ++c) v[c] = __shfl(v[c], 0);  // one value per wave: the branches below are uniform
#pragma unroll
  for (int c = 0; c < exact_batch(NHV); ++c) {
    if (c >= n) break;
    // |v - exact| <= (terms per lane + tree depth) * 2^-53 * sum|x w| <= that * ||x|| ||w||
    const double err = (double)(8 * NHV + 6) * 0x1p-53 * bound[c];
    const float r = (float)v[c];
    const double rd = (double)r;
    const double dn = 0.5 * (rd + (double)f32_next_down(r));
    const double up = 0.5 * (rd + (double)f32_next_up(r));
    out[c] = (v[c] - dn > err && up - v[c] > err) ? r : exact_logit_dd<NHV>(x, w + (long)ids[c] * H, H);
  }
}

// exact_logits in a function of its own, for rare paths whose caller should not reserve its registers.
template <int NHV>
__device__ __noinline__ void exact_logits_outlined(XRow<NHV> x, int H, const float* __restrict__ w,
                                                   const int (&ids)[kExactBatch], int n,
                                                   const double (&bound)[kExactBatch], float (&out)[kExactBatch]) {
  exact_logits<NHV>(x, H, w, ids, n, bound, out);
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

// Order-preserving map of fp32 onto uint32 (larger float <-> larger key), and back.
__device__ __forceinline__ uint32_t f32_key(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_f32(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Rank of (v, e) among the nc candidates held by lanes 0..nc-1 (value descending, id ascending), read lane by lane.
__device__ __forceinline__ int lane_rank(float v, int e, int nc) {
  int r = 0;
  for (int j = 0; j < nc; ++j) {
    const float vj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
    const int ej = __builtin_amdgcn_readlane(e, j);
    r += better(vj, ej, v, e);
  }
  return r;
}

// One wave per token. NJ: experts per lane (expert lane + 64 j), NHV: 16-byte x vectors per lane.
template <int NHV, int NJ>
__global__ void __launch_bounds__(kSelThreads) router_select_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ w, RouterPrep p, const float* __restrict__ bias,
    const uint16_t* __restrict__ wsg, int T, int H, int E, int Epad, int nslice, int top_k,
    const float* __restrict__ partial, const uint8_t* __restrict__ valid, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_w, float* __restrict__ gamma) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  Cand* cand = reinterpret_cast<Cand*>(smem) + (size_t)wave * 2 * E;
  Cand* sorted = cand + E;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;  // a whole wave; no workgroup barriers below
  if (valid && !valid[t]) {
    // a padding token: no expert (id E is dropped by align), weight 0, shared-expert gate 0
    if (lane < top_k) {
      topk_idx[(long)t * top_k + lane] = E;
      topk_w[(long)t * top_k + lane] = 0.f;
    }
    if (lane == 0 && gamma) gamma[t] = 0.f;
    return;
  }

  // every load up front: x row, shared-gate row, approximate logit slices, bias
  XRow<NHV> xrow;
  uint4 (&xv)[NHV] = xrow.v;
  uint4 gv[NHV];
#pragma unroll
  for (int j = 0; j < NHV; ++j) {
    const int h0 = 512 * j + 8 * lane;
    const bool ok = h0 < H;
    xv[j] = ok ? *reinterpret_cast<const uint4*>(x + (long)t * H + h0) : make_uint4(0, 0, 0, 0);
    gv[j] = (ok && wsg) ? *reinterpret_cast<const uint4*>(wsg + h0) : make_uint4(0, 0, 0, 0);
  }
  // The slices' partial sums and the bias, every load issued before the first is used. The loads take no branch:
  // a slice past nslice re-reads slice 0 and a column past Epad re-reads the lane's column of block 0 (both in
  // bounds), and the values that do not count are dropped afterwards. A load under a branch, feeding a running sum,
  // would cost a memory round trip each.
  float av[NJ];
  const float* prow = partial + (long)t * Epad + lane;
  const long zstride = (long)T * Epad;
  float pz[NJ][NHV], bj[NJ];  // nslice = ceil(H / 512) <= NHV
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int cj = 64 * j < Epad ? 64 * j : 0;  // uniform
#pragma unroll
    for (int z = 0; z < NHV; ++z) pz[j][z] = prow[(z < nslice ? z : 0) * zstride + cj];
    const int e = lane + 64 * j;
    bj[j] = bias ? bias[e < E ? e : 0] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const bool ok = lane + 64 * j < E;
    float sj = 0.f;
#pragma unroll
    for (int z = 0; z < NHV; ++z)
      if (z < nslice) sj += ok ? pz[j][z] : 0.f;
    if (bias) sj += ok ? bj[j] : 0.f;
    av[j] = ok ? sj : -__builtin_inff();
  }

  // norm of x and the shared-expert gate
  float ss = 0.f, gdot = 0.f;
#pragma unroll
  for (int j = 0; j < NHV; ++j) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float xf = xval(xrow, j, i);
      const uint32_t gw = i < 2 ? gv[j].x : i < 4 ? gv[j].y : i < 6 ? gv[j].z : gv[j].w;
      ss = fmaf(xf, xf, ss);
      gdot = fmaf(xf, (i & 1) ? bf16_hi(gw) : bf16_lo(gw), gdot);
    }
  }
  ss = wave_sum_f32(ss);
  if (wsg) {
    gdot = wave_sum_f32(gdot);
    if (lane == 0 && gamma) gamma[t] = 1.0f / (1.0f + __expf(-gdot));
  }
  const double xnorm = sqrt((double)ss) * (1.0 + 1e-5);
  const double delta = xnorm * (p.meta[0] + 0x1p-17 * p.meta[1]) + 1e-30;

  // k-th largest approximate value: binary search on the order-preserving keys, counting with ballots
  uint32_t key[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) key[j] = lane + 64 * j < E ? f32_key(av[j]) : 0u;
  uint32_t tau = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t trial = tau | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) cnt += __popcll(ballot(key[j] >= trial));
    if (cnt >= top_k) tau = trial;
  }
  const float vk = key_f32(tau);
  // bias rounding and the split / accumulation allowance
  const float d2 = (float)(2.0 * delta) + (bias ? 4.0f * __builtin_fabsf(vk) * 0x1p-24f : 0.f);
  const float theta = vk - d2;
  // candidates, compacted in id order into LDS
  int nc = 0;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const bool pred = lane + 64 * j < E && av[j] >= theta;
    const uint64_t m = ballot(pred);
    if (pred) cand[nc + __popcll(m & below)] = Cand{av[j], lane + 64 * j};
    nc += __popcll(m);
  }
  wave_sync();

  if (nc <= 64) {
    // lane i holds candidate i; ranks by reading the other lanes
    float vi = -__builtin_inff();
    int ei = 0x7fffffff;
    if (lane < nc) {
      vi = cand[lane].v;
      ei = cand[lane].e;
    }
    int r = lane_rank(vi, ei, nc);
    if (lane < nc) sorted[r] = Cand{vi, ei};
    wave_sync();
    if (lane < nc) {
      vi = sorted[lane].v;
      ei = sorted[lane].e;
    }
    // members of a cluster (adjacent gaps < d2) that reaches into the top_k need their exact logit
    const bool in = lane < nc;
    const float vp = __shfl_up(vi, 1);
    const uint64_t starts = ballot(in && (lane == 0 || vp - vi >= d2));
    const uint64_t upto = (2ull << lane) - 1;            // bits 0..lane
    const int cs = 63 - __clzll(starts & upto);            // this lane's cluster start (bit 0 is always set)
    const uint64_t next = starts & ~upto;
    const int last = next ? __builtin_ctzll(next) - 1 : nc - 1;  // this lane's cluster end
    uint64_t f = ballot(in && last > cs && cs < top_k);
    while (f) {
      int ids[kExactBatch], pos[kExactBatch];
      double bnd[kExactBatch];
      int n = 0;
#pragma unroll
      for (int c = 0; c < kExactBatch; ++c) {
        pos[c] = 0;
        ids[c] = 0;
        if (c < exact_batch(NHV) && f) {
          pos[c] = __builtin_ctzll(f);
          f &= f - 1;
          ids[c] = __builtin_amdgcn_readlane(ei, pos[c]);
          n = c + 1;
        }
      }
      // the batch's norms and biases loaded together, outside the branches above (an unused entry reads expert 0)
      float bb[kExactBatch];
#pragma unroll
      for (int c = 0; c < kExactBatch; ++c) {
        bnd[c] = xnorm * p.wnorm[ids[c]] * (1.0 + 1e-6);
        bb[c] = bias ? bias[ids[c]] : 0.f;
      }
      float l[kExactBatch];
      exact_logits<NHV>(xrow, H, w, ids, n, bnd, l);
#pragma unroll
      for (int c = 0; c < kExactBatch; ++c)
        if (c < n && lane == pos[c]) vi = bias ? l[c] + bb[c] : l[c];
    }
    r = lane_rank(vi, ei, nc);
    wave_sync();
    if (lane < nc && r < top_k) cand[r] = Cand{vi, ei};
    wave_sync();
  } else {
    // many near-equal values: the same steps through LDS
    rank_sort(cand, sorted, nc);
    wave_sync();
    if (lane == 0) {
      int cs = 0;
      for (int i = 0; i < nc; ++i) {
        if (i > 0 && sorted[i - 1].v - sorted[i].v >= d2) cs = i;  // cs: start of i's cluster
        int e2 = i;
        while (e2 + 1 < nc && sorted[e2].v - sorted[e2 + 1].v < d2) ++e2;
        cand[i].e = e2 > cs && cs < top_k;
      }
    }
    wave_sync();
    for (int base = 0; base < nc; base += 64) {
      uint64_t f = ballot(base + lane < nc && cand[base + lane].e);
      while (f) {
        int ids[kExactBatch], pos[kExactBatch];
        double bnd[kExactBatch];
        int n = 0;
#pragma unroll
        for (int c = 0; c < kExactBatch; ++c) {
          pos[c] = 0;
          ids[c] = 0;
          bnd[c] = 0.0;
          if (c < exact_batch(NHV) && f) {
            pos[c] = base + __builtin_ctzll(f);
            f &= f - 1;
            ids[c] = sorted[pos[c]].e;
            bnd[c] = xnorm * p.wnorm[ids[c]] * (1.0 + 1e-6);
            n = c + 1;
          }
        }
        float l[kExactBatch];
        exact_logits_outlined<NHV>(xrow, H, w, ids, n, bnd, l);
        if (lane == 0) {
#pragma unroll
          for (int c = 0; c < kExactBatch; ++c)
            if (c < n) sorted[pos[c]].v = bias ? l[c] + bias[ids[c]] : l[c];
        }
      }
    }
    wave_sync();
    rank_sort(sorted, cand, nc);
    wave_sync();
  }
  // renormalised softmax over the top_k (cand[0..top_k) in slot order)
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
                 int H, int E, int top_k, const uint8_t* valid, int32_t* topk_idx, float* topk_w, float* gamma,
                 const RouteWorkspace& ws, hipStream_t stream) {
  if (T == 0) return JANUS_MOE_OK;
  Carver pc(const_cast<void*>(prep));
  RouterPrep p = carve_prep(pc, E, H);
  const int nslice = ceil_div(H, kSlice);
  const int Epad = ceil_div(E, 64) * 64;
  hipLaunchKernelGGL(router_logits_kernel, dim3(ceil_div(T, 64), Epad / 64, nslice), dim3(256), 0, stream, x, p, T, H,
                     E, Epad, ws.partial);
  JANUS_LAUNCH_CHECK("router_logits");
  const size_t smem = (size_t)4 * 2 * E * sizeof(Cand);
  const dim3 sg(ceil_div(T, 4)), sb(kSelThreads);
  const int nhv = ceil_div(H, 512), nj = ceil_div(E, 64);
#define JANUS_SELECT(NHV_, NJ_)                                                                                   \
  hipLaunchKernelGGL((router_select_kernel<NHV_, NJ_>), sg, sb, smem, stream, x, w, p, bias, wsg, T, H, E, Epad, \
                     nslice, top_k, ws.partial, valid, topk_idx, topk_w, gamma)
#define JANUS_SELECT_NJ(NHV_)       \
  if (nj <= 2)                      \
    JANUS_SELECT(NHV_, 2);          \
  else if (nj <= 4)                 \
    JANUS_SELECT(NHV_, 4);          \
  else                              \
    JANUS_SELECT(NHV_, 16);
  if (nhv <= 1) {
    JANUS_SELECT_NJ(1)
  } else if (nhv <= 2) {
    JANUS_SELECT_NJ(2)
  } else if (nhv <= 4) {
    JANUS_SELECT_NJ(4)
  } else {
    JANUS_SELECT_NJ(8)
  }
#undef JANUS_SELECT_NJ
#undef JANUS_SELECT
  JANUS_LAUNCH_CHECK("router_select");
  return JANUS_MOE_OK;
}

int check_route_sizes(int T, int H, int E, int top_k) {
  JANUS_REQUIRE(T >= 0 && H > 0 && H % 32 == 0 && H <= 512 * kMaxHv && E > 0 && E <= 64 * kMaxJ && E % 4 == 0 &&
                    top_k > 0 && top_k <= 64 && top_k <= E && (long)T * H * 2 < (1l << 31),
                JANUS_MOE_EINVAL, "router: unsupported sizes T=%d H=%d E=%d top_k=%d (need H %% 32 == 0, H <= %d, "
                "E %% 4 == 0, E <= %d, top_k <= min(64, E), T * H < 2^30)", T, H, E, top_k, 512 * kMaxHv, 64 * kMaxJ);
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
  return launch_route(x, w_router, prep, bias, w_shared_gate, T, H, E, top_k, nullptr, topk_idx, topk_w, gamma, r,
                      (hipStream_t)stream);
}
