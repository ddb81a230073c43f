// Router on gfx950: the softmax / top-k / renormalise of Qwen3_5MoeTopKRouter.forward
// (transformers models/qwen3_5_moe/modeling_qwen3_5_moe.py:768-776) with a bit-exact selection rule:
//   logit(t, e) = fp32 round-to-nearest-even of the exact dot product x[t] . w[e] (+ bias[e] in fp32);
//   the top_k largest logits, ties to the lower expert id, in descending slot order.
//
// Two launches, no host sync:
//   router_logits  approximate logits for every (token, expert): bf16 MFMA over a two-plane split of the fp32 weight
//                  (w = hi + mid + r, |r| <= 2^-16 |w|) with fp32 accumulation. A workgroup takes 16, 32 or 64 tokens
//                  against 256 experts (so x is read from memory once) over one k range; the k ranges' partial sums go
//                  to memory, and so do the x statistics the selection needs (||x||^2 and x . w_shared_gate).
//   router_select  one wave per token: the candidate set {e : approx_e >= approx_(k) - 2 delta_t} provably contains the
//                  top_k, where delta_t >= |approx - exact| (Cauchy-Schwarz on the split residual plus an allowance for
//                  fp32 accumulation). Only candidates in a cluster of approximate values no further apart than
//                  2 delta that reaches into the top_k need their exact logit: an fp64 dot product whose error bound
//                  decides the fp32 rounding, or, within that bound of a rounding midpoint, a double-double sum.
// The routing weights are the renormalised softmax of the selected values: exact logits where a cluster was resolved,
// approximate ones elsewhere, each within delta_t of the exact logit, so a weight is within a factor exp(+-2 delta_t)
// of the one the exact logits give (delta_t is about 1e-5 ||x|| ||w|| as a worst case; the observed differences are
// at the fp32 rounding level).
#include "router.h"

#include <type_traits>

namespace janus {
namespace {

constexpr int kSelThreads = 256;  // 4 tokens per select workgroup
constexpr int kMaxHv = 8;         // 16-byte x vectors per lane in the exact path (H <= 4096)
constexpr int kMaxH = 512 * kMaxHv;
constexpr int kGroupE = 256;      // experts per logits workgroup: 4 waves x 4 blocks of 16
constexpr int kNeb = 4;           // 16-expert blocks per wave
constexpr int kMaxSplit = 16;     // k ranges per logit (partial sums)
constexpr int kAhead = 2;         // k-steps of weight fragments in flight per wave
constexpr uint32_t kOutside = 0x80000000u;  // a buffer offset past every buffer here: the load returns zeros

// Accumulation allowance, relative to ||x|| ||w||. A block is one MFMA chain over two k-steps (hi plane, mid plane,
// hi, mid: 128 products), so a product passes through at most 127 roundings in its block, then the block additions
// of its x tile (tile_k / 64), the tile additions and the k-range additions; the launch plan keeps those three
// together at most 19, so at most 146 roundings of at most 2^-23 relative (truncating arithmetic assumed):
// 146 * 2^-23 of sum |x (hi + mid)| <= 146 * 2^-23 * (1 + 2^-8) ||x|| ||w|| = 1.747e-5 ||x|| ||w||. The allowance
// 1.1796875 * 2^-16 = 1.800e-5 leaves 5.3e-7 for the final fp32 rounding of the exact logit (2^-24 relative).
constexpr double kAllowance = 0x1.2ep-16;
constexpr int kMaxRoundingSteps = 19;

// The two bf16 planes are stored in MFMA fragment order: block (b, s) of 1 KB holds rows 16b .. 16b+15, k 32s ..
// 32s+31, lane l = 16g + i of a 16x16x32 A operand at bytes 16l .. 16l+15 (row 16b + i, k 32s + 8g .. + 7), so a
// wave loads one fragment with one contiguous 1 KB read. Rows past E are zeros.
__host__ __device__ constexpr int eblocks(int E) { return (E + 15) / 16; }
struct RouterPrep {
  uint16_t* hi;      // [ceil(E/16), H/32, 64, 8] bf16
  uint16_t* mid;     // [ceil(E/16), H/32, 64, 8] bf16
  double* wnorm;     // [E] ||w_e||_2
  double* resnorm;   // [E] ||w_e - hi_e - mid_e||_2
  double* meta;      // [0] max_e resnorm, [1] max_e wnorm
};

RouterPrep carve_prep(Carver& c, int E, int H) {
  RouterPrep p;
  p.hi = c.take<uint16_t>((size_t)eblocks(E) * 16 * H);
  p.mid = c.take<uint16_t>((size_t)eblocks(E) * 16 * H);
  p.wnorm = c.take<double>(E);
  p.resnorm = c.take<double>(E);
  p.meta = c.take<double>(2);
  return p;
}

// Launch shape of both kernels, a function of the sizes only (the workspace size query uses it too).
struct RoutePlan {
  int mt;      // 16-token blocks per logits workgroup
  int sub;     // k of one x tile in LDS (128, 256 or 512)
  int nsub;    // x tiles per workgroup
  int kr;      // k range per workgroup (a multiple of 128)
  int nsplit;  // k ranges, = partial sums per logit
  int nj;      // experts per lane in router_select (2, 4 or 16)
  int epad;    // row stride of the partial sums, 64 * nj
};

RoutePlan route_plan(int T, int H, int E) {
  RoutePlan q;
  q.nj = E <= 128 ? 2 : E <= 256 ? 4 : 16;
  q.epad = 64 * q.nj;
  // Token tile against k split: the weights stream once per token tile (fewer, larger tiles), the partial sums go
  // through memory once per k range (fewer ranges); enough workgroups to cover the CUs decides between them. Measured
  // on MI355X at H = 2048, E = 256: 32-token tiles x 4 ranges at T = 2048, 64 x 4 at T = 4096, 64 x 1 at T = 16384.
  q.mt = T >= 4096 ? 4 : T >= 192 ? 2 : 1;
  const int tiles = ceil_div(T > 0 ? T : 1, 16 * q.mt), groups = ceil_div(E, kGroupE);
  // enough workgroups to cover the CUs once, each k range at least 128 wide
  int ns = 1;
  while (ns < kMaxSplit && tiles * groups * ns < 256 && ceil_div(H, 2 * ns) >= 128) ns *= 2;
  q.kr = ceil_div(ceil_div(H, ns), 128) * 128;
  q.nsplit = ceil_div(H, q.kr);
  q.sub = q.kr <= 128 ? 128 : q.kr <= 256 ? 256 : 512;
  q.nsub = ceil_div(q.kr, q.sub);
  return q;
}

// Orders this wave's LDS traffic: a wave's LDS operations execute in program order, so keeping the compiler from
// moving accesses across this point is enough for lanes to see each other's writes.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}


__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_down(v, off);
  return __shfl(v, 0);
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// ---- prepare: split rows, norms -------------------------------------------------------------------------------
// One workgroup per row of the padded planes (rows past E get zeros and no norms).
__global__ void __launch_bounds__(256) router_split_kernel(const float* __restrict__ w, int E, int H, RouterPrep p) {
  const int e = blockIdx.x;
  __shared__ double red[2][256];
  double r2 = 0.0, w2 = 0.0;
  for (int h = threadIdx.x; h < H; h += 256) {
    const float v = e < E ? w[(long)e * H + h] : 0.f;
    const __bf16 hi = static_cast<__bf16>(v);
    const float r1 = v - static_cast<float>(hi);
    const __bf16 mid = static_cast<__bf16>(r1);
    const float r2f = r1 - static_cast<float>(mid);
    const long at = (((long)(e >> 4) * (H / 32) + (h >> 5)) * 64 + ((h >> 3) & 3) * 16 + (e & 15)) * 8 + (h & 7);
    p.hi[at] = __builtin_bit_cast(uint16_t, hi);
    p.mid[at] = __builtin_bit_cast(uint16_t, mid);
    r2 += (double)r2f * (double)r2f;
    w2 += (double)v * (double)v;
  }
  if (e >= E) return;  // uniform: no barrier skipped by part of the workgroup
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
// grid (nsplit, ceil(T / 16MT), ceil(E / 256)), 4 waves. Workgroup (z, y, g): k range [z kr, min((z + 1) kr, H)),
// tokens 16MT y .. +16MT-1, experts 256 g .. +255. The k range varies fastest, so consecutive workgroups (which go to
// different XCDs in turn) share token tiles and each XCD's L2 holds the weights of fewer ranges. Wave w owns the
// expert blocks 256 g + 16 (w + 4i), i < 4, for every token of the tile. The x rows of the range go through LDS in tiles of SUB k (two alternating buffers when
// there are several); each wave streams its expert rows of both weight planes from memory into registers, kAhead
// k-steps ahead. Out-of-range rows and k read as zeros (buffer loads past the end), and zeros add nothing.
//
// Every two k-steps of 32 form a fresh block per (expert block, token block): one MFMA chain from zero over both
// steps' hi and mid planes, which VALU adds to the tile's running sum (the rounding count is the allowance above).
// Each wave w < MT also adds up ||x||^2 and x . w_shared_gate of the token rows 16w .. 16w+15 with two more MFMA
// chains per step: x against itself (the diagonal of the Gram block) and the gate row, replicated over the 16 rows
// of an A operand, against x. The squares are exact and their fp32 sum is within 2^-11 relative.
template <int MT, int SUB, bool MULTI>
__global__ void __launch_bounds__(256, 1) router_logits_kernel(const uint16_t* __restrict__ x, RouterPrep p,
                                                             const uint16_t* __restrict__ wsg, int T, int H, int E,
                                                             int epad, int kr, int nsub, float* __restrict__ partial,
                                                             float2* __restrict__ xstat) {
  constexpr int kRows = 16 * MT, kRowBytes = 2 * SUB, kTileBytes = kRows * kRowBytes;
  constexpr int kSteps = SUB / 32;             // k-steps per x tile
  constexpr int kCpr = SUB / 8;                // 16-byte chunks per row
  constexpr int kDma = kTileBytes / 1024 / 4;  // 1 KB buffer-to-LDS loads per wave per tile
  static_assert(kSteps % kAhead == 0 && (!MULTI || kSteps > kAhead), "x tile vs weight pipeline");
  constexpr int kOutStride = 4 * kGroupE + 16;  // bytes per token row of the output tile (shifted 4 banks a row)
  constexpr int kXsBytes = (MULTI ? 2 : 1) * kTileBytes > kRows * kOutStride ? (MULTI ? 2 : 1) * kTileBytes
                                                                               : kRows * kOutStride;
  __shared__ __attribute__((aligned(1024))) unsigned char xs[kXsBytes];  // x tiles, then the output tile
  __shared__ __attribute__((aligned(1024))) unsigned char gs[2 * kMaxH];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, nl = lane & 15;
  const int z = blockIdx.x, t0 = blockIdx.y * kRows, e0 = blockIdx.z * kGroupE;
  const int k0 = z * kr, kend = min(k0 + kr, H);
  const bool stats = blockIdx.z == 0;  // one expert group writes the x statistics
  const bool gate = stats && wsg != nullptr;
  const int nsteps = nsub * kSteps;

  // x tile sb of the range into buffer buf: row r's chunk c (8 k) sits at chunk position c ^ (r & 15). One load
  // fills 1 KB of the tile (lane l writes bytes 16 l .. 16 l + 15 of it), 64 / kCpr rows.
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), (short)0, (int)((long)T * H * 2), 0x00020000);
  auto issue_x = [&](int sb, int buf) __attribute__((always_inline)) {
    unsigned char* base = xs + buf * kTileBytes;
#pragma unroll
    for (int i = 0; i < kDma; ++i) {
      const int piece = wave * kDma + i;
      const int r = piece * (64 / kCpr) + lane / kCpr, c = (lane % kCpr) ^ (r & 15);
      const int k = k0 + sb * SUB + 8 * c, t = t0 + r;
      const uint32_t off = (t < T && k < kend) ? (uint32_t)(((long)t * H + k) * 2) : kOutside;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (JANUS_LDS void*)(base + piece * 1024), 16, off, 0, 0, 0);
    }
  };
  issue_x(0, 0);
  if (gate && wave == 0) {  // the gate row over the range, into gs
    const __amdgpu_buffer_rsrc_t gr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(wsg), (short)0, H * 2, 0x00020000);
    for (int i = 0; i < (kr + 511) / 512; ++i) {
      const int k = k0 + 512 * i + 8 * lane;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(gr, (JANUS_LDS void*)(gs + 1024 * i), 16,
                                               k < kend ? (uint32_t)(k * 2) : kOutside, 0, 0, 0);
    }
  }
  asm volatile("" ::: "memory");  // the loads into LDS issue before the weight loads below

  // this lane's weight fragments: expert block (e0 / 16) + w + 4i, from the range's first k-step on
  const int plane_bytes = eblocks(E) * 16 * H * 2;
  const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(p.hi, (short)0, plane_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t mr = __builtin_amdgcn_make_buffer_rsrc(p.mid, (short)0, plane_bytes, 0x00020000);
  uint32_t woff[kNeb];
#pragma unroll
  for (int i = 0; i < kNeb; ++i) {
    const int b = e0 / 16 + wave + 4 * i;
    woff[i] = b < eblocks(E) ? (uint32_t)(((b * (H / 32) + k0 / 32) * 64 + lane) * 16) : kOutside;
  }
  u32x4 wf[kAhead][kNeb][2];
  // a k-step past H loads the range's last real step again (finite weights against zero x): the buffer offset stays in
  // range through the VGPR part alone
  const int last_step = H / 32 - 1 - k0 / 32;
  auto load_w = [&](int slot, int step_in) __attribute__((always_inline)) {
    const int step = step_in < last_step ? step_in : last_step;
#pragma unroll
    for (int i = 0; i < kNeb; ++i) {
      wf[slot][i][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(hr, woff[i], 1024 * step, 0));
      wf[slot][i][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(mr, woff[i], 1024 * step, 0));
    }
  };
#pragma unroll
  for (int s = 0; s < kAhead; ++s) load_w(s, s);
  // A wave's loads complete in issue order: once step 0's weights are here, so are its loads into LDS. The empty asm
  // makes the compiler wait for them (with an exact count) before the barrier.
  {
    const u32x4 a = wf[0][0][0], b = wf[0][0][1];
    asm volatile("" ::"v"(a), "v"(b));
  }
  lds_barrier();

  static_assert(kAhead == 2, "a block is the two k-steps of one pass over the weight ring");
  f32x4 acc[kNeb][MT], tot[kNeb][MT];
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 sacc = zero4, gacc = zero4;  // Gram block of this wave's token rows; gate row . x
  for (int sb = 0; sb < (MULTI ? nsub : 1); ++sb) {
    const unsigned char* xt = xs + (MULTI ? (sb & 1) * kTileBytes : 0);
    if (MULTI && sb + 1 < nsub) {
      // the other buffer was last read in tile sb - 1, before the barrier that closed it
      issue_x(sb + 1, (sb + 1) & 1);
      asm volatile("" ::: "memory");
    }
#pragma unroll
    for (int i = 0; i < kNeb; ++i)
#pragma unroll
      for (int tb = 0; tb < MT; ++tb) acc[i][tb] = zero4;
#pragma unroll 1
    for (int s0 = 0; s0 < kSteps; s0 += kAhead) {
      f32x4 blk[kNeb][MT];
#pragma unroll
      for (int a = 0; a < kAhead; ++a) {
        const int ls = s0 + a, step = sb * kSteps + ls;
        bf16x8 xf[MT];
#pragma unroll
        for (int tb = 0; tb < MT; ++tb)
          xf[tb] = *reinterpret_cast<const bf16x8*>(xt + (16 * tb + nl) * kRowBytes + (((4 * ls + g) ^ nl) * 16));
        // every block's hi MFMA, then every block's mid MFMA: no MFMA waits for the one just issued
#pragma unroll
        for (int i = 0; i < kNeb; ++i)
#pragma unroll
          for (int tb = 0; tb < MT; ++tb)
            blk[i][tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[a][i][0]), xf[tb],
                                                                 a == 0 ? zero4 : blk[i][tb], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < kNeb; ++i)
#pragma unroll
          for (int tb = 0; tb < MT; ++tb)
            blk[i][tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[a][i][1]), xf[tb],
                                                                 blk[i][tb], 0, 0, 0);
        // x statistics of token rows 16 wave .. + 15 (every wave, without a branch; waves w >= MT have no rows)
        bf16x8 xw = xf[0];
#pragma unroll
        for (int tb = 1; tb < MT; ++tb) xw = wave == tb ? xf[tb] : xw;
        const bf16x8 gf = *reinterpret_cast<const bf16x8*>(gs + (sb * SUB + 32 * ls + 8 * g) * 2);
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xw, xw, sacc, 0, 0, 0);
        gacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(gf, xw, gacc, 0, 0, 0);
        // the next loads of this slot (past the last step: step kAhead - 1 again, unused)
        load_w(a, step + kAhead < nsteps ? step + kAhead : kAhead - 1);
        __builtin_amdgcn_sched_barrier(0);  // one k-step at a time
      }
#pragma unroll
      for (int i = 0; i < kNeb; ++i)
#pragma unroll
        for (int tb = 0; tb < MT; ++tb) acc[i][tb] += blk[i][tb];
    }
    if (MULTI) {
#pragma unroll
      for (int i = 0; i < kNeb; ++i)
#pragma unroll
        for (int tb = 0; tb < MT; ++tb) tot[i][tb] = sb == 0 ? acc[i][tb] : tot[i][tb] + acc[i][tb];
      // The loads issued after tile sb + 1's loads into LDS were consumed in this tile (kSteps > kAhead), so those
      // have completed; the barrier makes every wave's part visible and frees this tile's buffer.
      if (sb + 1 < nsub) lds_barrier();
    }
  }

  // The sums go to memory as whole rows: each wave writes its blocks into an LDS tile [token][expert] (over the x
  // tiles, which every wave is done with after the barrier), then each wave stores rows of up to 256 experts, lane l
  // experts 4l .. 4l + 3. Lane (g, nl) holds experts 16 (w + 4i) + 4g .. + 3 of token 16 tb + nl.
  lds_barrier();
#pragma unroll
  for (int i = 0; i < kNeb; ++i)
#pragma unroll
    for (int tb = 0; tb < MT; ++tb) {
      const f32x4 v = MULTI ? tot[i][tb] : acc[i][tb];
      *reinterpret_cast<float4*>(xs + (16 * tb + nl) * kOutStride + (16 * (wave + 4 * i) + 4 * g) * 4) =
          make_float4(v[0], v[1], v[2], v[3]);
    }
  lds_barrier();
#pragma unroll
  for (int r = wave; r < kRows; r += 4) {
    const int t = t0 + r, e = e0 + 4 * lane;
    if (t < T && e < E)  // non-temporal: read once, by the next kernel
      __builtin_nontemporal_store(*reinterpret_cast<const f32x4*>(xs + r * kOutStride + 16 * lane),
                                  reinterpret_cast<f32x4*>(partial + ((long)z * T + t) * epad + e));
  }
  // the Gram diagonal of row nl sits in lane (nl / 4, nl), element nl % 4; every lane's gacc holds its row's gate dot
  // (garbage without a gate row: gs unwritten, and the select kernel then ignores it)
  const int t = t0 + 16 * wave + nl;
  if (stats && wave < MT && g == (nl >> 2) && t < T) {
    const int r = nl & 3;
    const float ss = r == 0 ? sacc[0] : r == 1 ? sacc[1] : r == 2 ? sacc[2] : sacc[3];
    xstat[(long)z * T + t] = make_float2(ss, gacc[0]);
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
// dot product, in every lane. bound >= ||x|| ||w_c|| for every row.
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
__device__ __forceinline__ void load_xrow(const uint16_t* __restrict__ xrow, int H, XRow<NHV>& out) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < NHV; ++j) {
    const int h0 = 512 * j + 8 * lane;
    out.v[j] = h0 < H ? *reinterpret_cast<const uint4*>(xrow + h0) : make_uint4(0, 0, 0, 0);
  }
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
// accumulation of the same products (rare).
template <int NHV>
__device__ __forceinline__ float exact_logit_dd(XRow<NHV> x, const float* __restrict__ wrow, int H) {
  float wv[NHV][8];
  load_wrow<NHV>(wrow, H, true, wv);
  double hi = 0.0, lo = 0.0;
#pragma unroll
  for (int j = 0; j < NHV; ++j) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      double s2, e2;
      two_sum(hi, (double)xval(x, j, i) * (double)wv[j][i], s2, e2);
      hi = s2;
      lo += e2;
    }
    __builtin_amdgcn_sched_barrier(0);
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
                             int n, double bound, float (&out)[kExactBatch]) {
  float wv[kExactBatch][NHV][8];
#pragma unroll
  for (int c = 0; c < kExactBatch; ++c)
    if (c < exact_batch(NHV)) load_wrow<NHV>(w + (long)ids[c] * H, H, c < n, wv[c]);
  double v[kExactBatch];
#pragma unroll
  for (int c = 0; c < exact_batch(NHV); ++c) {
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < NHV; ++j) {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = fma((double)xval(x, j, i), (double)wv[c][j][i], acc);
      __builtin_amdgcn_sched_barrier(0);  // the fp64 operands of 8 products live at a time
    }
    v[c] = acc;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
    for (int c = 0; c < exact_batch(NHV); ++c) v[c] += __shfl_xor(v[c], off);
#pragma unroll
  for (int c = 0; c < exact_batch(NHV); ++c) v[c] = __shfl(v[c], 0);  // one value per wave: the branches below are uniform
  // |v - exact| <= (terms per lane + tree depth) * 2^-53 * sum|x w| <= that * ||x|| ||w||
  const double err = (double)(8 * NHV + 6) * 0x1p-53 * bound;
#pragma unroll
  for (int c = 0; c < exact_batch(NHV); ++c) {
    if (c >= n) break;
    const float r = (float)v[c];
    const double rd = (double)r;
    const double dn = 0.5 * (rd + (double)f32_next_down(r));
    const double up = 0.5 * (rd + (double)f32_next_up(r));
    out[c] = (v[c] - dn > err && up - v[c] > err) ? r : exact_logit_dd<NHV>(x, w + (long)ids[c] * H, H);
  }
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

// NJ consecutive floats at p (NJ = 2, 4 or 16; p aligned to NJ floats).
template <int NJ>
__device__ __forceinline__ void load_floats(const float* __restrict__ p, float (&out)[NJ]) {
  if constexpr (NJ == 2) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    out[0] = v.x; out[1] = v.y;
  } else {
#pragma unroll
    for (int q = 0; q < NJ / 4; ++q) {
      const float4 v = *reinterpret_cast<const float4*>(p + 4 * q);
      out[4 * q] = v.x; out[4 * q + 1] = v.y; out[4 * q + 2] = v.z; out[4 * q + 3] = v.w;
    }
  }
}

constexpr int kKeyLowBits = 16;  // low key bits the k-th value search leaves open (a lower bound is enough)

// One wave per token; lane l holds experts NJ l .. NJ l + NJ - 1. NHV: 16-byte x vectors per lane in the exact path.
template <int NHV, int NJ>
__global__ void __launch_bounds__(kSelThreads) router_select_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ w, RouterPrep p, const float* __restrict__ bias, int T,
    int H, int E, int epad, int nsplit, int top_k, double allowance, bool has_gate, const float* __restrict__ partial,
    const float2* __restrict__ xstat, const uint8_t* __restrict__ valid, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_w, float* __restrict__ gamma) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

  // The partial sums of this lane's experts, k range by k range in order, the x statistics and the bias. Every load
  // of a batch is issued before the first is used, and no branch separates a load from its use (a load whose result
  // feeds a branch-guarded sum waits for its own round trip): a batch is nsplit rounded up to a power of two (at most
  // 16, or 4 ranges at 16 experts a lane), a range past nsplit re-reads the batch's first and adds a zero.
  float av[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) av[j] = 0.f;
  const float* prow = partial + (long)t * epad + NJ * lane;
  const long zs = (long)T * epad;
  bool ok[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) ok[j] = NJ * lane + j < E;
  float bj[NJ];
  if constexpr (NJ <= 4) {
    // E % 4 == 0, so a lane's first expert in range means all of its experts are (the null case reads a dummy row)
    load_floats<NJ>(bias ? bias + (NJ * lane < E ? NJ * lane : 0) : prow, bj);
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j) bj[j] = bias ? bias[ok[j] ? NJ * lane + j : 0] : 0.f;
  }
  // lane z < nsplit loads range z's x statistics (a per-lane address: a vector load, in flight with the others)
  const float2 stl = xstat[(long)(lane < nsplit ? lane : 0) * T + t];
  auto gather = [&](auto kz_c) __attribute__((always_inline)) {
    constexpr int KZ = decltype(kz_c)::value;
    for (int z0 = 0; z0 < nsplit; z0 += KZ) {
      float pz[KZ][NJ];
#pragma unroll
      for (int q = 0; q < KZ; ++q) load_floats<NJ>(prow + (z0 + q < nsplit ? z0 + q : z0) * zs, pz[q]);
#pragma unroll
      for (int q = 0; q < KZ; ++q) {
        const bool on = z0 + q < nsplit;
#pragma unroll
        for (int j = 0; j < NJ; ++j) av[j] += on ? pz[q][j] : 0.f;
      }
    }
  };
  if (nsplit <= 1) {
    gather(std::integral_constant<int, 1>{});
  } else if (nsplit <= 2) {
    gather(std::integral_constant<int, 2>{});
  } else if (nsplit <= 4 || NJ > 4) {
    gather(std::integral_constant<int, 4>{});
  } else if (nsplit <= 8) {
    gather(std::integral_constant<int, 8>{});
  } else {
    gather(std::integral_constant<int, 16>{});
  }
  float ss = 0.f, gd = 0.f;
  for (int z = 0; z < nsplit; ++z) {
    ss += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(stl.x), z));
    gd += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(stl.y), z));
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) av[j] = ok[j] ? av[j] + (bias ? bj[j] : 0.f) : -__builtin_inff();

  if (has_gate && lane == 0 && gamma) gamma[t] = 1.0f / (1.0f + __expf(-gd));
  // ||x|| from the fp32 sum of squares (within 2^-11 relative: at most 2^12 roundings of at most 2^-23)
  const double xnorm = sqrt((double)ss * (1.0 + 0x1p-10));
  const double delta = xnorm * (p.meta[0] + allowance * p.meta[1]) + 1e-30;
  // d2 = 2 * max |approx - logit|: delta, plus with a bias the fp32 rounding of both bias additions (2^-24 of
  // either sum each), bounded with the largest |value| (and a margin for the first-order bound)
  double d2 = 2.0 * delta * (1.0 + 0x1p-20);
  if (bias) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) m = ok[j] ? fmaxf(m, __builtin_fabsf(av[j])) : m;
    d2 += 4.0 * 0x1p-24 * (double)wave_max_f32(m) * (1.0 + 0x1p-10) + 4.0 * 0x1p-24 * delta;
  }

  // A lower bound of the k-th largest approximate value: the k-th largest of the lanes' maxima (k distinct values are
  // at least that large), to kKeyLowBits of its order-preserving key by binary search over the high bits with one
  // ballot a step (the prefix found is that value's; the low bits are left zero).
  uint32_t key[NJ], kmax = 0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    key[j] = ok[j] ? f32_key(av[j]) : 0u;
    kmax = key[j] > kmax ? key[j] : kmax;
  }
  uint32_t tau = 0;
#pragma unroll
  for (int bit = 31; bit >= kKeyLowBits; --bit) {
    const uint32_t trial = tau | (1u << bit);
    if (__popcll(ballot(kmax >= trial)) >= top_k) tau = trial;
  }
  const double theta = (double)key_f32(tau) - d2;
  // candidates, compacted into LDS
  int nc = 0;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const bool pred = ok[j] && (double)av[j] >= theta;
    const uint64_t m = ballot(pred);
    if (pred) cand[nc + __popcll(m & below)] = Cand{av[j], NJ * lane + j};
    nc += __popcll(m);
  }
  wave_sync();
  const double bound = xnorm * p.meta[1] * (1.0 + 1e-6);  // >= ||x|| ||w_e|| for every expert

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
    // members of a cluster (adjacent gaps <= d2) that reaches into the top_k need their exact logit; the gaps are
    // exact in fp64
    const bool in = lane < nc;
    const float vp = __shfl_up(vi, 1);
    const uint64_t starts = ballot(in && (lane == 0 || (double)vp - (double)vi > d2));
    const uint64_t upto = (2ull << lane) - 1;            // bits 0..lane
    const int cs = 63 - __clzll(starts & upto);            // this lane's cluster start (bit 0 is always set)
    const uint64_t next = starts & ~upto;
    const int last = next ? __builtin_ctzll(next) - 1 : nc - 1;  // this lane's cluster end
    uint64_t f = ballot(in && last > cs && cs < top_k);
    if (f) {
      XRow<NHV> xrow;
      load_xrow<NHV>(x + (long)t * H, H, xrow);
      while (f) {
        int ids[kExactBatch], pos[kExactBatch];
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
        float bb[kExactBatch];  // issued with the rows' loads (an unused entry reads expert 0)
#pragma unroll
        for (int c = 0; c < kExactBatch; ++c) bb[c] = bias ? bias[ids[c]] : 0.f;
        float l[kExactBatch];
        exact_logits<NHV>(xrow, H, w, ids, n, bound, l);
#pragma unroll
        for (int c = 0; c < kExactBatch; ++c)
          if (c < n && lane == pos[c]) vi = bias ? l[c] + bb[c] : l[c];
      }
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
        if (i > 0 && (double)sorted[i - 1].v - (double)sorted[i].v > d2) cs = i;  // cs: start of i's cluster
        int e2 = i;
        while (e2 + 1 < nc && (double)sorted[e2].v - (double)sorted[e2 + 1].v <= d2) ++e2;
        cand[i].e = e2 > cs && cs < top_k;
      }
    }
    wave_sync();
    XRow<NHV> xrow;
    load_xrow<NHV>(x + (long)t * H, H, xrow);
    for (int base = 0; base < nc; base += 64) {
      uint64_t f = ballot(base + lane < nc && cand[base + lane].e);
      while (f) {
        int ids[kExactBatch], pos[kExactBatch];
        int n = 0;
#pragma unroll
        for (int c = 0; c < kExactBatch; ++c) {
          pos[c] = 0;
          ids[c] = 0;
          if (c < exact_batch(NHV) && f) {
            pos[c] = base + __builtin_ctzll(f);
            f &= f - 1;
            ids[c] = sorted[pos[c]].e;
            n = c + 1;
          }
        }
        float l[kExactBatch];
        exact_logits<NHV>(xrow, H, w, ids, n, bound, l);
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
  const RoutePlan q = route_plan(T, H, E);
  const size_t rows = (size_t)q.nsplit * (T > 0 ? T : 1);
  r.partial = c.take<float>(rows * q.epad);
  r.xstat = c.take<float2>(rows);
  return r;
}

int launch_route(const uint16_t* x, const float* w, const void* prep, const float* bias, const uint16_t* wsg, int T,
                 int H, int E, int top_k, const uint8_t* valid, int32_t* topk_idx, float* topk_w, float* gamma,
                 const RouteWorkspace& ws, hipStream_t stream) {
  if (T == 0) return JANUS_MOE_OK;
  Carver pc(const_cast<void*>(prep));
  RouterPrep p = carve_prep(pc, E, H);
  const RoutePlan q = route_plan(T, H, E);
  JANUS_REQUIRE(q.sub / 64 + q.nsub - 1 + q.nsplit - 1 <= kMaxRoundingSteps, JANUS_MOE_EINVAL,
                "router: plan for H=%d exceeds the accumulation allowance", H);
  const dim3 lg(q.nsplit, ceil_div(T, 16 * q.mt), ceil_div(E, kGroupE)), lb(256);
#define JANUS_LOGITS(MT_, SUB_, MULTI_)                                                                          \
  hipLaunchKernelGGL((router_logits_kernel<MT_, SUB_, MULTI_>), lg, lb, 0, stream, x, p, wsg, T, H, E, q.epad, q.kr, \
                     q.nsub, ws.partial, ws.xstat)
#define JANUS_LOGITS_SUB(MT_)       \
  if (q.nsub > 1)                   \
    JANUS_LOGITS(MT_, 512, true);   \
  else if (q.sub == 128)            \
    JANUS_LOGITS(MT_, 128, false);  \
  else if (q.sub == 256)            \
    JANUS_LOGITS(MT_, 256, false);  \
  else                              \
    JANUS_LOGITS(MT_, 512, false);
  if (q.mt == 1) {
    JANUS_LOGITS_SUB(1)
  } else if (q.mt == 2) {
    JANUS_LOGITS_SUB(2)
  } else {
    JANUS_LOGITS_SUB(4)
  }
#undef JANUS_LOGITS_SUB
#undef JANUS_LOGITS
  JANUS_LAUNCH_CHECK("router_logits");
  const size_t smem = (size_t)4 * 2 * E * sizeof(Cand);
  const dim3 sg(ceil_div(T, 4)), sb(kSelThreads);
  const int nhv = ceil_div(H, 512);
  const bool has_gate = wsg != nullptr;
#define JANUS_SELECT(NHV_, NJ_)                                                                                   \
  hipLaunchKernelGGL((router_select_kernel<NHV_, NJ_>), sg, sb, smem, stream, x, w, p, bias, T, H, E, q.epad,     \
                     q.nsplit, top_k, kAllowance, has_gate, ws.partial, ws.xstat,                                   \
                     valid, topk_idx, topk_w, gamma)
#define JANUS_SELECT_NJ(NHV_)       \
  if (q.nj == 2)                    \
    JANUS_SELECT(NHV_, 2);          \
  else if (q.nj == 4)               \
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
  JANUS_REQUIRE(T >= 0 && H > 0 && H % 32 == 0 && H <= kMaxH && E > 0 && E <= 64 * 16 && E % 4 == 0 &&
                    top_k > 0 && top_k <= 64 && top_k <= E && (long)T * H * 2 < (1l << 31),
                JANUS_MOE_EINVAL, "router: unsupported sizes T=%d H=%d E=%d top_k=%d (need H %% 32 == 0, H <= %d, "
                "E %% 4 == 0, E <= %d, top_k <= min(64, E), T * H < 2^30)", T, H, E, top_k, kMaxH, 64 * 16);
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
  JANUS_REQUIRE(E > 0 && H > 0 && H % 32 == 0, JANUS_MOE_EINVAL, "janus_moe_router_prepare: bad sizes E=%d H=%d", E, H);
  JANUS_REQUIRE(w_router && prep, JANUS_MOE_EINVAL, "janus_moe_router_prepare: null pointer");
  JANUS_REQUIRE(prep_bytes >= router_prep_bytes(E, H), JANUS_MOE_EWORKSPACE,
                "janus_moe_router_prepare: prep buffer %zu < %zu bytes", prep_bytes, router_prep_bytes(E, H));
  Carver pc(prep);
  RouterPrep p = carve_prep(pc, E, H);
  hipLaunchKernelGGL(router_split_kernel, dim3(eblocks(E) * 16), dim3(256), 0, (hipStream_t)stream, w_router, E, H, p);
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
