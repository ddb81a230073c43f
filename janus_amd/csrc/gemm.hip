// Grouped W4A16 GEMMs for gfx950: int4 group-128 weights decoded to bf16 in registers, bf16 MFMA with fp32
// accumulation. The semantics are those of the reference's per-tile kernel (janus/moe_w4a16.py:36-86): a tile is one
// expert times a run of its rows; the gate_up launch fuses silu(gate) * up into its epilogue (:83), the down launch
// scales by the routing weight (:84-85). Unlike the reference's bf16 y buffer and bf16 reshape-sum (:140), each
// weighted expert output is kept in fp32 in a per-token slot and a combine pass sums a token's slots in a fixed order
// and rounds once: the result is deterministic and carries no intermediate bf16 rounding.
//
// Work decomposition. A workgroup (4 waves) takes one chunk (up to 96 rows of one expert, or 96 consecutive tokens of
// the shared expert) and one column slab. Each wave owns 4 MFMA column blocks of 16 weight rows: it streams their int4
// words from HBM into a 3-deep register ring (one 16-byte load per lane per 128 k), decodes each word once and
// multiplies it against all of the chunk's rows. The activation rows of each 128-wide k stage go global -> LDS by
// 16-byte direct loads into a 3-slot ring shared by the 4 waves, so loads run two stages ahead of the MFMAs without
// holding registers. v_mfma_f32_16x16x32_bf16 takes the weights as its first operand: a lane's accumulator holds 4
// consecutive output columns of one row. Workgroup ids are dealt to the 8 XCDs round-robin; the slabs of one chunk
// get ids that land on the same XCD, so the chunk's activation rows come from that XCD's L2 after the first slab.
#include <type_traits>

#include "gemm.h"

namespace janus {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kColBlocks = 4;
constexpr int KS = 128;                                      // k per pipeline stage: one scale group
constexpr int kStages = 3;                                   // ring depth: loads run two stages ahead
constexpr int kRowBytes = KS * 2;                            // one activation row of a stage (bf16)
constexpr int kSlotBytes = kChunkRows * kRowBytes;           // one LDS ring slot
constexpr int kLoadsPerStage = kRowBlocks + 2 * kColBlocks;  // per wave: activation rounds, weight words, scales

enum { kGateUp = 0, kDown = 1 };

template <int V>
using Slot = std::integral_constant<int, V>;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Weight words and scales are loaded with inline asm, outside the compiler's load tracking (which, across the ring's
// loop, would wait for every outstanding load before each use). The stage's registers are then tied to the explicit
// vmcnt wait that retires their loads, so no use can be scheduled ahead of it.
__device__ __forceinline__ u32x4 load_words_nt(const u32x4* ptr) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(v) : "v"(ptr) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t load_u16(const uint16_t* ptr) {
  uint32_t v;
  asm volatile("global_load_ushort %0, %1, off" : "=v"(v) : "v"(ptr) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void wait_vmcnt_bind(u32x4 (&w)[4], uint32_t (&s)[4]) {
  asm volatile("s_waitcnt vmcnt(%8)"
               : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(s[0]), "+v"(s[1]), "+v"(s[2]), "+v"(s[3])
               : "n"(N)
               : "memory");
}

// One int32 word of 8 int4 weights sharing the bf16 scale `sb` -> the bf16 MFMA operand in k order 0..7.
// t = 0x4300 | (nibble ^ 8) read as bf16 is exactly 128 + (q + 8), q the two's-complement nibble. v_dot2_f32_bf16
// with the scale in one half of the other operand and 0 in the other half gives (q + 136) * s - 136 * s, every step
// exact in fp32, i.e. q * s exactly; the conversion to bf16 rounds it once to nearest even: bf16(q * s).
__device__ __forceinline__ bf16x8 decode8(uint32_t w, uint32_t sb) {
  const bf16x2 s_lo = __builtin_bit_cast(bf16x2, sb);
  const bf16x2 s_hi = __builtin_bit_cast(bf16x2, sb << 16);
  const float c = -136.0f * __uint_as_float(sb << 16);
  const bf16x2 t0 = __builtin_bit_cast(bf16x2, (w & 0x000F000Fu) ^ 0x43084308u);
  const bf16x2 t1 = __builtin_bit_cast(bf16x2, ((w >> 4) & 0x000F000Fu) ^ 0x43084308u);
  const bf16x2 t2 = __builtin_bit_cast(bf16x2, ((w >> 8) & 0x000F000Fu) ^ 0x43084308u);
  const bf16x2 t3 = __builtin_bit_cast(bf16x2, ((w >> 12) & 0x000F000Fu) ^ 0x43084308u);
  bf16x8 r;
  r[0] = static_cast<__bf16>(__builtin_amdgcn_fdot2_f32_bf16(t0, s_lo, c, false));
  r[1] = static_cast<__bf16>(__builtin_amdgcn_fdot2_f32_bf16(t1, s_lo, c, false));
  r[2] = static_cast<__bf16>(__builtin_amdgcn_fdot2_f32_bf16(t2, s_lo, c, false));
  r[3] = static_cast<__bf16>(__builtin_amdgcn_fdot2_f32_bf16(t3, s_lo, c, false));
  r[4] = static_cast<__bf16>(__builtin_amdgcn_fdot2_f32_bf16(t0, s_hi, c, false));
  r[5] = static_cast<__bf16>(__builtin_amdgcn_fdot2_f32_bf16(t1, s_hi, c, false));
  r[6] = static_cast<__bf16>(__builtin_amdgcn_fdot2_f32_bf16(t2, s_hi, c, false));
  r[7] = static_cast<__bf16>(__builtin_amdgcn_fdot2_f32_bf16(t3, s_hi, c, false));
  return r;
}

template <int MODE>
__global__ void __launch_bounds__(kThreads) w4a16_gemm_kernel(const GemmParams p) {
  // LDS ring of activation tiles, [stage][row][16-byte chunk] with chunk position = chunk ^ (row & 15): the 16 lanes of
  // a fragment read (same chunk, 16 rows) hit 16 different bank groups.
  __shared__ __attribute__((aligned(16))) unsigned char lds[kStages * kSlotBytes];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int g = lane >> 4, nl = lane & 15;

  // ---- work item: chunk c, column slab ----
  const int xcd = blockIdx.x & 7, within = blockIdx.x >> 3;
  const int c = (within / p.nslab) * 8 + xcd;
  const int slab = within % p.nslab;
  if (c >= p.n_shared_chunks + p.max_chunks) return;
  const bool shared = c < p.n_shared_chunks;
  int pos0, rows, N, K;
  const int32_t* wq;
  const uint16_t* wsc;
  if (shared) {
    pos0 = c * kChunkRows;
    rows = min(kChunkRows, p.T - pos0);
    wq = p.q_sh;
    wsc = p.s_sh;
    N = p.N_sh;
    K = p.K_sh;
  } else {
    const int r = c - p.n_shared_chunks;
    if (r >= *p.num_chunks) return;
    const int4 ch = p.chunks[r];
    pos0 = ch.y;
    rows = ch.z;
    N = p.N;
    K = p.K;
    wq = p.q + (long)ch.x * N * (K / 8);
    wsc = p.s + (long)ch.x * N * (K / 128);
  }
  constexpr int kWaveCols = (MODE == kGateUp) ? 32 : 64;  // h columns (gate_up) or output columns (down)
  const int out_cols = (MODE == kGateUp) ? N / 2 : N;
  if (slab * kWaveCols * kWaves >= out_cols) return;
  const int col0 = slab * kWaveCols * kWaves + wave * kWaveCols;
  const bool active = col0 < out_cols;
  const int nrb = (rows + 15) / 16;

  // ---- activation rows this lane loads: round r covers rows 16r..16r+15, this wave rows 16r + 4w + (lane >> 4) ----
  const uint16_t* asrc[kRowBlocks];
#pragma unroll
  for (int r = 0; r < kRowBlocks; ++r) {
    const int row = 16 * r + 4 * wave + (lane >> 4);
    const int rr = row < rows ? row : 0;  // padding rows re-read row 0: finite values, results discarded
    const uint16_t* base;
    if (MODE == kGateUp) {
      const int tok = shared ? pos0 + rr : p.sorted_ids[pos0 + rr] / p.topk;
      base = p.a + (long)tok * K;
    } else {
      base = shared ? p.a_sh + (long)(pos0 + rr) * K : p.a + (long)(pos0 + rr) * K;
    }
    asrc[r] = base + (((lane & 15) ^ (row & 15)) * 8);
  }

  // ---- weight rows of this lane, one per column block (an idle wave reads row 0 so every wave issues the same
  // number of loads per stage, which the vmcnt waits below count on) ----
  const u32x4* wrow[kColBlocks];
  const uint16_t* srow[kColBlocks];
#pragma unroll
  for (int cb = 0; cb < kColBlocks; ++cb) {
    int n;
    if (MODE == kGateUp)
      n = (cb < 2) ? col0 + 16 * cb + nl : N / 2 + col0 + 16 * (cb - 2) + nl;
    else
      n = col0 + 16 * cb + nl;
    if (!active) n = 0;
    wrow[cb] = reinterpret_cast<const u32x4*>(wq + (long)n * (K / 8)) + g;
    srow[cb] = wsc + (long)n * (K / 128);
  }

  f32x4 acc[kRowBlocks][kColBlocks];
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
    for (int cb = 0; cb < kColBlocks; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nkb = K / KS;
  u32x4 bw[kStages][kColBlocks];
  uint32_t sc[kStages][kColBlocks];

  auto issue = [&](auto slot_c, int kb) {
    constexpr int slot = decltype(slot_c)::value;
    unsigned char* dst = lds + slot * kSlotBytes + 4 * wave * kRowBytes;
#pragma unroll
    for (int r = 0; r < kRowBlocks; ++r)
      __builtin_amdgcn_global_load_lds(asrc[r] + kb * KS, dst + 16 * r * kRowBytes, 16, 0, 0);
#pragma unroll
    for (int cb = 0; cb < kColBlocks; ++cb) {
      bw[slot][cb] = load_words_nt(wrow[cb] + kb * (KS / 32));
      sc[slot][cb] = load_u16(srow[cb] + kb);
    }
  };
  auto compute = [&](auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const unsigned char* base = lds + slot * kSlotBytes;
#pragma unroll
    for (int t = 0; t < KS / 32; ++t) {
      bf16x8 bfrag[kColBlocks];
#pragma unroll
      for (int cb = 0; cb < kColBlocks; ++cb) bfrag[cb] = decode8(bw[slot][cb][t], sc[slot][cb]);
#pragma unroll
      for (int rb = 0; rb < kRowBlocks; ++rb) {
        if (rb < nrb) {
          const bf16x8 afrag = *reinterpret_cast<const bf16x8*>(base + (16 * rb + nl) * kRowBytes +
                                                                ((4 * g + t) ^ nl) * 16);
#pragma unroll
          for (int cb = 0; cb < kColBlocks; ++cb)
            acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfrag[cb], afrag, acc[rb][cb], 0, 0, 0);
        }
      }
    }
  };
  // Stage kb lives in ring slot kb % 3. Its loads are complete once at most one later stage's loads are outstanding;
  // the barrier then publishes the LDS tile and retires every wave's reads of slot (kb + 2) % 3 (stage kb - 1), which
  // the following issue overwrites.
  auto step = [&](auto slot_c, int kb) {
    constexpr int slot = decltype(slot_c)::value;
    if (kb + 1 < nkb)
      wait_vmcnt_bind<kLoadsPerStage>(bw[slot], sc[slot]);
    else
      wait_vmcnt_bind<0>(bw[slot], sc[slot]);
    __builtin_amdgcn_s_barrier();
    if (kb + 2 < nkb) issue(Slot<(slot + 2) % kStages>{}, kb + 2);
    if (active) compute(slot_c);
  };

  issue(Slot<0>{}, 0);
  if (nkb > 1) issue(Slot<1>{}, 1);
  for (int kb = 0; kb < nkb; kb += kStages) {
    step(Slot<0>{}, kb);
    if (kb + 1 >= nkb) break;
    step(Slot<1>{}, kb + 1);
    if (kb + 2 >= nkb) break;
    step(Slot<2>{}, kb + 2);
  }
  if (!active) return;

  // ---- epilogue: lane holds rows 16 rb + nl, columns 16 cb + 4 g + i ----
  if (MODE == kGateUp) {
    uint16_t* hbase = shared ? p.h_sh : p.h;
    const int hw = N / 2;
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb) {
      const int m = rb * 16 + nl;
      if (rb >= nrb || m >= rows) continue;
      uint16_t* hrow = hbase + (long)(pos0 + m) * hw;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        float hv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gv = acc[rb][cb][i], uv = acc[rb][cb + 2][i];
          hv[i] = gv / (1.0f + __expf(-gv)) * uv;
        }
        uint2 st;
        st.x = pack_bf16x2(hv[0], hv[1]);
        st.y = pack_bf16x2(hv[2], hv[3]);
        *reinterpret_cast<uint2*>(hrow + col0 + 16 * cb + 4 * g) = st;
      }
    }
  } else {
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb) {
      const int m = rb * 16 + nl;
      if (rb >= nrb || m >= rows) continue;
      int tok, slot;
      float wt;
      if (shared) {
        tok = pos0 + m;
        slot = p.topk;
        wt = p.gamma ? p.gamma[tok] : 1.0f;
      } else {
        const int id = p.sorted_ids[pos0 + m];
        tok = id / p.topk;
        slot = id - tok * p.topk;
        wt = p.route_w[id];
      }
      float* orow = p.slots + ((long)tok * p.nslots + slot) * N + col0 + 4 * g;
#pragma unroll
      for (int cb = 0; cb < kColBlocks; ++cb)
        *reinterpret_cast<float4*>(orow + 16 * cb) =
            make_float4(wt * acc[rb][cb][0], wt * acc[rb][cb][1], wt * acc[rb][cb][2], wt * acc[rb][cb][3]);
    }
  }
}

// out[t, n] = bf16(sum_j slots[t, j, n]), four columns per thread, slots summed in order.
__global__ void combine_kernel(const float4* __restrict__ slots, int nslots, uint2* __restrict__ out, int T, int H4) {
  const long n = (long)T * H4;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long t = i / H4, col = i - t * H4;
    const float4* src = slots + t * nslots * H4 + col;
    float4 s = src[0];
    for (int j = 1; j < nslots; ++j) {
      const float4 v = src[(long)j * H4];
      s.x += v.x;
      s.y += v.y;
      s.z += v.z;
      s.w += v.w;
    }
    out[i] = make_uint2(pack_bf16x2(s.x, s.y), pack_bf16x2(s.z, s.w));
  }
}

// bf16 weights of an int4 group-128 matrix [rows, K]: the decode the GEMMs use, written out (one word per thread).
__global__ void dequant_kernel(const uint32_t* __restrict__ q, const uint16_t* __restrict__ s, long rows, int K,
                               bf16x8* __restrict__ out) {
  const long words = rows * (K / 8);
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (long)gridDim.x * blockDim.x) {
    const long r = i / (K / 8);
    const int j = (int)(i % (K / 8));
    const uint32_t sb = s[r * (K / 128) + (j * 8) / 128];
    bf16x8 v = decode8(q[i], sb);
    if (sb & 0x8000u) {  // 0 * (negative scale) is -0 in IEEE arithmetic; the decode's difference gives +0
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (__builtin_bit_cast(uint16_t, v[e]) == 0) v[e] = __builtin_bit_cast(__bf16, (uint16_t)0x8000u);
    }
    out[i] = v;
  }
}

template <int MODE>
int launch_gemm(const GemmParams& p, hipStream_t stream) {
  const int total = p.n_shared_chunks + p.max_chunks;
  if (total == 0) return JANUS_MOE_OK;
  const long grid = (long)ceil_div(total, 8) * 8 * p.nslab;
  JANUS_REQUIRE(grid < (1l << 31), JANUS_MOE_EINVAL, "grouped GEMM grid too large");
  hipLaunchKernelGGL((w4a16_gemm_kernel<MODE>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p);
  JANUS_LAUNCH_CHECK(MODE == kGateUp ? "w4a16 gate_up" : "w4a16 down");
  return JANUS_MOE_OK;
}

}  // namespace

int launch_gate_up(const GemmParams& p, hipStream_t stream) { return launch_gemm<kGateUp>(p, stream); }
int launch_down(const GemmParams& p, hipStream_t stream) { return launch_gemm<kDown>(p, stream); }

int launch_combine(const float* slots, int nslots, uint16_t* out, int T, int H, hipStream_t stream) {
  const long n4 = (long)T * (H / 4);
  if (n4 == 0) return JANUS_MOE_OK;
  long blocks = (n4 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, reinterpret_cast<const float4*>(slots),
                     nslots, reinterpret_cast<uint2*>(out), T, H / 4);
  JANUS_LAUNCH_CHECK("combine");
  return JANUS_MOE_OK;
}

int launch_dequant(const int32_t* q, const uint16_t* s, long rows, int K, uint16_t* out, hipStream_t stream) {
  const long words = rows * (K / 8);
  if (words == 0) return JANUS_MOE_OK;
  long blocks = (words + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, reinterpret_cast<const uint32_t*>(q), s,
                     rows, K, reinterpret_cast<bf16x8*>(out));
  JANUS_LAUNCH_CHECK("dequant");
  return JANUS_MOE_OK;
}

}  // namespace janus
