// Grouped W4A16 GEMMs for gfx950: int4 group-128 weights decoded to bf16 in registers, bf16 MFMA with fp32
// accumulation. The semantics are those of the reference's per-tile kernel (janus/moe_w4a16.py:36-86): a tile
// is one expert times a run of its rows; the gate_up launch fuses silu(gate) * up into its epilogue (:83), the down
// launch scales by the routing weight (:84-85) and, unlike the reference's bf16 y buffer and reshape-sum (:140),
// adds the fp32 product straight into an fp32 [T, H] accumulator, so the top-k combine is fp32 and rounds once.
//
// Work decomposition. A workgroup (4 waves) takes one chunk (up to 64 rows of one expert, or 64 consecutive tokens of
// the shared expert) and one column slab. The 64 activation rows of a 128- or 256-wide k super-block are staged in LDS
// (double-buffered) and shared by the 4 waves; each wave owns 4 MFMA column blocks of 16 weight rows, streams their
// int4 words straight from HBM into registers (one 16-byte load per lane per 128 k), decodes them once and multiplies
// them against all 64 rows. MFMA v_mfma_f32_16x16x32_bf16 takes the weights as its first operand, so a lane's
// accumulator holds 4 consecutive output columns of one row. Workgroup ids are laid out so that the slabs of one chunk
// land on the same XCD (ids are dealt to the 8 XCDs round-robin): the chunk's activation rows are then read from HBM
// once per XCD and from its L2 afterwards.
#include "gemm.h"

namespace janus {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kColBlocks = 4;
constexpr int kRowBlocks = kChunkRows / 16;

enum { kGateUp = 0, kDown = 1 };

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

template <int KS>
struct Stage {
  static constexpr int kWpl = KS / 32;           // weight words per lane per column block per super-block
  static constexpr int kVecs = kWpl / 4;          // 16-byte loads of them
  static constexpr int kLdsStride = KS + 8;       // bf16 per LDS row: consecutive rows shift by 4 banks
  static constexpr int kAVecs = KS / 4 / 8;       // 16-byte activation loads per thread per super-block
};

template <int MODE, int KS>
__global__ void __launch_bounds__(kThreads) w4a16_gemm_kernel(const GemmParams p) {
  using S = Stage<KS>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][kChunkRows * S::kLdsStride];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int g = lane >> 4, nl = lane & 15;

  // ---- work item: chunk c, column slab; the slabs of one chunk share an XCD ----
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

  // ---- activation row staged by this thread ----
  const int ar = tid >> 2, apart = tid & 3;
  const uint16_t* arow = nullptr;
  if (ar < rows) {
    if (MODE == kGateUp) {
      const int tok = shared ? pos0 + ar : p.sorted_ids[pos0 + ar] / p.topk;
      arow = p.a + (long)tok * K;
    } else {
      arow = shared ? p.a_sh + (long)(pos0 + ar) * K : p.a + (long)(pos0 + ar) * K;
    }
    arow += apart * (KS / 4);
  }

  // ---- weight rows of this lane (one per column block) ----
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
    wrow[cb] = reinterpret_cast<const u32x4*>(wq + (long)n * (K / 8)) + g * S::kVecs;
    srow[cb] = wsc + (long)n * (K / 128) + ((KS == 256) ? (g >> 1) : 0);
  }

  f32x4 acc[kRowBlocks][kColBlocks];
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
    for (int cb = 0; cb < kColBlocks; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nkb = K / KS;
  uint4 areg[S::kAVecs];
  u32x4 bcur[kColBlocks][S::kVecs], bnext[kColBlocks][S::kVecs];
  uint32_t scur[kColBlocks], snext[kColBlocks];

  auto load_a = [&](int kb) {
#pragma unroll
    for (int v = 0; v < S::kAVecs; ++v)
      areg[v] = arow ? reinterpret_cast<const uint4*>(arow + kb * KS)[v] : make_uint4(0, 0, 0, 0);
  };
  auto store_a = [&](int buf) {
    uint4* dst = reinterpret_cast<uint4*>(&lds[buf][ar * S::kLdsStride + apart * (KS / 4)]);
#pragma unroll
    for (int v = 0; v < S::kAVecs; ++v) dst[v] = areg[v];
  };
  auto load_b = [&](int kb, u32x4 (&bw)[kColBlocks][S::kVecs], uint32_t (&sc)[kColBlocks]) {
    if (!active) return;
#pragma unroll
    for (int cb = 0; cb < kColBlocks; ++cb) {
#pragma unroll
      for (int v = 0; v < S::kVecs; ++v) bw[cb][v] = __builtin_nontemporal_load(wrow[cb] + kb * (KS / 32) + v);
      sc[cb] = srow[cb][kb * (KS / 128)];
    }
  };
  auto compute = [&](int buf, const u32x4 (&bw)[kColBlocks][S::kVecs], const uint32_t (&sc)[kColBlocks]) {
    if (!active) return;
#pragma unroll
    for (int t = 0; t < S::kWpl; ++t) {
      bf16x8 bfrag[kColBlocks];
#pragma unroll
      for (int cb = 0; cb < kColBlocks; ++cb) {
        bfrag[cb] = decode8(bw[cb][t / 4][t % 4], sc[cb]);
      }
#pragma unroll
      for (int rb = 0; rb < kRowBlocks; ++rb) {
        const bf16x8 afrag =
            *reinterpret_cast<const bf16x8*>(&lds[buf][(rb * 16 + nl) * S::kLdsStride + (g * S::kWpl + t) * 8]);
#pragma unroll
        for (int cb = 0; cb < kColBlocks; ++cb)
          acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfrag[cb], afrag, acc[rb][cb], 0, 0, 0);
      }
    }
  };

  load_a(0);
  load_b(0, bcur, scur);
  store_a(0);
  __syncthreads();
  for (int kb = 0; kb < nkb; kb += 2) {
    const bool more1 = kb + 1 < nkb;
    if (more1) {
      load_a(kb + 1);
      load_b(kb + 1, bnext, snext);
    }
    compute(0, bcur, scur);
    if (more1) store_a(1);
    __syncthreads();
    if (!more1) break;
    const bool more2 = kb + 2 < nkb;
    if (more2) {
      load_a(kb + 2);
      load_b(kb + 2, bcur, scur);
    }
    compute(1, bnext, snext);
    if (more2) store_a(0);
    __syncthreads();
  }
  if (!active) return;

  // ---- epilogue: lane holds rows rb*16 + nl, columns 16*cb + 4*g + i ----
  if (MODE == kGateUp) {
    uint16_t* hbase = shared ? p.h_sh : p.h;
    const int hw = N / 2;
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb) {
      const int m = rb * 16 + nl;
      if (m >= rows) continue;
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
      if (m >= rows) continue;
      int tok;
      float wt;
      if (shared) {
        tok = pos0 + m;
        wt = p.gamma ? p.gamma[tok] : 1.0f;
      } else {
        const int id = p.sorted_ids[pos0 + m];
        tok = id / p.topk;
        wt = p.route_w[id];
      }
      float* orow = p.acc + (long)tok * N + col0 + 4 * g;
#pragma unroll
      for (int cb = 0; cb < kColBlocks; ++cb)
#pragma unroll
        for (int i = 0; i < 4; ++i) unsafeAtomicAdd(orow + 16 * cb + i, wt * acc[rb][cb][i]);
    }
  }
}

__global__ void finalize_kernel(const float4* __restrict__ acc, uint2* __restrict__ out, long n4) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (long)gridDim.x * blockDim.x) {
    const float4 v = acc[i];
    out[i] = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
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
  const bool has_sh = p.n_shared_chunks > 0;
  const int K = p.K, Ksh = has_sh ? p.K_sh : p.K;
  const int total = p.n_shared_chunks + p.max_chunks;
  if (total == 0) return JANUS_MOE_OK;
  const long grid = (long)ceil_div(total, 8) * 8 * p.nslab;
  JANUS_REQUIRE(grid < (1l << 31), JANUS_MOE_EINVAL, "grouped GEMM grid too large");
  // 128-wide k super-blocks: 225 registers per lane, two waves per SIMD (the 256-wide variant needs 273: one wave).
  (void)K;
  (void)Ksh;
  hipLaunchKernelGGL((w4a16_gemm_kernel<MODE, 128>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p);
  JANUS_LAUNCH_CHECK(MODE == kGateUp ? "w4a16 gate_up" : "w4a16 down");
  return JANUS_MOE_OK;
}

}  // namespace

int launch_gate_up(const GemmParams& p, hipStream_t stream) { return launch_gemm<kGateUp>(p, stream); }
int launch_down(const GemmParams& p, hipStream_t stream) { return launch_gemm<kDown>(p, stream); }

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

int launch_finalize(const float* acc, uint16_t* out, long n, hipStream_t stream) {
  const long n4 = n / 4;
  if (n4 == 0) return JANUS_MOE_OK;
  long blocks = (n4 + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(finalize_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     reinterpret_cast<const float4*>(acc), reinterpret_cast<uint2*>(out), n4);
  JANUS_LAUNCH_CHECK("finalize");
  return JANUS_MOE_OK;
}

}  // namespace janus
