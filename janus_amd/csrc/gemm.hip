// Grouped W4A16 GEMMs for gfx950: int4 group-128 weights decoded to bf16 in registers, bf16 MFMA with fp32
// accumulation. The semantics are those of the reference's per-tile kernel (janus/moe_w4a16.py:36-86): a tile is one
// expert times a run of its rows; the gate_up launch fuses silu(gate) * up into its epilogue (:83), the down launch
// scales by the routing weight (:84-85). Unlike the reference's bf16 y buffer and bf16 reshape-sum (:140), each
// weighted expert output is kept in a per-token slot as int16 codes with one fp32 scale per 64 columns (16 significant
// bits against the block's largest value, where bf16 keeps 8 per value), and a combine pass sums a token's slots in
// fp32 in a fixed order and rounds once: the result is deterministic.
//
// Work decomposition. A workgroup (4 waves) takes one chunk (up to 96 rows of one expert, or 96 consecutive tokens of
// the shared expert) and one column slab. Each wave owns 4 MFMA column blocks of 16 weight rows: it streams their int4
// words from HBM into a 2-deep register ring (one 16-byte load per lane per 128 k), decodes each word once and
// multiplies it against all of the chunk's rows. The activation rows of each 128-wide k stage are staged through
// registers into an LDS double buffer shared by the 4 waves, one stage ahead of the MFMAs (they are mostly L2 hits:
// every slab of a chunk reads the same rows). v_mfma_f32_16x16x32_bf16 takes the weights as its first operand: a
// lane's accumulator holds 4 consecutive output columns of one row. Workgroup ids are dealt to the 8 XCDs round-robin;
// the slabs of one chunk get ids that land on the same XCD, so the chunk's activation rows come from that XCD's L2
// after the first slab.
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "gemm.h"

namespace janus {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kColBlocks = 4;
constexpr int KS = 128;                                      // k per pipeline stage: one scale group
constexpr int kStages = 3;                                   // activation and weight rings: loads run two stages ahead
constexpr int kRowBytes = KS * 2;                            // one activation row of a stage (bf16)
template <int RB>
constexpr int slot_bytes() { return 16 * RB * kRowBytes; }  // one LDS activation buffer of an RB-row-block tile

enum { kGateUp = 0, kDown = 1 };

template <int V>
using Slot = std::integral_constant<int, V>;

// Compile-time loop: f(integral_constant<int, I>) for I in [0, N).
template <int... Is, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, Is...>, F&& f) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, static_cast<F&&>(f));
}

// The k pipeline over nkb stages of KS k. Activations go from global memory straight into LDS (buffer loads that write
// LDS, no register staging) and weight words and scales into registers; both are rings of kStages slots, slot = stage
// mod kStages, and each stage's loads are issued kStages - 1 stages ahead, activations first. The compiler does not
// order a buffer-to-LDS load before later LDS reads, so the pipeline does: before the barrier that opens stage kb,
// every wave consumes stage kb's weight registers in an empty asm, for which the compiler waits with an exact count
// (every global load here is one it tracks). A wave's loads complete in issue order, so its stage-kb activation loads,
// issued before those weights, have landed too; the barrier then publishes the whole tile. The same barrier tells
// every wave that all reads of the stage before are done, so its slot can be refilled right after it.
//   issue_a(slot, kb) / issue_b(slot, kb)   stage kb's activation tile into LDS slot / weights into register slot
//   wait_b(slot, kb)                        the empty asm on stage kb's weight registers (ring slot `slot`)
//   compute(slot, kb)                       MFMAs of stage kb, held in slot `slot`
//   before(kb)                              the caller's own loads for after the k loop, issued ahead of stage kb's
//                                           MFMAs (so their latency hides behind the last stages)
template <int NKB, typename IssueA, typename IssueB, typename WaitB, typename Compute, typename Before>
__device__ __attribute__((always_inline)) inline void run_pipeline(int nkb, bool active, IssueA&& issue_a,
                                                                   IssueB&& issue_b, WaitB&& wait_b,
                                                                   Compute&& compute, Before&& before) {
  constexpr int ahead = kStages - 1;
  auto step = [&](auto slot_c, int kb) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    wait_b(slot_c, kb);
    lds_barrier();
    if (kb + ahead < nkb) {
      issue_a(Slot<(slot + ahead) % kStages>{}, kb + ahead);
      asm volatile("" ::: "memory");  // the compiler may not hoist the weight loads above the activation loads
      issue_b(Slot<(slot + ahead) % kStages>{}, kb + ahead);
    }
    before(kb);
    if (active) compute(slot_c, kb);
  };
  static_for<ahead>([&](auto s_c) __attribute__((always_inline)) {
    if (decltype(s_c)::value < nkb) {
      issue_a(s_c, decltype(s_c)::value);
      asm volatile("" ::: "memory");
      issue_b(s_c, decltype(s_c)::value);
    }
  });
  if constexpr (NKB > 0) {
    static_for<NKB>([&](auto kb_c) __attribute__((always_inline)) {
      step(Slot<decltype(kb_c)::value % kStages>{}, decltype(kb_c)::value);
    });
  } else {
    for (int kb = 0; kb < nkb; kb += kStages) {
      static_for<kStages>([&](auto s_c) __attribute__((always_inline)) {
        if (kb + decltype(s_c)::value < nkb) step(s_c, kb + decltype(s_c)::value);
      });
    }
  }
}

// One int32 word of 8 int4 weights sharing the bf16 scale `sb` -> the bf16 MFMA operand in k order 0..7.
// Each nibble, its top bit flipped (offset binary n = q + 8, 0..15), goes into the low four bits of a byte. Read as an
// fp8 e4m3 byte (OCP: bias 7, subnormals) such a byte is exactly n * 2^-9: exponent field 0 gives the subnormals
// 0..7 * 2^-9, exponent field 1 the normals (8 + m) * 2^-9. v_cvt_pk_f32_fp8 widens two of them per instruction, and
// fma(n 2^-9, 512 s, -8 s) = q s exactly: the product has at most 12 significant bits and the sum is the exact
// q s, which has at most 12 too, so the fma's rounding changes nothing. The packed conversion to bf16 then rounds once
// to nearest even: bf16(q * s). Per word: two masks (one with a shift), four widenings, eight fmas, four packs.
struct Scale {
  float m, c;  // 512 s and -8 s
};
__device__ __forceinline__ Scale make_scale(uint32_t sb) {
  const float s = __uint_as_float(sb << 16);
  return Scale{512.0f * s, -8.0f * s};
}
__device__ __forceinline__ bf16x8 decode8(uint32_t w, const Scale& s) {
  // bytes j of lo / hi: elements 2j / 2j + 1, as n = nibble ^ 8 (v_bitop3 truth table 0x6A: (S0 & S1) ^ S2)
  const uint32_t lo = __builtin_amdgcn_bitop3_b32(w, 0x0F0F0F0Fu, 0x08080808u, 0x6A);
  const uint32_t hi = __builtin_amdgcn_bitop3_b32(w >> 4, 0x0F0F0F0Fu, 0x08080808u, 0x6A);
  const float2_t l0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false);  // elements 0, 2
  const float2_t l1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);   // elements 4, 6
  const float2_t h0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);  // elements 1, 3
  const float2_t h1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);   // elements 5, 7
  const float v[8] = {l0[0], h0[0], l0[1], h0[1], l1[0], h1[0], l1[1], h1[1]};
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = static_cast<__bf16>(fmaf(v[j], s.m, s.c));
  return r;
}
__device__ __forceinline__ bf16x8 decode8(uint32_t w, uint32_t sb) { return decode8(w, make_scale(sb)); }

// NVFP4 (janus/hybrid.py:400-423, janus/moe_w4a16.py:19-33, 68-72): byte b of the word holds elements 2b (low nibble)
// and 2b + 1 (high nibble) as e2m1 codes, the same k order as the int4 words. W = bf16(fp32(e2m1 * S)) with
// S = fp32(e4m3 block scale * fp32 global scale of the row): the reference's two fp32 products, then one rounding to
// bf16. v_cvt_scalef32_pk_f32_fp4 widens the two codes of a byte exactly (scale 1); 16 VALU per word.
__device__ __forceinline__ bf16x8 decode8_nvfp4(uint32_t w, float S) {
  const float2_t v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
  const float2_t v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
  const float2_t v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
  const float2_t v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
  const float v[8] = {v0[0], v0[1], v1[0], v1[1], v2[0], v2[1], v3[0], v3[1]};
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = static_cast<__bf16>(v[j] * S);
  return r;
}
// S of an e4m3 block-scale byte (OCP e4m3fn, as gfx950's fp8 conversions read it) and the row's global scale.
__device__ __forceinline__ float nvfp4_block_scale(uint32_t e4m3_byte, float global) {
  return __builtin_amdgcn_cvt_f32_fp8((int)e4m3_byte, 0) * global;
}

// Per-codec scale state of one column block for one 128-k stage, and the decode of its word t.
//   int4 group-128: one bf16 scale per stage (2 bytes per row).
//   NVFP4: two e4m3 block scales per lane (the lane's words t = 0, 1 fall in block 2g, t = 2, 3 in block 2g + 1; the
//   lane loads the two bytes at 2g of the row's eight per stage) times the row's global scale.
enum { kInt4 = 0, kNvfp4 = 1 };
template <int CODEC>
struct Codec;
template <>
struct Codec<kInt4> {
  static constexpr int kScaleBytesPerStage = 2;  // per row
  using State = Scale;
  __device__ static State make(uint32_t sc, float) { return make_scale(sc); }
  __device__ static bf16x8 decode(uint32_t w, const State& s, int) { return decode8(w, s); }
};
template <>
struct Codec<kNvfp4> {
  static constexpr int kScaleBytesPerStage = 8;
  struct State {
    float s0, s1;
  };
  __device__ static State make(uint32_t sc, float global) {
    return State{nvfp4_block_scale(sc & 0xFFu, global), nvfp4_block_scale((sc >> 8) & 0xFFu, global)};
  }
  __device__ static bf16x8 decode(uint32_t w, const State& s, int t) { return decode8_nvfp4(w, t < 2 ? s.s0 : s.s1); }
};

// NKB: k stages (K / 128) fixed at compile time, the whole k loop unrolled so the compiler's wait counts for the
// weight registers are exact (a runtime loop makes it wait for every outstanding load); 0 = runtime K.
//
// One work unit: chunk c (c < n_shared_chunks: shared-expert tokens c * kChunkRows.., else routed chunk
// c - n_shared_chunks) times column slab `slab`. lds: the workgroup's ring of activation tiles, one array per slot
// (separate arrays let the compiler see that a load into one slot does not write the slot being read, so its wait for
// the loads into LDS before a read covers only that slot's), each [row][16-byte chunk] with chunk position =
// chunk ^ (row & 15): the 16 lanes of a fragment read (same chunk, 16 rows) hit 16 different bank groups. Uniform over
// the workgroup; a unit past the chunk list or the columns does nothing.
// The activation ring: kStages separate LDS arrays (see gemm_unit).
struct LdsRing {
  unsigned char* s0;
  unsigned char* s1;
  unsigned char* s2;
  template <typename S>
  __device__ __forceinline__ unsigned char* slot(S) const {
    return S::value == 0 ? s0 : S::value == 1 ? s1 : s2;
  }
};

// An empty asm that takes every activation and weight fragment of a 32-k step at one point (see compute).
__device__ __forceinline__ void pin_fragments(bf16x8 (&a)[6], bf16x8 (&b)[kColBlocks]) {
  static_assert(kColBlocks == 4, "the asm lists every fragment");
  asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(b[0]), "+v"(b[1]),
                    "+v"(b[2]), "+v"(b[3]));
}
__device__ __forceinline__ void pin_fragments(bf16x8 (&a)[1], bf16x8 (&b)[kColBlocks]) {
  asm volatile("" : "+v"(a[0]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
}

template <int MODE, int NKB, int CODEC, int RB>
__device__ __attribute__((always_inline)) inline void gemm_unit(const GemmParams& p, int c, int slab,
                                                                LdsRing lds, bool poison = false) {
  using C = Codec<CODEC>;
  int tid = threadIdx.x;
  // the lane's index math is redone for every unit: kept from a caller's earlier iteration, it would hold registers
  // across the whole k loop
  asm volatile("" : "+v"(tid));
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const int g = lane >> 4, nl = lane & 15;

  const bool shared = c < p.n_shared_chunks;
  int pos0, rows, N, K;
  const int32_t* wq;
  const unsigned char* wsc;
  const float* wgl = nullptr;  // NVFP4: global scale of each weight row
  if (shared) {
    pos0 = c * (16 * RB);
    rows = min((16 * RB), p.T - pos0);
    wq = p.q_sh;
    wsc = reinterpret_cast<const unsigned char*>(p.s_sh);
    if (CODEC == kNvfp4) wgl = p.gsc_sh;
    N = p.N_sh;
    K = p.K_sh;
  } else {
    // the count and the entry are loaded together (one memory round trip): r < max_chunks is inside the list, and an
    // entry past the count is not used
    const int r = c - p.n_shared_chunks;
    const int nch = *p.num_chunks;
    const int4 ch = p.chunks[r];
    if (r >= nch) return;
    pos0 = ch.y;
    rows = ch.z;
    N = p.N;
    K = p.K;
    wq = p.q + (long)ch.x * N * (K / 8);
    wsc = reinterpret_cast<const unsigned char*>(p.s) + (long)ch.x * N * (K / KS) * C::kScaleBytesPerStage;
    if (CODEC == kNvfp4) wgl = p.gsc + (long)ch.x * N;
  }
  constexpr int kWaveCols = (MODE == kGateUp) ? 32 : 64;  // h columns (gate_up) or output columns (down)
  const int out_cols = (MODE == kGateUp) ? N / 2 : N;
  if (slab * kWaveCols * kWaves >= out_cols) return;
  const int col0 = slab * kWaveCols * kWaves + wave * kWaveCols;
  const bool active = col0 < out_cols;
  const int nrb = (rows + 15) / 16;

  // ---- activation rows this lane loads: load r covers rows 16r..16r+15, this wave's instruction rows 16r + 4w ..
  // 16r + 4w + 3 (64 lanes x 16 bytes = 4 rows of a stage, written to LDS in lane order). Lane l writes LDS chunk
  // position l & 15 of row 16r + 4w + (l >> 4); position q of row m holds global chunk q ^ (m & 15), so the 16 lanes of
  // a fragment read (one chunk, 16 rows) hit 16 different bank groups. The load of a row past the chunk gets an offset
  // beyond the buffer, which the hardware answers with zeros. Byte offsets are 32-bit (the host bounds the buffers
  // below 2 GiB). A routed gate_up unit's rows are tokens looked up through sorted_ids, all six lookups issued before
  // the first is used (a load selected against another value under a branch would be waited for at once).
  const unsigned char* abase;
  uint32_t abytes;
  if (MODE == kGateUp) {
    abase = reinterpret_cast<const unsigned char*>(p.a);
    abytes = p.a_bytes;
  } else {
    abase = reinterpret_cast<const unsigned char*>(shared ? p.a_sh : p.a);
    abytes = shared ? p.a_sh_bytes : p.a_bytes;
  }
  const __amdgpu_buffer_rsrc_t arsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(abase), (short)0, (int)abytes, 0x00020000);
  constexpr uint32_t kOutside = 0x80000000u;  // past every activation buffer
  const int lrow = 4 * wave + (lane >> 4);    // this lane's row within a load's 16 (row & 15 of every row it loads)
  const uint32_t achunk = (uint32_t)(((lane & 15) ^ lrow) * 16);
  // sized for the largest tile (a size that depends on RB trips the host compiler on the buffer-load builtin below);
  // entries past RB are never read
  uint32_t aoff[kRowBlocks];
  if (MODE == kGateUp && !shared) {
    int id[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int row = 16 * r + lrow;
      id[r] = p.sorted_ids[pos0 + (row < rows ? row : 0)];
    }
#pragma unroll
    for (int r = 0; r < RB; ++r)
      aoff[r] = (16 * r + lrow < rows) ? (uint32_t)(id[r] / p.topk) * (uint32_t)(K * 2) + achunk : kOutside;
  } else {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int row = 16 * r + lrow;
      aoff[r] = row < rows ? (uint32_t)(pos0 + row) * (uint32_t)(K * 2) + achunk : kOutside;
    }
  }

  // ---- weight rows of this lane, one per column block (an idle wave reads row 0 and discards it) ----
  // the unit's weight and scale rows as buffer resources (32-bit lane offsets, the stage's offset an immediate)
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(wq), (short)0, (int)((uint32_t)N * (uint32_t)(K / 2)), 0x00020000);
  const __amdgpu_buffer_rsrc_t srsrc_w = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<unsigned char*>(wsc), (short)0, (int)((uint32_t)N * (uint32_t)(K / KS * C::kScaleBytesPerStage)),
      0x00020000);
  uint32_t woff[kColBlocks], soff[kColBlocks];
  float gq[kColBlocks];
#pragma unroll
  for (int cb = 0; cb < kColBlocks; ++cb) {
    int n;
    if (MODE == kGateUp)
      n = (cb < 2) ? col0 + 16 * cb + nl : N / 2 + col0 + 16 * (cb - 2) + nl;
    else
      n = col0 + 16 * cb + nl;
    if (!active) n = 0;
    woff[cb] = (uint32_t)n * (uint32_t)(K / 2) + g * 16;
    // NVFP4: the lane's two block scales of a stage sit at byte 2g of the stage's 8 (unbatched); batched, the lane
    // loads the 8 bytes of stage 4m + g of each four-stage batch m (see stage_scale)
    soff[cb] = (uint32_t)n * (uint32_t)(K / KS * C::kScaleBytesPerStage) +
               (CODEC == kNvfp4 ? (NKB >= 4 && NKB % 4 == 0 ? g * 8 : g * 2) : 0);
    gq[cb] = CODEC == kNvfp4 ? wgl[n] : 0.0f;
  }

  f32x4 acc[RB][kColBlocks];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < kColBlocks; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nkb = NKB > 0 ? NKB : K / KS;
  u32x4 bw[kStages][kColBlocks];
  uint32_t sc[kStages][kColBlocks];
  // Scales with the k loop unrolled come in batches of four stages, one 8-byte load per column block, issued with the
  // weights of stage 4m; two batches are live at a time.
  //   int4: the row's bf16 scales of groups 4m .. 4m + 3 (adjacent).
  //   NVFP4: the row's 32 e4m3 bytes of the batch are 8 per stage; lane g loads stage 4m + g's 8 bytes, and a lane
  //   takes its two bytes of stage 4m + s (at byte 2g) from lane (nl, s) with two cross-lane reads: one load per four
  //   stages instead of a 2-byte load every stage.
  constexpr bool kBatchScales = NKB >= 4 && NKB % 4 == 0;
  u32x2 scb[2][kColBlocks];

  // the LDS destination is wave-uniform (it goes to M0) and the stage's k offset rides in the SGPR offset
  const int uwave = __builtin_amdgcn_readfirstlane(wave);
  // The last two row blocks are loaded only when the chunk reaches them (each load is one more instruction through
  // the CU's address unit, which the GEMM keeps busy); their LDS rows otherwise keep older data, read but never
  // multiplied. They are issued first in a stage's group, so the waits the compiler derives for the paths that skip
  // them (fewer loads in flight) cost at most those two early loads on the paths that issue them.
  constexpr int kAlwaysRb = RB < 4 ? RB : 4;
  const int unrb = __builtin_amdgcn_readfirstlane(nrb);
  auto issue_a = [&](auto slot_c, int kb) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    unsigned char* dst = lds.slot(slot_c) + (4 * uwave) * kRowBytes;
    auto load = [&](int r) __attribute__((always_inline)) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (JANUS_LDS void*)(dst + 16 * r * kRowBytes), 16, aoff[r],
                                               kb * (KS * 2), 0, 0);
    };
#pragma unroll
    for (int r = kAlwaysRb; r < RB; ++r)
      if (r < unrb) load(r);
#pragma unroll
    for (int r = 0; r < kAlwaysRb; ++r) load(r);
  };
  auto load_b = [&](auto slot_c, int kb) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int cb = 0; cb < kColBlocks; ++cb) {
      bw[slot][cb] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, woff[cb], kb * (KS / 2), 0));
      if constexpr (kBatchScales) {
        if (kb % 4 == 0)
          scb[(kb / 4) & 1][cb] = __builtin_bit_cast(
              u32x2, __builtin_amdgcn_raw_buffer_load_b64(srsrc_w, soff[cb], kb * C::kScaleBytesPerStage, 0));
      } else {
        sc[slot][cb] = __builtin_amdgcn_raw_buffer_load_b16(srsrc_w, soff[cb], kb * C::kScaleBytesPerStage, 0);
      }
    }
  };
  // stage kb's scale bits of column block cb: int4, the bf16 bits (the batched form keeps them in either half of a
  // word); NVFP4, the two e4m3 bytes of the lane's blocks
  auto stage_scale = [&](auto slot_c, int kb, int cb) __attribute__((always_inline)) -> uint32_t {
    constexpr int slot = decltype(slot_c)::value;
    if constexpr (kBatchScales && CODEC == kInt4) {
      const u32x2 v = scb[(kb / 4) & 1][cb];
      const uint32_t word = (kb & 2) ? v[1] : v[0];
      return (kb & 1) ? word >> 16 : word & 0xFFFFu;
    } else if constexpr (kBatchScales) {
      const u32x2 v = scb[(kb / 4) & 1][cb];
      const int src = nl + 16 * (kb & 3);  // the lane that loaded stage kb's 8 bytes
      const uint32_t lo = __shfl((int)v[0], src), hi = __shfl((int)v[1], src);
      const uint32_t word = (g & 2) ? hi : lo;
      return (g & 1) ? word >> 16 : word & 0xFFFFu;
    } else {
      return sc[slot][cb];
    }
  };
  // the scale registers of stage kb as loaded (a batch's registers at each of its stages)
  auto scale_regs = [&](auto slot_c, int kb, int cb) __attribute__((always_inline)) -> u32x2 {
    constexpr int slot = decltype(slot_c)::value;
    if constexpr (kBatchScales) {
      return scb[(kb / 4) & 1][cb];
    } else {
      return u32x2{sc[slot][cb], 0u};
    }
  };
  auto wait_b = [&](auto slot_c, int kb) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    const u32x4 w0 = bw[slot][0], w1 = bw[slot][1], w2 = bw[slot][2], w3 = bw[slot][3];
    const u32x2 s0 = scale_regs(slot_c, kb, 0), s1 = scale_regs(slot_c, kb, 1), s2 = scale_regs(slot_c, kb, 2),
                s3 = scale_regs(slot_c, kb, 3);
    asm volatile("" ::"v"(w0), "v"(w1), "v"(w2), "v"(w3), "v"(s0), "v"(s1), "v"(s2), "v"(s3));
  };
  auto compute = [&](auto slot_c, int kb) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    const unsigned char* base = lds.slot(slot_c);
    typename C::State scl[kColBlocks];
#pragma unroll
    for (int cb = 0; cb < kColBlocks; ++cb) scl[cb] = C::make(stage_scale(slot_c, kb, cb), gq[cb]);
#pragma unroll
    for (int t = 0; t < KS / 32; ++t) {
      // every row block's fragment is read before the decode, which covers the LDS latency (rows past the chunk hold
      // copies of its first row, so the reads are defined); only the chunk's row blocks are multiplied. An empty asm
      // takes the activation fragments together with the decoded weights, so the compiler can neither sink a read into
      // its row block's branch, next to its first use, nor hoist the wait for the reads above the decode.
      bf16x8 afrag[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        afrag[rb] = *reinterpret_cast<const bf16x8*>(base + (16 * rb + nl) * kRowBytes + ((4 * g + t) ^ nl) * 16);
      __builtin_amdgcn_sched_barrier(0);  // the reads issue before the decode
      if constexpr (RB == 1) {
        // one row block: each column block's weights are decoded right before their MFMA (one fragment live)
#pragma unroll
        for (int cb = 0; cb < kColBlocks; ++cb) {
          bf16x8 b = C::decode(bw[slot][cb][t], scl[cb], t);
          asm volatile("" : "+v"(b), "+v"(afrag[0]));
          acc[0][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b, afrag[0], acc[0][cb], 0, 0, 0);
        }
        continue;
      }
      bf16x8 bfrag[kColBlocks];
#pragma unroll
      for (int cb = 0; cb < kColBlocks; ++cb) bfrag[cb] = C::decode(bw[slot][cb][t], scl[cb], t);
      pin_fragments(afrag, bfrag);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if (rb < nrb) {
#pragma unroll
          for (int cb = 0; cb < kColBlocks; ++cb)
            acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfrag[cb], afrag[rb], acc[rb][cb], 0, 0, 0);
        }
      }
    }
  };
  // down: each row's assignment id (the token, for the shared expert) and its routing weight, for the epilogue. The
  // ids are loaded ahead of the second-to-last stage and the weights, which need them, ahead of the last, so neither
  // waits after the k loop. (Rows past the chunk read its first row's: loads without a branch, values not used.)
  int id[RB];
  float wt[RB];
  auto before = [&](int kb) __attribute__((always_inline)) {
    if constexpr (MODE == kDown) {
      if (kb == (nkb >= 2 ? nkb - 2 : 0)) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int m = rb * 16 + nl;
          id[rb] = shared ? pos0 + (m < rows ? m : 0) : p.sorted_ids[pos0 + (m < rows ? m : 0)];
        }
      }
      if (kb == nkb - 1) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          wt[rb] = shared ? (p.gamma ? p.gamma[id[rb]] : 1.0f) : p.route_w[id[rb]];
      }
    }
  };
  static_assert(kColBlocks == 4, "wait_b lists every column block");
  run_pipeline<NKB>(nkb, active, issue_a, load_b, wait_b, compute, before);
  if (!active) return;

  // ---- epilogue: lane holds rows 16 rb + nl, columns 16 cb + 4 g + i ----
  if (MODE == kGateUp) {
    uint16_t* hbase = shared ? p.h_sh : p.h;
    const int hw = N / 2;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int m = rb * 16 + nl;
      if (rb >= nrb || m >= rows) continue;
      uint16_t* hrow = hbase + (long)(pos0 + m) * hw;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        float hv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gv = acc[rb][cb][i], uv = acc[rb][cb + 2][i];
          // silu(g) u = g u / (1 + e^-g) with the hardware exp and reciprocal (about 1 ulp each): h is rounded to
          // bf16 next, which absorbs them; an IEEE division would cost several times the instructions
          hv[i] = gv * uv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv));
        }
        uint2 st;
        st.x = pack_bf16x2(hv[0], hv[1]);
        st.y = pack_bf16x2(hv[2], hv[3]);
        *reinterpret_cast<uint2*>(hrow + col0 + 16 * cb + 4 * g) = st;
      }
    }
  } else {
    // each row's slot offset, before the first store (a divisor constant the compiler keeps in scratch would
    // otherwise be reloaded, and waited for, between the stores)
    long orow_off[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int tok = shared ? id[rb] : id[rb] / p.topk;
      const int slot = shared ? p.topk : id[rb] - tok * p.topk;
      orow_off[rb] = ((long)tok * p.nslots + slot) * N;
    }
    if (poison) {  // this unit's h rows were not known to be complete: its rows become NaN instead of wrong values
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) wt[rb] = __builtin_nanf("");
    }
    // Slot encoding of a row's 64 columns (this wave's block): the 4 lanes of the row (g = 0..3) share the largest
    // |acc|; code = rint(acc * sign(w) * 32767 / max|acc|), scale = |w| max|acc| / 32767 (NaN with w, for a poisoned
    // row). fma(v, f, 1.5 * 2^23) rounds v * f to an integer to nearest even and, as |v f| < 2^15 (the reciprocal's
    // error is far below 0.5 / 32767), leaves its two's complement in the low 16 bits of the result. Lane g stores its
    // column blocks 0, 1 as stored groups 2g, 2g + 1 and its blocks 2, 3 as 8 + 2g, 9 + 2g (slot_stored_group), so
    // every store instruction writes 64 contiguous bytes per row. The maxima are taken for every row block before the
    // first branch: the cross-lane reads need all lanes.
    float amax[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float a = 0.f;
#pragma unroll
      for (int cb = 0; cb < kColBlocks; ++cb)
#pragma unroll
        for (int i = 0; i < 4; ++i) a = fmaxf(a, fabsf(acc[rb][cb][i]));
      a = fmaxf(a, __shfl_xor(a, 16));
      amax[rb] = fmaxf(a, __shfl_xor(a, 32));
    }
    constexpr float kRound = 12582912.0f;  // 1.5 * 2^23
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int m = rb * 16 + nl;
      if (rb >= nrb || m >= rows) continue;
      const float w = wt[rb];
      const float f0 = amax[rb] > 0.f ? 32767.0f * __builtin_amdgcn_rcpf(amax[rb]) : 0.f;
      const float f = w < 0.f ? -f0 : f0;
      uint32_t code[2 * kColBlocks];
#pragma unroll
      for (int cb = 0; cb < kColBlocks; ++cb)
#pragma unroll
        for (int i = 0; i < 4; i += 2)
          code[2 * cb + i / 2] = __builtin_amdgcn_perm(__float_as_uint(fmaf(acc[rb][cb][i + 1], f, kRound)),
                                                       __float_as_uint(fmaf(acc[rb][cb][i], f, kRound)), 0x05040100u);
      int16_t* orow = p.slots + orow_off[rb] + col0;
      *reinterpret_cast<uint4*>(orow + 8 * g) = make_uint4(code[0], code[1], code[2], code[3]);
      *reinterpret_cast<uint4*>(orow + 32 + 8 * g) = make_uint4(code[4], code[5], code[6], code[7]);
      if (g == 0) p.slot_scale[(orow_off[rb] + col0) / kSlotBlock] = fabsf(w) * amax[rb] * (1.0f / 32767.0f);
    }
  }
}

// One launch per GEMM: workgroup ids are dealt to the 8 XCDs round-robin, and the slabs of chunk c go to ids on XCD
// c mod 8, so they share its L2.
// Workgroups per CU: two for the 96-row tile, three for the 16-row tile (fewer accumulator registers).
template <int RB>
constexpr int wg_per_cu() { return RB == 1 ? 3 : 2; }

template <int MODE, int NKB, int CODEC, int RB>
__global__ void __launch_bounds__(kThreads, wg_per_cu<RB>()) w4a16_gemm_kernel(const GemmParams p) {
  static_assert(kStages == 3, "one array per ring slot");
  constexpr int kSlotBytes = slot_bytes<RB>();
  __shared__ __attribute__((aligned(16))) unsigned char lds0[kSlotBytes], lds1[kSlotBytes], lds2[kSlotBytes];
  const LdsRing lds{lds0, lds1, lds2};
  const int xcd = blockIdx.x & 7, within = blockIdx.x >> 3;
  const int c = (within / p.nslab) * 8 + xcd;
  if (c >= p.n_shared_chunks + p.max_chunks) return;
  gemm_unit<MODE, NKB, CODEC, RB>(p, c, within % p.nslab, lds);
}

// Both GEMMs in one persistent launch of two (16-row tile: three) workgroups per CU. The work units sit in one queue per
// XCD: queue q holds a set of chunks (shared-expert chunks first, as c counts them first; the routed chunks in expert
// order), their gate_up units chunk by chunk, then their down units in the same order. A workgroup reads the id of the
// XCD it runs on and takes tickets from that queue until it runs dry, so every unit of a chunk, producer or consumer of
// its h rows, runs under one L2, and the down units of early chunks fill the CUs that gate_up's last units leave idle.
// With the 96-row tile queue q holds a contiguous range of chunks: the chunks of one expert (or of the shared expert)
// then mostly share an L2 and read its weights from HBM once (T=16384: 1129 -> 1109 us, T=2048: 215 -> 212 us). The
// 16-row tile deals chunks c = q, q + nq, ... instead, which measured 11% faster at T=96 than the contiguous ranges.
// A down unit waits until all gate_up units of its chunk have counted themselves done. With the 96-row tile, down
// ticket u belongs to the queue's chunk u / slabs in list order. With the 16-row tile the chunks go in the order their
// gate_up units finish: the gate_up unit that completes a chunk (the last of its slabs to count itself done) appends
// it to the queue's ready list, and down ticket u takes the chunk at position u / slabs of that list, waiting until it
// is written, so it waits for whichever chunk finishes next rather than one particular chunk. At T=96 gate_up units
// of equal work take 28-77 us and the fixed order left down units waiting for the slowest (launch 123.0 -> 115.4 us);
// with the 96-row tile the ready list measured the same at T=2048 and 1.5% slower at T=16384. Either way a down unit
// never waits for a unit without a workgroup: every gate_up unit of the queue has a lower ticket, so a running
// workgroup took it, and gate_up units wait for nothing; they all finish, and every chunk enters the list. The wait is
// bounded: after spin_limit polls (0: none) it gives up, sets kStatusGaveUp in the device status word and (16-row
// tile) takes the chunk of the list order, writing NaN for its rows instead of a result computed on h rows that may be
// incomplete; the launch still ends.
constexpr int kSchedQueues = 8;   // ticket counters, one per XCD
constexpr int kXccIdReg = 20 | (0 << 6) | ((16 - 1) << 11);  // s_getreg operand: HW_REG_XCC_ID, bits 0..15

template <int NKB_GU, int NKB_DN, int CODEC, int RB>
__global__ void __launch_bounds__(kThreads, wg_per_cu<RB>()) moe_experts_kernel(const GemmParams gu,
                                                                                 const GemmParams dn,
                                                                                 int* __restrict__ sched, int nq,
                                                                                 int spin_limit,
                                                                                 int* __restrict__ status) {
  static_assert(kStages == 3, "one array per ring slot");
  constexpr int kSlotBytes = slot_bytes<RB>();
  __shared__ __attribute__((aligned(16))) unsigned char lds0[kSlotBytes], lds1[kSlotBytes], lds2[kSlotBytes];
  const LdsRing lds{lds0, lds1, lds2};
  __shared__ int ticket, gave_up, down_chunk;
  // Every branch of this loop is uniform over a wave: wave 0 does the bookkeeping with all its lanes. A branch on the
  // thread id would give the loop a per-lane exit, and the compiler may then run the other lanes around the loop ahead
  // of lane 0, through barriers, on a stale ticket. The counters are bumped by buffer atomics that only lane 0 keeps
  // in range: the hardware drops the other lanes' out-of-range atomics (same-address atomics from 64 lanes would run
  // one after another).
  const bool first_wave = __builtin_amdgcn_readfirstlane(threadIdx.x) < kWave;
  const int nwords = sched_words(gu.max_chunks, gu.n_shared_chunks);
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(sched, (short)0, nwords * 4, 0x00020000);
  const bool lane0 = (threadIdx.x & (kWave - 1)) == 0;
  auto bump = [&](int word) __attribute__((always_inline)) {  // sched[word] += 1 by lane 0; the old value in lane 0
    return __builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(1, srsrc, lane0 ? word * 4 : 0x7FFFFFF0, 0, 0);
  };
  const int q = (int)(__builtin_amdgcn_s_getreg(kXccIdReg) & 0xF) % nq;
  const int total = gu.n_shared_chunks + *gu.num_chunks;
  // this queue's chunks: c0, c0 + cstep, ... (ncq of them)
  const int c0 = RB == 1 ? q : (int)((long)q * total / nq);
  const int cstep = RB == 1 ? nq : 1;
  const int ncq = RB == 1 ? (total > q ? (total - q + nq - 1) / nq : 0) : (int)((long)(q + 1) * total / nq) - c0;
  const int ngu = ncq * gu.nslab, nall = ngu + ncq * dn.nslab;
  const int total_max = gu.n_shared_chunks + gu.max_chunks;
  const int ready_word = kSchedWordsFixed + total_max + q * ((total_max + nq - 1) / nq);  // this queue's ready list
  if (first_wave) ticket = __builtin_amdgcn_readfirstlane(bump(q));
  __syncthreads();
  int t = __builtin_amdgcn_readfirstlane(ticket);
  while (t < nall) {
    // the next ticket's atomic (a few microseconds when the GEMMs load the memory system) is in flight during this
    // unit. Holding two tickets cannot deadlock either: a workgroup whose next ticket is a gate_up unit holds a gate_up
    // unit now (the queue lists every gate_up unit before the first down unit), and gate_up units wait for nothing.
    int next = 0;
    if (first_wave) next = bump(q);
    if (t < ngu) {
      const int c = __builtin_amdgcn_readfirstlane(c0 + cstep * (t / gu.nslab));
      gemm_unit<kGateUp, NKB_GU, CODEC, RB>(gu, c, t % gu.nslab, lds);
      // every wave's h stores have reached the L2 before the count that publishes them
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (first_wave) {
        const int old = __builtin_amdgcn_readfirstlane(bump(kSchedWordsFixed + c));
        if (RB == 1 && old == gu.nslab - 1) {  // the chunk's last gate_up unit: append the chunk to the ready list
          const int pos = __builtin_amdgcn_readfirstlane(bump(kReadyWord + q));
          // the list word is still zero: adding c + 1 writes it
          (void)__builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(c + 1, srsrc, lane0 ? (ready_word + pos) * 4 : 0x7FFFFFF0,
                                                               0, 0);
        }
      }
    } else {
      const int u = t - ngu;
      const int idx = u / dn.nslab;  // the chunk at this position of the ready list
      if (first_wave) {
        int give_up = 0, entry = 0;
        for (int spins = 0;; ++spins) {
          if (spins >= spin_limit) {
            give_up = 1;
            if (lane0) __hip_atomic_fetch_or(status, kStatusGaveUp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          if (RB == 1) {
            entry = __builtin_amdgcn_readfirstlane(
                __hip_atomic_load(sched + ready_word + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            if (entry > 0) break;
          } else {
            const int fixed = c0 + cstep * idx;
            const int n = __builtin_amdgcn_readfirstlane(
                __hip_atomic_load(sched + kSchedWordsFixed + fixed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            if (n >= gu.nslab) {
              entry = fixed + 1;
              break;
            }
          }
          __builtin_amdgcn_s_sleep(2);
        }
        asm volatile("buffer_inv sc0" ::: "memory");  // this CU's L1 drops any stale copy of the chunk's h rows
        gave_up = give_up;
        down_chunk = give_up ? c0 + cstep * idx : entry - 1;
      }
      __syncthreads();
      const int c = __builtin_amdgcn_readfirstlane(down_chunk);
      gemm_unit<kDown, NKB_DN, CODEC, RB>(dn, c, u % dn.nslab, lds, __builtin_amdgcn_readfirstlane(gave_up) != 0);
    }
    if (first_wave) ticket = __builtin_amdgcn_readfirstlane(next);
    __syncthreads();
    t = __builtin_amdgcn_readfirstlane(ticket);
  }
}

// out[t, n] = bf16(sum_j slot value (t, j, n)), four columns (one group) per thread, slots summed in order in fp32.
// The codes and scales of up to 8 slots are loaded together before the additions. A padding token (valid[t] == 0)
// gets zeros and its slots are not read. With ids (the caller's top-k ids [T, topk], int64), slot j < topk of token t
// counts only when its id is in [0, E): the GEMMs never write the slot of a dropped assignment, so it is skipped (the
// loads still issue, their values unused).
template <bool kIds>
__global__ void combine_kernel(const uint2* __restrict__ slots, const float* __restrict__ scales, int nslots,
                               uint2* __restrict__ out, int T, int H4, const uint8_t* __restrict__ valid,
                               const int64_t* __restrict__ ids, int topk, int E) {
  constexpr int kBatch = 8;
  constexpr int kGroups = kSlotBlock / 4;  // groups of 4 columns per scale block
  const long n = (long)T * H4;
  const int nblk = H4 / kGroups;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long t = i / H4, col = i - t * H4;
    if (valid && !valid[t]) {
      out[i] = make_uint2(0u, 0u);
      continue;
    }
    uint32_t keep = ~0u;  // bit j: slot j counts
    if (kIds) {
      for (int j = 0; j < topk && j < 32; ++j) {
        const int64_t e = ids[t * topk + j];
        if (e < 0 || e >= E) keep &= ~(1u << j);
      }
    }
    const uint2* src = slots + t * nslots * H4 + (col & ~(long)(kGroups - 1)) + slot_stored_group((int)col % kGroups);
    const float* ssrc = scales + t * nslots * nblk + col / kGroups;
    float4 s = slot_decode4(src[0], ssrc[0]);
    if (kIds && !(keep & 1u)) s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j0 = 1; j0 < nslots; j0 += kBatch) {
      uint2 v[kBatch];
      float sc[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (j0 + j < nslots) {
          const u32x2 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src + (long)(j0 + j) * H4));
          v[j] = make_uint2(raw[0], raw[1]);
          sc[j] = ssrc[(long)(j0 + j) * nblk];
        }
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (j0 + j < nslots && (!kIds || ((keep >> (j0 + j)) & 1u))) {
          const float4 d = slot_decode4(v[j], sc[j]);
          s.x += d.x;
          s.y += d.y;
          s.z += d.z;
          s.w += d.w;
        }
      }
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

// bf16 weights of an NVFP4 matrix [rows, K]: packed e2m1 bytes [rows, K/2] (as int32 words), e4m3 block scales
// [rows, K/16], fp32 global scale per row [rows] (janus/hybrid.py:415-423, the dequantise path's values).
__global__ void dequant_nvfp4_kernel(const uint32_t* __restrict__ q, const uint8_t* __restrict__ s,
                                     const float* __restrict__ gs, long rows, int K, bf16x8* __restrict__ out) {
  const long words = rows * (K / 8);
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (long)gridDim.x * blockDim.x) {
    const long r = i / (K / 8);
    const int j = (int)(i % (K / 8));
    out[i] = decode8_nvfp4(q[i], nvfp4_block_scale(s[r * (K / 16) + j / 2], gs[r]));
  }
}

// Column slab width: h columns (gate_up) or output columns (down) of one workgroup.
template <int MODE>
constexpr int slab_cols() { return kWaves * (MODE == kGateUp ? 32 : 64); }

template <int MODE>
int launch_gemm(const GemmParams& params, hipStream_t stream) {
  GemmParams p = params;
  const int total = p.n_shared_chunks + p.max_chunks;
  if (total == 0) return JANUS_MOE_OK;
  const bool same_k = p.n_shared_chunks == 0 || p.K_sh == p.K;
  const int nkb = same_k ? p.K / KS : 0;
  const int out = MODE == kGateUp ? max(p.N, p.N_sh) / 2 : max(p.N, p.N_sh);
  p.nslab = ceil_div(out, slab_cols<MODE>());
  const long grid = (long)ceil_div(total, 8) * 8 * p.nslab;
  JANUS_REQUIRE(grid < (1l << 31), JANUS_MOE_EINVAL, "grouped GEMM grid too large");
  const dim3 g((unsigned)grid), b(kThreads);
  JANUS_REQUIRE(p.codec == kInt4 || (p.codec == kNvfp4 && p.gsc && (p.n_shared_chunks == 0 || p.gsc_sh)),
                JANUS_MOE_EINVAL, "grouped GEMM: codec %d (NVFP4 needs global scales, the shared expert's too)",
                p.codec);
  JANUS_REQUIRE(p.chunk_rows == 16 * kRowBlocks || p.chunk_rows == 16, JANUS_MOE_EINVAL,
                "grouped GEMM: chunk_rows=%d (16 or %d)", p.chunk_rows, 16 * kRowBlocks);
  // the 16-row tile keeps the unrolled k loops of the 35B-A3B shapes (K = 2048 and 512) and the runtime-K loop
#define JANUS_GEMM_CASES(CODEC)                                                                                \
  if (p.chunk_rows == 16) {                                                                                   \
    switch (nkb) {                                                                                            \
      case 4: hipLaunchKernelGGL((w4a16_gemm_kernel<MODE, 4, CODEC, 1>), g, b, 0, stream, p); break;          \
      case 16: hipLaunchKernelGGL((w4a16_gemm_kernel<MODE, 16, CODEC, 1>), g, b, 0, stream, p); break;        \
      default: hipLaunchKernelGGL((w4a16_gemm_kernel<MODE, 0, CODEC, 1>), g, b, 0, stream, p); break;         \
    }                                                                                                         \
  } else {                                                                                                    \
    switch (nkb) {                                                                                            \
      case 2: hipLaunchKernelGGL((w4a16_gemm_kernel<MODE, 2, CODEC, kRowBlocks>), g, b, 0, stream, p); break;   \
      case 4: hipLaunchKernelGGL((w4a16_gemm_kernel<MODE, 4, CODEC, kRowBlocks>), g, b, 0, stream, p); break;   \
      case 8: hipLaunchKernelGGL((w4a16_gemm_kernel<MODE, 8, CODEC, kRowBlocks>), g, b, 0, stream, p); break;   \
      case 16: hipLaunchKernelGGL((w4a16_gemm_kernel<MODE, 16, CODEC, kRowBlocks>), g, b, 0, stream, p); break; \
      default: hipLaunchKernelGGL((w4a16_gemm_kernel<MODE, 0, CODEC, kRowBlocks>), g, b, 0, stream, p); break;  \
    }                                                                                                         \
  }
  if (p.codec == kNvfp4) {
    JANUS_GEMM_CASES(kNvfp4)
  } else {
    JANUS_GEMM_CASES(kInt4)
  }
#undef JANUS_GEMM_CASES
  JANUS_LAUNCH_CHECK(MODE == kGateUp ? "w4a16 gate_up" : "w4a16 down");
  return JANUS_MOE_OK;
}

struct DeviceShape {
  int cus, xccs;
};
DeviceShape device_shape() {
  static DeviceShape cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return DeviceShape{0, 0};
  DeviceShape& d = cache[dev];
  if (d.cus == 0) {
    int cus = 0, xccs = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
    if (hipDeviceGetAttribute(&xccs, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) xccs = 0;
    d.xccs = xccs;
    d.cus = cus;
  }
  return d;
}

}  // namespace

int launch_experts_fused(const GemmParams& gu_in, const GemmParams& dn_in, int* sched, int* status,
                         hipStream_t stream) {
  const char* env = getenv("JANUS_MOE_SCHEDULE");
  if (env && strcmp(env, "split") == 0) return kNotFused;
  if (!status) return kNotFused;
  // a CU mask can leave an XCD without workgroups, and its queue would never drain
  if (getenv("HSA_CU_MASK") || getenv("ROC_GLOBAL_CU_MASK")) return kNotFused;
  GemmParams gu = gu_in, dn = dn_in;
  if (gu.n_shared_chunks + gu.max_chunks == 0) return kNotFused;
  if (gu.n_shared_chunks && (gu.K_sh != gu.K || dn.K_sh != dn.K)) return kNotFused;
  const DeviceShape d = device_shape();
  if (d.cus <= 0 || d.xccs <= 0) return kNotFused;
  const int nq = d.xccs < kSchedQueues ? d.xccs : kSchedQueues;
  gu.nslab = ceil_div(max(gu.N, gu.N_sh) / 2, slab_cols<kGateUp>());
  dn.nslab = ceil_div(max(dn.N, dn.N_sh), slab_cols<kDown>());
  const int nkb_gu = gu.K / KS, nkb_dn = dn.K / KS;
  const bool small = gu.chunk_rows == 16;
  const dim3 g((unsigned)((small ? wg_per_cu<1>() : wg_per_cu<kRowBlocks>()) * d.cus)), b(kThreads);
  // polls of about 1 us: a wait lasts at most one gate_up unit. JANUS_MOE_SPIN_LIMIT (a count, 0 = give up at once)
  // lets a test force the give-up path from the host.
  int spin_limit = 1 << 18;
  if (const char* lim = getenv("JANUS_MOE_SPIN_LIMIT")) spin_limit = atoi(lim) < 0 ? 0 : atoi(lim);
  const bool nv_ok = gu.codec == kNvfp4 && gu.gsc && dn.gsc && (gu.n_shared_chunks == 0 || (gu.gsc_sh && dn.gsc_sh));
#define JANUS_EXPERTS(GU, DN, CODEC, RB) \
  hipLaunchKernelGGL((moe_experts_kernel<GU, DN, CODEC, RB>), g, b, 0, stream, gu, dn, sched, nq, spin_limit, status)
  if (small && gu.codec == kInt4 && nkb_gu == 16 && nkb_dn == 4)
    JANUS_EXPERTS(16, 4, kInt4, 1);
  else if (small && nv_ok && nkb_gu == 16 && nkb_dn == 4)
    JANUS_EXPERTS(16, 4, kNvfp4, 1);
  else if (small)
    return kNotFused;
  else if (gu.codec == kInt4 && nkb_gu == 16 && nkb_dn == 4)
    JANUS_EXPERTS(16, 4, kInt4, kRowBlocks);
  else if (gu.codec == kInt4 && nkb_gu == 4 && nkb_dn == 2)
    JANUS_EXPERTS(4, 2, kInt4, kRowBlocks);
  else if (nv_ok && nkb_gu == 16 && nkb_dn == 4)
    JANUS_EXPERTS(16, 4, kNvfp4, kRowBlocks);
  else
    return kNotFused;
#undef JANUS_EXPERTS
  JANUS_LAUNCH_CHECK("w4a16 experts");
  return JANUS_MOE_OK;
}

int launch_gate_up(const GemmParams& p, hipStream_t stream) { return launch_gemm<kGateUp>(p, stream); }
int launch_down(const GemmParams& p, hipStream_t stream) { return launch_gemm<kDown>(p, stream); }

int launch_combine(const int16_t* slots, const float* slot_scale, int nslots, uint16_t* out, int T, int H,
                   const uint8_t* valid, const int64_t* ids, int topk, int E, hipStream_t stream) {
  const long n4 = (long)T * (H / 4);
  if (n4 == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(H % kSlotBlock == 0, JANUS_MOE_EINVAL, "combine: H=%d is not a multiple of %d", H, kSlotBlock);
  JANUS_REQUIRE(!ids || (topk > 0 && topk <= 32), JANUS_MOE_EINVAL, "combine: top_k=%d with id checks (at most 32)",
                topk);
  long blocks = (n4 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (ids)
    hipLaunchKernelGGL(combine_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       reinterpret_cast<const uint2*>(slots), slot_scale, nslots, reinterpret_cast<uint2*>(out), T,
                       H / 4, valid, ids, topk, E);
  else
    hipLaunchKernelGGL(combine_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       reinterpret_cast<const uint2*>(slots), slot_scale, nslots, reinterpret_cast<uint2*>(out), T,
                       H / 4, valid, nullptr, 0, 0);
  JANUS_LAUNCH_CHECK("combine");
  return JANUS_MOE_OK;
}

int launch_dequant_nvfp4(const uint8_t* q, const uint8_t* s, const float* gs, long rows, int K, uint16_t* out,
                         hipStream_t stream) {
  const long words = rows * (K / 8);
  if (words == 0) return JANUS_MOE_OK;
  long blocks = (words + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL(dequant_nvfp4_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     reinterpret_cast<const uint32_t*>(q), s, gs, rows, K, reinterpret_cast<bf16x8*>(out));
  JANUS_LAUNCH_CHECK("dequant_nvfp4");
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
