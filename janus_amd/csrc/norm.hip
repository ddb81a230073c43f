// The MoE layer's neighbours on the serving path (janus/hybrid.py:1077-1105, `_serve_level`): before it,
// `_add_norm(x, h_attn, post_attention_layernorm)`; after it, the next `_add_norm(x, moe_out, next norm, valid)`
// (janus/hybrid.py:250-273). One wave per token row: the row's values stay in registers between the residual add and
// the normalisation, so a row is read once and written once.
//   residual add: x = bf16(fp32(residual) + fp32(h)), torch's bf16 add (one rounding of the exact fp32 sum);
//   Qwen3_5RMSNorm: n = bf16(fp32(x) * rsqrt(mean(fp32(x)^2) + eps) * (1 + fp32(w))), the products in that order;
//   n is 0 where valid[t] == 0 (the DeltaNet input mask).
// Lane l of the wave holds columns 4 (l + 64 j) .. +3, j < NV, so every load is a coalesced 8-byte (bf16) or 16-byte
// (fp32 slot) access; the sum of squares is reduced in a fixed lane order, so the standalone kernel and the fused
// combine give the same bits.
#include "norm.h"
#include "gemm.h"

namespace janus {
namespace {

constexpr int kNormWaves = 4;  // token rows per workgroup

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// The normalisation of a row held as fp32 values of its bf16 x (v[j][0..3] = columns 4 (lane + 64 j) .. +3), written
// as bf16 to n_row. ncol4 = H / 4.
// The lane's norm weights (columns 4 (lane + 64 j) .. +3), loaded before the row's other reads are used.
template <int NV>
__device__ __forceinline__ void load_norm_weights(const uint16_t* __restrict__ w, int ncol4, uint2 (&wb)[NV]) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c4 = lane + kWave * j;
    wb[j] = c4 < ncol4 ? *reinterpret_cast<const uint2*>(w + 4 * c4) : make_uint2(0u, 0u);
  }
}

template <int NV>
__device__ __forceinline__ void rmsnorm_row(const float (&v)[NV][4], int H, int ncol4, const uint2 (&wbs)[NV],
                                            float eps, bool keep, uint16_t* n_row) {
  const int lane = threadIdx.x & (kWave - 1);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) ss = fmaf(v[j][i], v[j][i], ss);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float rs = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c4 = lane + kWave * j;
    if (c4 >= ncol4) continue;
    const uint2 wb = wbs[j];
    const float wv[4] = {bf16_to_f32(wb.x & 0xFFFFu), bf16_to_f32(wb.x >> 16), bf16_to_f32(wb.y & 0xFFFFu),
                         bf16_to_f32(wb.y >> 16)};
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = keep ? (v[j][i] * rs) * (1.0f + wv[i]) : 0.f;
    *reinterpret_cast<uint2*>(n_row + 4 * c4) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
  }
}

template <int NV>
__global__ void __launch_bounds__(kNormWaves * kWave) add_rmsnorm_kernel(
    const uint16_t* residual, const uint16_t* h, const uint16_t* __restrict__ w, float eps,
    const uint8_t* __restrict__ valid, int T, int H, uint16_t* x_out, uint16_t* n_out) {  // x_out/residual, n_out/h may alias
  const int lane = threadIdx.x & (kWave - 1);
  const long t = (long)blockIdx.x * kNormWaves + threadIdx.x / kWave;
  if (t >= T) return;  // whole waves; no barriers
  const int ncol4 = H / 4;
  uint2 wb[NV], rbs[NV], hbs[NV];
  load_norm_weights<NV>(w, ncol4, wb);
  // every load of the row before the first store: the outputs may alias the inputs (an element is read and written by
  // the same lane only), so the compiler would otherwise wait for each column group's loads in turn
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c4 = lane + kWave * j;
    rbs[j] = c4 < ncol4 ? *reinterpret_cast<const uint2*>(residual + t * H + 4 * c4) : make_uint2(0u, 0u);
    hbs[j] = (h && c4 < ncol4) ? *reinterpret_cast<const uint2*>(h + t * H + 4 * c4) : make_uint2(0u, 0u);
  }
  float v[NV][4];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c4 = lane + kWave * j;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[j][i] = 0.f;
    if (c4 >= ncol4) continue;
    const uint2 rb = rbs[j];
    float x[4] = {bf16_to_f32(rb.x & 0xFFFFu), bf16_to_f32(rb.x >> 16), bf16_to_f32(rb.y & 0xFFFFu),
                  bf16_to_f32(rb.y >> 16)};
    if (h) {
      const uint2 hb = hbs[j];
      x[0] += bf16_to_f32(hb.x & 0xFFFFu);
      x[1] += bf16_to_f32(hb.x >> 16);
      x[2] += bf16_to_f32(hb.y & 0xFFFFu);
      x[3] += bf16_to_f32(hb.y >> 16);
    }
    const uint2 xb = make_uint2(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]));
    v[j][0] = bf16_to_f32(xb.x & 0xFFFFu);
    v[j][1] = bf16_to_f32(xb.x >> 16);
    v[j][2] = bf16_to_f32(xb.y & 0xFFFFu);
    v[j][3] = bf16_to_f32(xb.y >> 16);
    if (x_out) *reinterpret_cast<uint2*>(x_out + t * H + 4 * c4) = xb;
  }
  rmsnorm_row<NV>(v, H, ncol4, wb, eps, !valid || valid[t], n_out + t * H);
}

// The combine with the next residual add and norm: moe = bf16(sum_j slots[t, j]) in slot order (the plain combine's
// value), x = bf16(x_res + moe) written back over x_res, n = the norm of x. A token the MoE skipped (moe_valid[t] == 0)
// contributes moe = 0 and its slots are not read. The slots are read kSlotBatch at a time for all of the lane's
// columns, so a row costs ceil(nslots / kSlotBatch) memory round trips (one slot at a time for rows past 2048
// columns, whose registers would not allow two waves per SIMD otherwise).
template <int NV>
__global__ void __launch_bounds__(kNormWaves * kWave) combine_add_rmsnorm_kernel(
    const uint2* __restrict__ slots, const float* __restrict__ scales, int nslots,
    const uint8_t* __restrict__ moe_valid, uint16_t* x_res, const uint16_t* __restrict__ w, float eps,
    const uint8_t* __restrict__ valid, int T, int H, uint16_t* n_out) {
  const int lane = threadIdx.x & (kWave - 1);
  const long t = (long)blockIdx.x * kNormWaves + threadIdx.x / kWave;
  if (t >= T) return;
  const int ncol4 = H / 4;
  const bool routed = !moe_valid || moe_valid[t];
  uint2 wb[NV], rb[NV];
  load_norm_weights<NV>(w, ncol4, wb);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c4 = lane + kWave * j;
    rb[j] = c4 < ncol4 ? *reinterpret_cast<const uint2*>(x_res + t * H + 4 * c4) : make_uint2(0u, 0u);
  }
  constexpr int kSlotBatch = NV <= 8 ? 3 : 1;
  float4 s[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) s[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (routed) {
    // the lane's column group c4 = lane + 64 j sits at its stored position within its scale block
    constexpr int kGroups = kSlotBlock / 4;
    const int nblk = ncol4 / kGroups;
    const long row0 = t * nslots;
    const int q = (lane & ~(kGroups - 1)) | slot_stored_group(lane & (kGroups - 1));
    for (int k0 = 0; k0 < nslots; k0 += kSlotBatch) {
      uint2 a[kSlotBatch][NV];
      float sc[kSlotBatch][NV];
#pragma unroll
      for (int kk = 0; kk < kSlotBatch; ++kk)
#pragma unroll
        for (int j = 0; j < NV; ++j)
          if (k0 + kk < nslots && lane + kWave * j < ncol4) {
            a[kk][j] = slots[(row0 + k0 + kk) * ncol4 + kWave * j + q];
            sc[kk][j] = scales[(row0 + k0 + kk) * nblk + (lane + kWave * j) / kGroups];
          }
#pragma unroll
      for (int kk = 0; kk < kSlotBatch; ++kk) {
        if (k0 + kk >= nslots) break;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
          if (lane + kWave * j >= ncol4) continue;
          const float4 d = slot_decode4(a[kk][j], sc[kk][j]);
          if (k0 + kk == 0) {
            s[j] = d;  // slot 0 starts the sum, as in the plain combine
          } else {
            s[j].x += d.x;
            s[j].y += d.y;
            s[j].z += d.z;
            s[j].w += d.w;
          }
        }
      }
    }
  }
  float v[NV][4];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c4 = lane + kWave * j;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[j][i] = 0.f;
    if (c4 >= ncol4) continue;
    const uint2 mb = make_uint2(pack_bf16x2(s[j].x, s[j].y), pack_bf16x2(s[j].z, s[j].w));  // the MoE output, bf16
    const float x[4] = {bf16_to_f32(rb[j].x & 0xFFFFu) + bf16_to_f32(mb.x & 0xFFFFu),
                        bf16_to_f32(rb[j].x >> 16) + bf16_to_f32(mb.x >> 16),
                        bf16_to_f32(rb[j].y & 0xFFFFu) + bf16_to_f32(mb.y & 0xFFFFu),
                        bf16_to_f32(rb[j].y >> 16) + bf16_to_f32(mb.y >> 16)};
    const uint2 xb = make_uint2(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]));
    v[j][0] = bf16_to_f32(xb.x & 0xFFFFu);
    v[j][1] = bf16_to_f32(xb.x >> 16);
    v[j][2] = bf16_to_f32(xb.y & 0xFFFFu);
    v[j][3] = bf16_to_f32(xb.y >> 16);
    *reinterpret_cast<uint2*>(x_res + t * H + 4 * c4) = xb;
  }
  rmsnorm_row<NV>(v, H, ncol4, wb, eps, !valid || valid[t], n_out + t * H);
}

}  // namespace

int check_norm_sizes(int T, int H) {
  JANUS_REQUIRE(T >= 0 && H > 0 && H % 4 == 0 && H <= kMaxNormH, JANUS_MOE_EINVAL,
                "rmsnorm: unsupported sizes T=%d H=%d (need H %% 4 == 0, H <= %d)", T, H, kMaxNormH);
  return JANUS_MOE_OK;
}

#define JANUS_NORM_CASES(KERNEL, ...)                                                                             \
  switch (ceil_div(H, 4 * kWave)) {                                                                              \
    case 1: hipLaunchKernelGGL(KERNEL<1>, g, b, 0, stream, __VA_ARGS__); break;                                   \
    case 2: hipLaunchKernelGGL(KERNEL<2>, g, b, 0, stream, __VA_ARGS__); break;                                   \
    case 3: case 4: hipLaunchKernelGGL(KERNEL<4>, g, b, 0, stream, __VA_ARGS__); break;                           \
    case 5: case 6: case 7: case 8: hipLaunchKernelGGL(KERNEL<8>, g, b, 0, stream, __VA_ARGS__); break;           \
    default: hipLaunchKernelGGL(KERNEL<16>, g, b, 0, stream, __VA_ARGS__); break;                                 \
  }

int launch_add_rmsnorm(const uint16_t* residual, const uint16_t* h, const uint16_t* w, float eps, const uint8_t* valid,
                       int T, int H, uint16_t* x_out, uint16_t* n_out, hipStream_t stream) {
  if (T == 0) return JANUS_MOE_OK;
  const dim3 g(ceil_div(T, kNormWaves)), b(kNormWaves * kWave);
  JANUS_NORM_CASES(add_rmsnorm_kernel, residual, h, w, eps, valid, T, H, x_out, n_out)
  JANUS_LAUNCH_CHECK("add_rmsnorm");
  return JANUS_MOE_OK;
}

int launch_combine_add_rmsnorm(const int16_t* slots, const float* slot_scale, int nslots, const uint8_t* moe_valid,
                               uint16_t* x_res, const uint16_t* w, float eps, const uint8_t* valid, int T, int H,
                               uint16_t* n_out, hipStream_t stream) {
  if (T == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(H % kSlotBlock == 0, JANUS_MOE_EINVAL, "combine_add_rmsnorm: H=%d is not a multiple of %d", H,
                kSlotBlock);
  const dim3 g(ceil_div(T, kNormWaves)), b(kNormWaves * kWave);
  JANUS_NORM_CASES(combine_add_rmsnorm_kernel, reinterpret_cast<const uint2*>(slots), slot_scale, nslots, moe_valid,
                   x_res, w, eps, valid, T, H, n_out)
  JANUS_LAUNCH_CHECK("combine_add_rmsnorm");
  return JANUS_MOE_OK;
}
#undef JANUS_NORM_CASES

}  // namespace janus

using namespace janus;

extern "C" int janus_moe_add_rmsnorm(const uint16_t* residual, const uint16_t* h, const uint16_t* weight, float eps,
                                     const uint8_t* valid, int T, int H, uint16_t* x_out, uint16_t* n_out,
                                     janus_stream_t stream) {
  int rc = check_norm_sizes(T, H);
  if (rc) return rc;
  if (T == 0) return JANUS_MOE_OK;
  JANUS_REQUIRE(residual && weight && n_out, JANUS_MOE_EINVAL, "janus_moe_add_rmsnorm: null pointer");
  JANUS_REQUIRE(eps >= 0.f, JANUS_MOE_EINVAL, "janus_moe_add_rmsnorm: eps=%g must not be negative", (double)eps);
  return launch_add_rmsnorm(residual, h, weight, eps, valid, T, H, x_out, n_out, (hipStream_t)stream);
}
