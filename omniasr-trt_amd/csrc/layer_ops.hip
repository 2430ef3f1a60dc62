// The step's element-wise layer ops for gfx950, each one launch where torch takes one or two:
//   rms_norm   y = x * rsqrt(mean(x^2) + eps) * w per row (F.rms_norm, src/omniasr_trt/modeling.py's RMSNorm);
//   silu_mul   out = inner * silu(gate) for the fused gate|inner projection's halves (decode.py:34-54's layout,
//              the FFN of SpecDecoder.step, src/omniasr_trt/spec.py:97-106).
// bf16 in and out, fp32 arithmetic.  rms_norm rounds once, after both products, as F.rms_norm does, but adds the
// row's squares in its own order (fused multiply-adds per thread, then a wave and workgroup reduction): where that
// sum differs from torch's in its last bit, rsqrt can too, and an output can round to the neighbouring bf16 value
// (measured: ~3 of 10^6 elements); silu_mul rounds silu(gate) to bf16 and then the product, as torch's two kernels
// do, bit for bit.  At step sizes ([40, 4096],
// [40, 2 x 11008]) both are a few hundred KB, so they are latency-bound: one workgroup per row for the norm (the
// row's sum of squares in registers, one LDS reduction), one thread per 8 outputs for silu_mul.
#include <math.h>

#include "common.h"

namespace omni {

constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;  // 16-byte chunks per thread: dim <= 256 x 4 x 8 = 8192

__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                                const uint16_t* __restrict__ w, uint16_t* y,
                                                                int64_t y_stride, int dim, float eps) {
  __shared__ float part[kNormThreads / kWave];
  const int tid = threadIdx.x;
  const uint16_t* xr = x + (int64_t)blockIdx.x * x_stride;
  u32x4_t v[kNormChunks], wv[kNormChunks];  // the weights load with x: one memory round trip, not two
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int i = (tid + c * kNormThreads) * 8;
    v[c] = i < dim ? *reinterpret_cast<const u32x4_t*>(xr + i) : u32x4_t{0u, 0u, 0u, 0u};
    wv[c] = i < dim ? *reinterpret_cast<const u32x4_t*>(w + i) : u32x4_t{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = bf16x8_elem(v[c], e);
      ss = __builtin_fmaf(f, f, ss);
    }
  }
  ss = wave_sum(ss);
  if (lane_id() == 0) part[tid / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / kWave; ++i) tot += part[i];  // the same order in every thread
  const float rstd = rsqrtf(tot / (float)dim + eps);
  uint16_t* yr = y + (int64_t)blockIdx.x * y_stride;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int i = (tid + c * kNormThreads) * 8;
    if (i >= dim) continue;
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = pack_bf16x2(bf16x8_elem(v[c], 2 * q) * rstd * bf16x8_elem(wv[c], 2 * q),
                         bf16x8_elem(v[c], 2 * q + 1) * rstd * bf16x8_elem(wv[c], 2 * q + 1));
    *reinterpret_cast<u32x4_t*>(yr + i) = o;
  }
}

__device__ __forceinline__ float silu_bf16(float g) { return round_through_bf16(g / (1.f + expf(-g))); }

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gi, int64_t gi_stride,
                                                       uint16_t* out, int64_t out_stride, int rows, int ffn) {
  const int per_row = ffn / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)rows * per_row) return;
  const int64_t row = idx / per_row;
  const int col = (int)(idx - row * per_row) * 8;
  const uint16_t* gr = gi + row * gi_stride;
  const u32x4_t gate = *reinterpret_cast<const u32x4_t*>(gr + col);
  const u32x4_t inner = *reinterpret_cast<const u32x4_t*>(gr + ffn + col);
  u32x4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = pack_bf16x2(bf16x8_elem(inner, 2 * q) * silu_bf16(bf16x8_elem(gate, 2 * q)),
                       bf16x8_elem(inner, 2 * q + 1) * silu_bf16(bf16x8_elem(gate, 2 * q + 1)));
  *reinterpret_cast<u32x4_t*>(out + row * out_stride + col) = o;
}

}  // namespace omni

extern "C" int omni_rms_norm(const void* x, int64_t x_stride, const void* weight, void* y, int64_t y_stride,
                             int32_t rows, int32_t dim, float eps, int32_t dtype, void* stream) {
  if (dtype != OMNI_BF16) return OMNI_ERR_DTYPE;
  if (rows < 0 || dim < 0) return OMNI_ERR_INVALID;
  if (dim % 8 != 0 || dim > omni::kNormThreads * omni::kNormChunks * 8) return OMNI_ERR_SHAPE;
  if (rows == 0 || dim == 0) return OMNI_OK;
  if (!x || !weight || !y || x_stride < dim || y_stride < dim || x_stride % 8 || y_stride % 8) return OMNI_ERR_INVALID;
  omni::rms_norm_kernel<<<rows, omni::kNormThreads, 0, (hipStream_t)stream>>>(
      static_cast<const uint16_t*>(x), x_stride, static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(y),
      y_stride, dim, eps);
  return omni_launch_status();
}

extern "C" int omni_silu_mul(const void* gate_inner, int64_t gate_inner_stride, void* out, int64_t out_stride,
                             int32_t rows, int32_t ffn, int32_t dtype, void* stream) {
  if (dtype != OMNI_BF16) return OMNI_ERR_DTYPE;
  if (rows < 0 || ffn < 0) return OMNI_ERR_INVALID;
  if (ffn % 8 != 0) return OMNI_ERR_SHAPE;
  if (rows == 0 || ffn == 0) return OMNI_OK;
  if (!gate_inner || !out || gate_inner_stride < 2 * (int64_t)ffn || out_stride < ffn || gate_inner_stride % 8 ||
      out_stride % 8)
    return OMNI_ERR_INVALID;
  const int64_t items = (int64_t)rows * (ffn / 8);
  omni::silu_mul_kernel<<<(unsigned)((items + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      static_cast<const uint16_t*>(gate_inner), gate_inner_stride, static_cast<uint16_t*>(out), out_stride, rows,
      ffn);
  return omni_launch_status();
}
