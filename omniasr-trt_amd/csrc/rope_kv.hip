// RoPE + KV-cache append for gfx950.
//
// Work of ``kernels.rope_kv`` / ``_rope_kv`` (src/omniasr_trt/kernels.py:294-306, 31-54) with the
// rounding of ``apply_rope`` (src/omniasr_trt/modeling.py:301-306): each product is rounded to fp32
// on its own and the difference / sum rounded again (PyTorch evaluates ``re * c - im * s`` as three
// element-wise kernels), then the result is rounded to the element type.  The Triton kernel fuses
// the products into FMAs; PyTorch does not, and the PyTorch rounding is the one reproduced here,
// so bf16 outputs are bit-identical to ``apply_rope``.
//
// Layout: one thread moves 16 bytes of q, of k and of v (8 bf16 = 4 rotation pairs, or 4 fp32 = 2
// pairs) with 128-bit loads and stores; a block covers 256 such pieces of one token; the grid is
// (tokens, pieces / 256).  Work per token is 3*H*D elements in and out, so at decode sizes the
// launch is latency-bound and at prefill sizes HBM-bound.
#include "common.h"

namespace omni {

template <typename Elem>
struct RopeVec;

template <>
struct RopeVec<uint16_t> {  // bf16: 8 elements = 4 pairs in 16 bytes
  static constexpr int kElems = 8;
  __device__ static void load(const uint16_t* p, float* f) {
    u32x4_t v = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = bf16x8_elem(v, e);
  }
  __device__ static void store(uint16_t* p, const float* f) {
    u32x4_t v;
#pragma unroll
    for (int w = 0; w < 4; ++w) v[w] = pack_bf16x2(f[2 * w], f[2 * w + 1]);
    *reinterpret_cast<u32x4_t*>(p) = v;
  }
  typedef u32x4_t Raw;  // 16 bytes moved as they are
  __device__ static Raw raw(const uint16_t* p) { return *reinterpret_cast<const u32x4_t*>(p); }
  __device__ static void store_raw(uint16_t* p, Raw v) { *reinterpret_cast<u32x4_t*>(p) = v; }
};

template <>
struct RopeVec<float> {  // fp32: 4 elements = 2 pairs in 16 bytes
  static constexpr int kElems = 4;
  __device__ static void load(const float* p, float* f) {
    f32x4_t v = *reinterpret_cast<const f32x4_t*>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = v[e];
  }
  __device__ static void store(float* p, const float* f) {
    f32x4_t v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = f[e];
    *reinterpret_cast<f32x4_t*>(p) = v;
  }
  typedef u32x4_t Raw;
  __device__ static Raw raw(const float* p) { return *reinterpret_cast<const u32x4_t*>(p); }
  __device__ static void store_raw(float* p, Raw v) { *reinterpret_cast<u32x4_t*>(p) = v; }
};

// (re, im) -> (re*c - im*s, re*s + im*c), every operation rounded separately.
__device__ __forceinline__ void rotate_pair(float re, float im, float c, float s, float& o_re,
                                            float& o_im) {
#pragma clang fp contract(off)
  const float a = re * c;
  const float b = im * s;
  const float d = re * s;
  const float e = im * c;
  o_re = a - b;
  o_im = d + e;
}

template <typename Elem>
__global__ __launch_bounds__(256) void rope_kv_append_kernel(
    const Elem* __restrict__ qkv, int64_t qkv_row_stride, const float* __restrict__ cs,
    int64_t cs_rows, const int64_t* __restrict__ pos, const int64_t* __restrict__ slots,
    const int64_t* __restrict__ cache_pos, Elem* __restrict__ q_out, Elem* __restrict__ k_cache,
    Elem* __restrict__ v_cache, int64_t stride_row, int64_t stride_head, int64_t stride_pos,
    int64_t cache_rows, int64_t cache_len, int heads, int head_dim) {
  using V = RopeVec<Elem>;
  constexpr int kE = V::kElems;
  const int per_head = head_dim / kE;
  const int piece = blockIdx.y * blockDim.x + threadIdx.x;
  if (piece >= heads * per_head) return;
  const int64_t n = blockIdx.x;
  const int h = piece / per_head;
  const int e0 = (piece - h * per_head) * kE;  // first element of this thread's 16 bytes

  // Every load that does not depend on a loaded value is issued first (the token's q, k and v, its position, cache
  // row and cache position); only the cos / sin row waits for the position.
  const Elem* row = qkv + n * qkv_row_stride + (int64_t)h * head_dim + e0;
  const int64_t hd = (int64_t)heads * head_dim;
  float xq[kE], xk[kE];
  V::load(row, xq);
  V::load(row + hd, xk);
  typename V::Raw vraw = V::raw(row + 2 * hd);
  const int64_t p = pos[n];
  const int64_t r = slots ? slots[n] : n;
  const int64_t cp = cache_pos ? cache_pos[n] : p;
  const int64_t pt = clamp64(p, 0, cs_rows - 1);  // table row (valid positions never clamp)
  // cs[p] holds (c, s) of pair j at floats 2j, 2j+1: this thread's pairs are floats e0 .. e0+kE-1.
  const f32x4_t* csr = reinterpret_cast<const f32x4_t*>(cs + pt * head_dim + e0);
  float c[kE / 2], s[kE / 2];
#pragma unroll
  for (int w = 0; w < kE / 4; ++w) {
    const f32x4_t t = csr[w];
    c[2 * w] = t[0];
    s[2 * w] = t[1];
    c[2 * w + 1] = t[2];
    s[2 * w + 1] = t[3];
  }

  float y[kE];

  // q
#pragma unroll
  for (int j = 0; j < kE / 2; ++j) rotate_pair(xq[2 * j], xq[2 * j + 1], c[j], s[j], y[2 * j], y[2 * j + 1]);
  V::store(q_out + (n * heads + h) * (int64_t)head_dim + e0, y);

  if (r < 0 || r >= cache_rows || cp < 0 || cp >= cache_len) return;  // outside the cache: no write
  const int64_t off = r * stride_row + (int64_t)h * stride_head + cp * stride_pos + e0;

  // k
#pragma unroll
  for (int j = 0; j < kE / 2; ++j) rotate_pair(xk[2 * j], xk[2 * j + 1], c[j], s[j], y[2 * j], y[2 * j + 1]);
  V::store(k_cache + off, y);
  // v: copied as it is
  V::store_raw(v_cache + off, vraw);
}

}  // namespace omni

using namespace omni;

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int omni_rope_kv_append(const void* qkv, int64_t qkv_row_stride, const float* cs,
                                   int64_t cs_rows, const int64_t* pos, const int64_t* slots,
                                   const int64_t* cache_pos, void* q_out, void* k_cache,
                                   void* v_cache, int64_t stride_row, int64_t stride_head,
                                   int64_t stride_pos, int64_t cache_rows, int64_t cache_len,
                                   int64_t n_tokens, int32_t heads, int32_t head_dim, int32_t dtype,
                                   void* stream) {
  if (n_tokens < 0 || heads <= 0 || head_dim <= 0) return OMNI_ERR_INVALID;
  if (n_tokens == 0) return OMNI_OK;
  if (!qkv || !cs || !pos || !q_out || !k_cache || !v_cache) return OMNI_ERR_INVALID;
  if (head_dim % 8 != 0) return OMNI_ERR_SHAPE;
  if (cs_rows <= 0 || cache_rows <= 0 || cache_len <= 0) return OMNI_ERR_INVALID;
  if (n_tokens > 0x7fffffffLL) return OMNI_ERR_INVALID;
  int esize;
  if (dtype == OMNI_BF16) esize = 2;
  else if (dtype == OMNI_F32) esize = 4;
  else return OMNI_ERR_DTYPE;
  const int ev = 16 / esize;  // elements per 16 bytes
  // 128-bit accesses: every row / head / position start must be 16-byte aligned.
  if (!aligned16(qkv) || !aligned16(q_out) || !aligned16(k_cache) || !aligned16(v_cache) ||
      !aligned16(cs))
    return OMNI_ERR_INVALID;
  if (qkv_row_stride % ev || stride_row % ev || stride_head % ev || stride_pos % ev)
    return OMNI_ERR_INVALID;
  if (qkv_row_stride < 3LL * heads * head_dim) return OMNI_ERR_INVALID;
  const int pieces = heads * (head_dim / ev);
  dim3 grid((unsigned)n_tokens, (unsigned)((pieces + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == OMNI_BF16) {
    rope_kv_append_kernel<uint16_t><<<grid, 256, 0, s>>>(
        (const uint16_t*)qkv, qkv_row_stride, cs, cs_rows, pos, slots, cache_pos, (uint16_t*)q_out,
        (uint16_t*)k_cache, (uint16_t*)v_cache, stride_row, stride_head, stride_pos, cache_rows,
        cache_len, heads, head_dim);
  } else {
    rope_kv_append_kernel<float><<<grid, 256, 0, s>>>(
        (const float*)qkv, qkv_row_stride, cs, cs_rows, pos, slots, cache_pos, (float*)q_out,
        (float*)k_cache, (float*)v_cache, stride_row, stride_head, stride_pos, cache_rows,
        cache_len, heads, head_dim);
  }
  return omni_launch_status();
}
