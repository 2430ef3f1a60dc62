// Greedy argmax of the verify logits and acceptance / rollback of a drafted step, for gfx950.
//
// argmax: ``F.log_softmax(logits, -1).argmax(-1)`` (src/omniasr_trt/spec.py:107,
// src/omniasr_trt/decode.py:219).  PyTorch's log-softmax evaluates (x_i - max) - log(sum exp(x_j -
// max)) in fp32 and rounds it to the logits' type; argmax then takes the first index of the maximum
// of those rounded values.  The rounding is monotone in x_i and x_i = max gives round(-lse), so the
// result is the first index whose rounded log-probability equals round(-lse) -- for bf16 logits not
// necessarily the index of the largest logit: rounding merges near-top values into one bucket and
// the lowest index of that bucket wins.
//
// accept: ``_accept`` (src/omniasr_trt/kernels.py:271-291).
//
// Layout: the argmax takes one 256-thread workgroup per logit row (row_argmax_kernel): 128-bit loads of
// the whole row issued together, max, sum and first index reduced through wave shuffles and LDS; then
// accept_kernel accepts each slot with one thread.  Without an argmax output, or for vocabularies past
// what 16 chunks per thread of 256 threads cover, one 1024-thread workgroup per slot reads the slot's T
// rows in turn and its first lane accepts (greedy_accept_kernel): one launch, but the rows of a slot in
// sequence, which costs more than the second launch.
#include <limits.h>
#include <math.h>

#include "common.h"

namespace omni {

struct AcceptArgs {
  const int64_t* tokens;  // [rows, T] fed tokens
  const int64_t* nxt_in;  // [rows, T] argmaxes (omni_accept) or NULL (computed here)
  int64_t* nxt_out;       // [rows, T] or NULL
  int32_t* out;
  int64_t out_stride, out_cap;
  int64_t* tok;
  int64_t* last;
  uint8_t* done;
  int64_t* draft_next;  // NULL: not tracked
  const int64_t* start;
  const uint8_t* use_draft;
  int T;
  int64_t limit, eos;
  // logits (omni_greedy_accept)
  const void* logits;
  int64_t logits_stride;
  int vocab;
};

// Acceptance of row b given its argmaxes g(j); one thread.
template <typename G>
__device__ void accept_row(const AcceptArgs& a, int b, G g) {
  if (a.done[b]) return;
  const int T = a.T;
  const int64_t p = a.last[b] + 1;
  int kept = T - 1;  // leading fed tokens equal to the argmax before them
  for (int j = 0; j < T - 1; ++j) {
    if (a.tokens[(int64_t)b * T + j + 1] != g(j)) {
      kept = j;
      break;
    }
  }
  int n = kept;
  bool ended = false;
  for (int j = 0; j <= kept; ++j) {
    if (g(j) == a.eos || p + j >= a.limit) {
      n = j;
      ended = true;
      break;
    }
  }
  int32_t* orow = a.out + (int64_t)b * a.out_stride;
  for (int j = 0; j <= n; ++j) {
    const int64_t at = (p + j) < (a.out_cap - 1) ? (p + j) : (a.out_cap - 1);
    orow[at] = (int32_t)g(j);
  }
  a.tok[b] = g(n);
  a.last[b] = p + n;
  a.done[b] = ended ? 1 : 0;
  if (a.draft_next) {
    const int64_t base = a.use_draft[b] ? a.start[b] : a.draft_next[b];
    a.draft_next[b] = base + n + 1;
  }
}

__global__ __launch_bounds__(64) void accept_kernel(AcceptArgs a, int rows) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= rows) return;
  const int64_t* g = a.nxt_in + (int64_t)b * a.T;
  accept_row(a, b, [g](int j) { return g[j]; });
}

// ---------------------------------------------------------------------------------------------- argmax

template <typename L>
struct LogitChunk;

template <>
struct LogitChunk<uint16_t> {  // bf16: 8 values per 16 bytes
  static constexpr int kElems = 8;
  __device__ static float get(const u32x4_t& v, int e) { return bf16x8_elem(v, e); }
  __device__ static float round(float f) { return round_through_bf16(f); }
  __device__ static float scalar(const uint16_t* p) { return bf16_to_f32(*p); }
  // 8 values from an address that need not be 16-byte aligned
  __device__ static u32x4_t gather(const uint16_t* p) {
    u32x4_t v;
#pragma unroll
    for (int w = 0; w < 4; ++w) v[w] = (uint32_t)p[2 * w] | ((uint32_t)p[2 * w + 1] << 16);
    return v;
  }
};

template <>
struct LogitChunk<float> {  // fp32: 4 values per 16 bytes
  static constexpr int kElems = 4;
  __device__ static float get(const u32x4_t& v, int e) { return __uint_as_float(v[e]); }
  __device__ static float round(float f) { return f; }
  __device__ static float scalar(const float* p) { return *p; }
  __device__ static u32x4_t gather(const float* p) {
    u32x4_t v;
#pragma unroll
    for (int w = 0; w < 4; ++w) v[w] = __float_as_uint(p[w]);
    return v;
  }
};

constexpr int kAcceptThreads = 1024;
constexpr int kAcceptWaves = kAcceptThreads / kWave;

// Block-wide reductions of one value per row (rows < RG); ``red`` holds kAcceptWaves * RG entries.
template <int RG, typename F, typename Op>
__device__ __forceinline__ void block_reduce_rows(F (&v)[RG], F* red, Op op) {
  const int lane = lane_id(), wave = threadIdx.x / kWave;
#pragma unroll
  for (int r = 0; r < RG; ++r) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v[r] = op(v[r], __shfl_xor(v[r], o, kWave));
    if (lane == 0) red[wave * RG + r] = v[r];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    F x = red[r];
    for (int w = 1; w < kAcceptWaves; ++w) x = op(x, red[w * RG + r]);
    v[r] = x;
  }
  __syncthreads();
}

// KPT: 16-byte chunks per thread per row; RG: rows processed together; ALIGNED: rows start on 16 bytes (else
// every chunk is gathered with element loads).
template <typename L, int KPT, int RG, bool ALIGNED>
__global__ __launch_bounds__(kAcceptThreads) void greedy_accept_kernel(AcceptArgs a) {
  using C = LogitChunk<L>;
  constexpr int kE = C::kElems;
  __shared__ float redf[kAcceptWaves * RG];
  __shared__ int redi[kAcceptWaves * RG];
  __shared__ int64_t gsh[64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int T = a.T, V = a.vocab;
  const int nchunks = V / kE;  // whole 16-byte chunks; the tail (V % kE values) is read scalar
  const L* base = reinterpret_cast<const L*>(a.logits);

  for (int r0 = 0; r0 < T; r0 += RG) {
    u32x4_t x[RG][KPT];
    const L* rowp[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {  // rows past T (uniform) are neither read nor used
      const bool rv = r0 + r < T;
      rowp[r] = base + ((int64_t)b * T + (rv ? r0 + r : 0)) * a.logits_stride;
#pragma unroll
      for (int k = 0; k < KPT; ++k) {
        const int ci = tid + k * kAcceptThreads;
        const bool ok = rv && ci < nchunks;
        if constexpr (ALIGNED)
          x[r][k] = ok ? reinterpret_cast<const u32x4_t*>(rowp[r])[ci] : u32x4_t{0u, 0u, 0u, 0u};
        else
          x[r][k] = ok ? C::gather(rowp[r] + (int64_t)ci * kE) : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    const int tail0 = nchunks * kE;  // first tail index
    const bool has_tail = tid < V - tail0;
    float tail[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) tail[r] = has_tail && r0 + r < T ? C::scalar(rowp[r] + tail0 + tid) : -INFINITY;

    // max
    float m[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      float v = tail[r];
#pragma unroll
      for (int k = 0; k < KPT; ++k)
        if (tid + k * kAcceptThreads < nchunks) {
#pragma unroll
          for (int e = 0; e < kE; ++e) v = fmaxf(v, C::get(x[r][k], e));
        }
      m[r] = v;
    }
    block_reduce_rows<RG>(m, redf, [](float p, float q) { return fmaxf(p, q); });
    // sum of exp(x - max)
    float s[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      float v = has_tail ? expf(tail[r] - m[r]) : 0.f;
#pragma unroll
      for (int k = 0; k < KPT; ++k)
        if (tid + k * kAcceptThreads < nchunks) {
#pragma unroll
          for (int e = 0; e < kE; ++e) v += expf(C::get(x[r][k], e) - m[r]);
        }
      s[r] = v;
    }
    block_reduce_rows<RG>(s, redf, [](float p, float q) { return p + q; });
    // first index whose rounded log-probability is the top one
    int first[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const float lse = logf(s[r]);
      const float top = C::round(0.f - lse);
      int best = INT_MAX;
#pragma unroll
      for (int k = 0; k < KPT; ++k) {
        const int ci = tid + k * kAcceptThreads;
        if (ci < nchunks) {
#pragma unroll
          for (int e = kE - 1; e >= 0; --e)
            if (C::round((C::get(x[r][k], e) - m[r]) - lse) == top) best = min(best, ci * kE + e);
        }
      }
      if (has_tail && C::round((tail[r] - m[r]) - lse) == top) best = min(best, tail0 + tid);
      first[r] = best;
    }
    block_reduce_rows<RG>(first, redi, [](int p, int q) { return min(p, q); });
    if (tid == 0) {
#pragma unroll
      for (int r = 0; r < RG; ++r)
        if (r0 + r < T) gsh[r0 + r] = first[r] == INT_MAX ? 0 : first[r];
    }
  }
  __syncthreads();
  if (a.nxt_out && tid < T) a.nxt_out[(int64_t)b * T + tid] = gsh[tid];
  if (tid == 0) accept_row(a, b, [](int j) { return gsh[j]; });
}

// ---------------------------------------------------------------------------------------------- row argmax

// The argmax alone, one 256-thread workgroup per logit row (rows x T workgroups instead of rows): the same rule
// and arithmetic as greedy_accept_kernel, its result written to ``nxt_out``; accept_kernel then accepts.  Two
// short launches instead of one long one: each row's read, three reductions and compare are a fraction of what
// one workgroup per slot does for T rows in sequence.
constexpr int kRowThreads = 256;
constexpr int kRowWaves = kRowThreads / kWave;

template <typename F, typename Op>
__device__ __forceinline__ F row_reduce(F v, F* red, Op op) {
  const int lane = lane_id(), wave = threadIdx.x / kWave;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, kWave));
  if (lane == 0) red[wave] = v;
  __syncthreads();
  F x = red[0];
#pragma unroll
  for (int w = 1; w < kRowWaves; ++w) x = op(x, red[w]);
  __syncthreads();
  return x;
}

template <typename L, int KPT, bool ALIGNED>
__global__ __launch_bounds__(kRowThreads) void row_argmax_kernel(AcceptArgs a) {
  using C = LogitChunk<L>;
  constexpr int kE = C::kElems;
  __shared__ float redf[kRowWaves];
  __shared__ int redi[kRowWaves];
  const int row = blockIdx.x;  // b * T + t
  const int tid = threadIdx.x;
  const int V = a.vocab;
  const int nchunks = V / kE;
  const L* rowp = reinterpret_cast<const L*>(a.logits) + (int64_t)row * a.logits_stride;
  u32x4_t x[KPT];
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    const int ci = tid + k * kRowThreads;
    const bool ok = ci < nchunks;
    if constexpr (ALIGNED)
      x[k] = ok ? reinterpret_cast<const u32x4_t*>(rowp)[ci] : u32x4_t{0u, 0u, 0u, 0u};
    else
      x[k] = ok ? C::gather(rowp + (int64_t)ci * kE) : u32x4_t{0u, 0u, 0u, 0u};
  }
  const int tail0 = nchunks * kE;
  const bool has_tail = tid < V - tail0;
  const float tail = has_tail ? C::scalar(rowp + tail0 + tid) : -INFINITY;
  float m = tail;
#pragma unroll
  for (int k = 0; k < KPT; ++k)
    if (tid + k * kRowThreads < nchunks) {
#pragma unroll
      for (int e = 0; e < kE; ++e) m = fmaxf(m, C::get(x[k], e));
    }
  m = row_reduce(m, redf, [](float p, float q) { return fmaxf(p, q); });
  float sum = has_tail ? expf(tail - m) : 0.f;
#pragma unroll
  for (int k = 0; k < KPT; ++k)
    if (tid + k * kRowThreads < nchunks) {
#pragma unroll
      for (int e = 0; e < kE; ++e) sum += expf(C::get(x[k], e) - m);
    }
  sum = row_reduce(sum, redf, [](float p, float q) { return p + q; });
  const float lse = logf(sum);
  const float top = C::round(0.f - lse);
  int best = INT_MAX;
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    const int ci = tid + k * kRowThreads;
    if (ci < nchunks) {
#pragma unroll
      for (int e = kE - 1; e >= 0; --e)
        if (C::round((C::get(x[k], e) - m) - lse) == top) best = min(best, ci * kE + e);
    }
  }
  if (has_tail && C::round((tail - m) - lse) == top) best = min(best, tail0 + tid);
  best = row_reduce(best, redi, [](int p, int q) { return min(p, q); });
  if (tid == 0) a.nxt_out[row] = best == INT_MAX ? 0 : best;
}

}  // namespace omni

using namespace omni;

static int accept_common_check(const int64_t* tokens, int32_t* out, int64_t out_stride, int64_t out_cap,
                               int64_t* tok, int64_t* last, uint8_t* done, int64_t* draft_next,
                               const int64_t* start, const uint8_t* use_draft, int32_t rows, int32_t T) {
  if (rows < 0) return OMNI_ERR_INVALID;
  if (T < 1 || T > 64) return OMNI_ERR_SHAPE;
  if (rows == 0) return OMNI_OK;
  if (!tokens || !out || !tok || !last || !done) return OMNI_ERR_INVALID;
  if (out_cap <= 0 || out_stride < out_cap) return OMNI_ERR_INVALID;
  if (draft_next && (!start || !use_draft)) return OMNI_ERR_INVALID;
  return 1;  // proceed
}

static AcceptArgs make_accept_args(const int64_t* tokens, int32_t* out, int64_t out_stride, int64_t out_cap,
                                   int64_t* tok, int64_t* last, uint8_t* done, int64_t* draft_next,
                                   const int64_t* start, const uint8_t* use_draft, int32_t T,
                                   int64_t limit, int64_t eos) {
  AcceptArgs a = {};
  a.tokens = tokens;
  a.out = out;
  a.out_stride = out_stride;
  a.out_cap = out_cap;
  a.tok = tok;
  a.last = last;
  a.done = done;
  a.draft_next = draft_next;
  a.start = start;
  a.use_draft = use_draft;
  a.T = T;
  a.limit = limit;
  a.eos = eos;
  return a;
}

extern "C" int omni_accept(const int64_t* tokens, const int64_t* nxt, int32_t* out, int64_t out_stride,
                           int64_t out_cap, int64_t* tok, int64_t* last, uint8_t* done, int64_t* draft_next,
                           const int64_t* start, const uint8_t* use_draft, int32_t rows,
                           int32_t tokens_per_row, int64_t limit, int64_t eos, void* stream) {
  int st = accept_common_check(tokens, out, out_stride, out_cap, tok, last, done, draft_next, start,
                               use_draft, rows, tokens_per_row);
  if (st <= 0) return st;
  if (!nxt) return OMNI_ERR_INVALID;
  AcceptArgs a = make_accept_args(tokens, out, out_stride, out_cap, tok, last, done, draft_next, start,
                                  use_draft, tokens_per_row, limit, eos);
  a.nxt_in = nxt;
  accept_kernel<<<(rows + 63) / 64, 64, 0, (hipStream_t)stream>>>(a, rows);
  return omni_launch_status();
}

template <typename L, int KPT>
static void launch_greedy(const AcceptArgs& a, int rows, bool aligned, hipStream_t s) {
  // Rows read together: RG rows x KPT 16-byte chunks in flight per thread (<= 32 VGPRs, no spills
  // under the 128-VGPR cap of a 1024-thread workgroup).
  constexpr int RG = KPT <= 2 ? 4 : (KPT == 4 ? 2 : 1);
  if (aligned) greedy_accept_kernel<L, KPT, RG, true><<<rows, kAcceptThreads, 0, s>>>(a);
  else greedy_accept_kernel<L, KPT, RG, false><<<rows, kAcceptThreads, 0, s>>>(a);
}

extern "C" int omni_greedy_accept(const void* logits, int64_t logits_stride, int32_t vocab,
                                  int32_t logits_dtype, const int64_t* tokens, int64_t* nxt, int32_t* out,
                                  int64_t out_stride, int64_t out_cap, int64_t* tok, int64_t* last,
                                  uint8_t* done, int64_t* draft_next, const int64_t* start,
                                  const uint8_t* use_draft, int32_t rows, int32_t tokens_per_row,
                                  int64_t limit, int64_t eos, void* stream) {
  int st = accept_common_check(tokens, out, out_stride, out_cap, tok, last, done, draft_next, start,
                               use_draft, rows, tokens_per_row);
  if (st <= 0) return st;
  if (!logits || vocab <= 0 || logits_stride < vocab) return OMNI_ERR_INVALID;
  int esize;
  if (logits_dtype == OMNI_BF16) esize = 2;
  else if (logits_dtype == OMNI_F32) esize = 4;
  else return OMNI_ERR_DTYPE;
  const int ev = 16 / esize;
  if ((uintptr_t)logits % esize) return OMNI_ERR_INVALID;
  const bool aligned = ((uintptr_t)logits & 15u) == 0 && logits_stride % ev == 0;
  const int64_t nchunks = vocab / ev;
  int kpt = (int)((nchunks + kAcceptThreads - 1) / kAcceptThreads);
  if (kpt > 16) return OMNI_ERR_SHAPE;  // vocabularies up to 131072 bf16 / 65536 fp32 entries
  AcceptArgs a = make_accept_args(tokens, out, out_stride, out_cap, tok, last, done, draft_next, start,
                                  use_draft, tokens_per_row, limit, eos);
  a.nxt_out = nxt;
  a.logits = logits;
  a.logits_stride = logits_stride;
  a.vocab = vocab;
  hipStream_t s = (hipStream_t)stream;
  // Argmax by row, then the acceptance (when the argmaxes have somewhere to go and a row fits 16 chunks per
  // thread of a 256-thread workgroup: vocabularies up to 32768 bf16 / 16384 fp32 entries).
  const int64_t rkpt = (nchunks + kRowThreads - 1) / kRowThreads;
  if (nxt && rkpt <= 16 && (int64_t)rows * tokens_per_row <= INT_MAX) {  // the grid has one workgroup per row
    const int rk = rkpt <= 1 ? 1 : rkpt <= 2 ? 2 : rkpt <= 4 ? 4 : rkpt <= 8 ? 8 : 16;
    const int nrows = rows * tokens_per_row;
#define OMNI_ROW_ARGMAX(L, K)                                                       \
  do {                                                                              \
    if (aligned) row_argmax_kernel<L, K, true><<<nrows, kRowThreads, 0, s>>>(a);    \
    else row_argmax_kernel<L, K, false><<<nrows, kRowThreads, 0, s>>>(a);           \
  } while (0)
    if (logits_dtype == OMNI_BF16) {
      switch (rk) {
        case 1: OMNI_ROW_ARGMAX(uint16_t, 1); break;
        case 2: OMNI_ROW_ARGMAX(uint16_t, 2); break;
        case 4: OMNI_ROW_ARGMAX(uint16_t, 4); break;
        case 8: OMNI_ROW_ARGMAX(uint16_t, 8); break;
        default: OMNI_ROW_ARGMAX(uint16_t, 16); break;
      }
    } else {
      switch (rk) {
        case 1: OMNI_ROW_ARGMAX(float, 1); break;
        case 2: OMNI_ROW_ARGMAX(float, 2); break;
        case 4: OMNI_ROW_ARGMAX(float, 4); break;
        case 8: OMNI_ROW_ARGMAX(float, 8); break;
        default: OMNI_ROW_ARGMAX(float, 16); break;
      }
    }
#undef OMNI_ROW_ARGMAX
    st = omni_launch_status();
    if (st != OMNI_OK) return st;
    a.nxt_in = nxt;
    accept_kernel<<<(rows + 63) / 64, 64, 0, s>>>(a, rows);
    return omni_launch_status();
  }
  const int k = kpt <= 1 ? 1 : kpt <= 2 ? 2 : kpt <= 4 ? 4 : kpt <= 8 ? 8 : 16;
  if (logits_dtype == OMNI_BF16) {
    switch (k) {
      case 1: launch_greedy<uint16_t, 1>(a, rows, aligned, s); break;
      case 2: launch_greedy<uint16_t, 2>(a, rows, aligned, s); break;
      case 4: launch_greedy<uint16_t, 4>(a, rows, aligned, s); break;
      case 8: launch_greedy<uint16_t, 8>(a, rows, aligned, s); break;
      default: launch_greedy<uint16_t, 16>(a, rows, aligned, s); break;
    }
  } else {
    switch (k) {
      case 1: launch_greedy<float, 1>(a, rows, aligned, s); break;
      case 2: launch_greedy<float, 2>(a, rows, aligned, s); break;
      case 4: launch_greedy<float, 4>(a, rows, aligned, s); break;
      case 8: launch_greedy<float, 8>(a, rows, aligned, s); break;
      default: launch_greedy<float, 16>(a, rows, aligned, s); break;
    }
  }
  return omni_launch_status();
}
