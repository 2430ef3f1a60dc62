// Multi-query split-K flash-decode verification attention for gfx950.
//
// Semantics of ``kernels.draft_attention`` (``_beam_ctx`` CAUSAL=True + ``_beam_combine``,
// src/omniasr_trt/kernels.py:338-358, 56-113, 146-161) and, with one query per row, of
// ``kernels.decode_attention`` (src/omniasr_trt/kernels.py:406-423, 163-211): query i of row b
// attends to keys [0, lengths[b] + i); softmax in fp32; split partials (acc, m, l) are merged by
// log-sum-exp with w_s = exp(m_s - max m) (0 for an empty split) and out = sum w_s acc_s /
// sum w_s l_s (0 when that sum is 0).
//
// Work decomposition: one wavefront per (key split, head, row) -- grid (splits, heads, rows), 64
// threads.  A wave streams its split's keys 32 at a time and serves all of the row's T <= 16
// queries with that single read of K and V.  Splits beyond a row's last key exit at once, so the
// grid depends on the key bucket only (graph capture) while ragged rows read just their own keys.
// The last split of a (row, head) to finish merges the partials (an atomic ticket per (row, head),
// reset by the merging wave); a row with one split writes its output directly.
//
// bf16, head_dim a multiple of 128: both products run on v_mfma_f32_16x16x32_bf16 with the T
// queries padded to the 16-wide MFMA dimension, and every K/V element is loaded straight into the
// MFMA operand layout with 128-bit loads (no LDS):
//   S^T = K Q^T  -- A = K (16 keys x 32 dims), B = Q^T.  Lane (c = lane%16, g = lane/16) loads
//                   key kb + 8*(c/4) + 4*mb + c%4 (mb = 0, 1) so that the output of the two MFMAs
//                   leaves lane (c, g) the scores of query c for keys kb + 8g .. kb + 8g + 7;
//   O  = P V     -- A = P (those 8 scores, rounded to bf16, are exactly lane (c, g)'s A operand),
//                   B = V (32 keys x 16 dims).  Output column c of block (gg, e) is dimension
//                   128*gg + 8c + e, so lane (c, g) loads 8 consecutive dimensions of 8 keys
//                   (8 x 16 bytes) and transposes them in registers into the 8 B operands.
// fp32, or bf16 with another head_dim: a vector-ALU wave with fp32 products (the reference's
// IEEE path for fp32 agreement checks).
#include <math.h>

#include "common.h"

namespace omni {

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  int64_t s_row, s_head, s_pos, cache_len;
  const int64_t* lengths;
  int T, H, D;
  int chunk, splits;
  float scale_log2;  // softmax scale * log2(e): scores are kept in the log2 domain
  float* part_o;     // [rows, H, splits, T, D]
  float* part_ml;    // [rows, H, splits, T, 2]: (m, l)
  int* counters;     // [rows * H]
  void* out;         // [rows * T, H, D]
  int separate;      // partials only: a second launch merges them
};

struct SplitRange {
  int64_t n;      // keys every query of the row sees (lengths[b], clamped to the cache)
  int64_t stop;   // end of this split's keys
  int64_t start;  // first key of this split
  int nact;       // splits holding keys of this row (>= 1: an empty row still writes zeros)
};

__device__ __forceinline__ SplitRange split_range(const AttnArgs& a, int b, int sp) {
  SplitRange r;
  r.n = clamp64(a.lengths[b], 0, a.cache_len);
  int64_t total = r.n + a.T - 1;  // keys the last query sees
  total = total < a.cache_len ? total : a.cache_len;
  const int64_t covered = (int64_t)a.splits * a.chunk;
  total = total < covered ? total : covered;
  int64_t nact = ceil_div64(total, a.chunk);
  r.nact = (int)(nact < 1 ? 1 : nact);
  r.start = (int64_t)sp * a.chunk;
  const int64_t e = r.start + a.chunk;
  r.stop = e < total ? e : total;
  return r;
}

template <typename OutT>
__device__ __forceinline__ void store4(OutT* p, f32x4_t v);

template <>
__device__ __forceinline__ void store4<float>(float* p, f32x4_t v) {
  *reinterpret_cast<f32x4_t*>(p) = v;
}

template <>
__device__ __forceinline__ void store4<uint16_t>(uint16_t* p, f32x4_t v) {
  uint2 w;
  w.x = pack_bf16x2(v[0], v[1]);
  w.y = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<uint2*>(p) = w;
}

// Log-sum-exp merge of the ``nact`` partials of (row b, head h) by one wave; writes the output.
template <typename OutT>
__device__ void merge_splits(const AttnArgs& a, int b, int h, int nact) {
  const int lane = lane_id();
  const int64_t split0 = ((int64_t)b * a.H + h) * a.splits;
  OutT* out = reinterpret_cast<OutT*>(a.out);
  for (int t = 0; t < a.T; ++t) {
    float top = -INFINITY;
    for (int s = lane; s < nact; s += kWave) top = fmaxf(top, a.part_ml[((split0 + s) * a.T + t) * 2]);
    top = wave_max(top);
    float den = 0.f;
    for (int s = lane; s < nact; s += kWave) {
      const float m = a.part_ml[((split0 + s) * a.T + t) * 2];
      const float w = m == -INFINITY ? 0.f : exp2f(m - top);
      den += w * a.part_ml[((split0 + s) * a.T + t) * 2 + 1];
    }
    den = wave_sum(den);
    const float div = den > 0.f ? den : 1.f;
    OutT* orow = out + ((int64_t)(b * a.T + t) * a.H + h) * a.D;
    for (int d = lane * 4; d < a.D; d += kWave * 4) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      for (int s = 0; s < nact; ++s) {
        const float m = a.part_ml[((split0 + s) * a.T + t) * 2];
        const float w = m == -INFINITY ? 0.f : exp2f(m - top);
        const f32x4_t po = *reinterpret_cast<const f32x4_t*>(a.part_o + ((split0 + s) * a.T + t) * a.D + d);
        acc += w * po;
      }
      store4<OutT>(orow + d, acc / div);
    }
  }
}

// After a split wrote its partial: the last of the row's ``nact`` splits merges them all.
template <typename OutT>
__device__ __forceinline__ void finish_split(const AttnArgs& a, int b, int h, int nact) {
  if (a.separate) return;
  // Release at agent scope: this wave's partial leaves its XCD's L2 before the ticket is taken
  // (the L2s of the 8 XCDs are not coherent with each other).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  int ticket = 0;
  if (lane_id() == 0) ticket = atomicAdd(&a.counters[b * a.H + h], 1);
  ticket = __shfl(ticket, 0, kWave);
  if (ticket != nact - 1) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // the other splits' partials, not stale lines
  merge_splits<OutT>(a, b, h, nact);
  if (lane_id() == 0) a.counters[b * a.H + h] = 0;  // every split of this (row, head) has arrived
}

// ---------------------------------------------------------------------------------------------- MFMA

template <int D>
__global__ __launch_bounds__(64) void verify_attn_mfma_kernel(AttnArgs a) {
  constexpr int KS = D / 32;  // k-steps of S^T = K Q^T
  constexpr int NG = D / 128;  // 128-wide output groups
  const int sp = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const SplitRange r = split_range(a, b, sp);
  if (sp >= r.nact) return;
  const int lane = threadIdx.x, c = lane & 15, g = lane >> 4;
  const int T = a.T;

  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(a.k) + b * a.s_row + h * a.s_head;
  const uint16_t* vbase = reinterpret_cast<const uint16_t*>(a.v) + b * a.s_row + h * a.s_head;
  const int64_t last_key = a.cache_len - 1;

  // B operand of S^T = K Q^T: lane (c, g) holds q[c][32s + 8g .. 32s + 8g + 7].
  u32x4_t qop[KS];
  {
    const u32x4_t zero = {0u, 0u, 0u, 0u};
    const uint16_t* qrow =
        reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)(b * T + c) * a.H + h) * D + g * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) qop[s] = c < T ? *reinterpret_cast<const u32x4_t*>(qrow + s * 32) : zero;
  }

  float m_run = -INFINITY;  // running max of query c (log2 domain), equal over g
  float l_run = 0.f;        // this lane's share of query c's sum of probabilities
  f32x4_t o[NG * 8];        // o[8gg + e][i]: output row 4g + i, dimension 128gg + 8c + e
#pragma unroll
  for (int nb = 0; nb < NG * 8; ++nb) o[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int64_t see_all = r.stop < r.n ? r.stop : r.n;  // keys below this are seen by every query
  const int64_t lim_c = (r.n + c) < r.stop ? (r.n + c) : r.stop;  // query c's key limit here

  for (int64_t kb = r.start; kb < r.stop; kb += 32) {
    // ---- S^T for 32 keys: two 16-key MFMA blocks
    f32x4_t sacc[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      int64_t key = kb + 8 * (c >> 2) + 4 * mb + (c & 3);
      key = key < last_key ? key : last_key;
      const uint16_t* kp = kbase + key * a.s_pos + g * 8;
      u32x4_t kr[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) kr[s] = *reinterpret_cast<const u32x4_t*>(kp + s * 32);
      sacc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sacc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[s]),
                                                           __builtin_bit_cast(bf16x8_t, qop[s]),
                                                           sacc[mb], 0, 0, 0);
    }
    // ---- V rows kb + 8g + j, dimensions 128gg + 8c .. +7
    u32x4_t vr[NG][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int64_t key = kb + 8 * g + j;
      key = key < last_key ? key : last_key;
      const uint16_t* vp = vbase + key * a.s_pos + c * 8;
#pragma unroll
      for (int gg = 0; gg < NG; ++gg) vr[gg][j] = *reinterpret_cast<const u32x4_t*>(vp + gg * 128);
    }

    float sv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) sv[j] = sacc[j >> 2][j & 3] * a.scale_log2;
    if (kb + 32 > see_all) {  // the tile reaches past some query's keys or the split's end
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t key = kb + 8 * g + j;
        if (key >= lim_c) sv[j] = -INFINITY;
        if (key >= r.stop) {  // not a key of this row: zero V so that 0 * garbage stays 0
#pragma unroll
          for (int gg = 0; gg < NG; ++gg) vr[gg][j] = u32x4_t{0u, 0u, 0u, 0u};
        }
      }
    }
    float mx = sv[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mx = fmaxf(mx, sv[j]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float p[8];
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = exp2f(sv[j] - m_use);
      psum += p[j];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    u32x4_t pop;
#pragma unroll
    for (int w = 0; w < 4; ++w) pop[w] = pack_bf16x2(p[2 * w], p[2 * w + 1]);

    // rescale the output rows this lane holds (rows 4g + i live in lanes c = 4g + i)
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i, kWave);
#pragma unroll
    for (int nb = 0; nb < NG * 8; ++nb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[nb][i] *= al[i];
    }

    // ---- O += P V: B operand (gg, e) = element e of vr[gg][0..7]
#pragma unroll
    for (int gg = 0; gg < NG; ++gg) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x4_t bop;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t lo = vr[gg][2 * w][e >> 1];
          const uint32_t hi = vr[gg][2 * w + 1][e >> 1];
          bop[w] = (e & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
        o[gg * 8 + e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, pop),
                                                                __builtin_bit_cast(bf16x8_t, bop),
                                                                o[gg * 8 + e], 0, 0, 0);
      }
    }
  }

  // ---- finish: per-query sums, then either the output or this split's partial
  float l_tot = l_run + __shfl_xor(l_run, 16, kWave);
  l_tot += __shfl_xor(l_tot, 32, kWave);
  float li[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) li[i] = __shfl(l_tot, 4 * g + i, kWave);
  if (r.nact == 1 && !a.separate) {
    uint16_t* out = reinterpret_cast<uint16_t*>(a.out);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * g + i;
      if (t >= T) continue;
      const float div = li[i] > 0.f ? li[i] : 1.f;
#pragma unroll
      for (int gg = 0; gg < NG; ++gg) {
        u32x4_t w;
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = pack_bf16x2(o[gg * 8 + 2 * q][i] / div, o[gg * 8 + 2 * q + 1][i] / div);
        *reinterpret_cast<u32x4_t*>(out + ((int64_t)(b * T + t) * a.H + h) * D + gg * 128 + c * 8) = w;
      }
    }
    return;
  }
  const int64_t base = (((int64_t)b * a.H + h) * a.splits + sp) * T;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * g + i;
    if (t >= T) continue;
#pragma unroll
    for (int gg = 0; gg < NG; ++gg) {
      f32x4_t* po = reinterpret_cast<f32x4_t*>(a.part_o + (base + t) * D + gg * 128 + c * 8);
      po[0] = f32x4_t{o[gg * 8 + 0][i], o[gg * 8 + 1][i], o[gg * 8 + 2][i], o[gg * 8 + 3][i]};
      po[1] = f32x4_t{o[gg * 8 + 4][i], o[gg * 8 + 5][i], o[gg * 8 + 6][i], o[gg * 8 + 7][i]};
    }
  }
  if (g == 0 && c < T) {
    a.part_ml[(base + c) * 2] = m_run;
    a.part_ml[(base + c) * 2 + 1] = l_tot;
  }
  finish_split<uint16_t>(a, b, h, r.nact);
}

// ---------------------------------------------------------------------------------------------- VALU

constexpr int kValuMaxT = 16;
constexpr int kValuMaxD = 512;
constexpr int kValuDPL = kValuMaxD / kWave;  // output dimensions per lane

template <typename Elem>
__device__ __forceinline__ float load_elem(const Elem* p);
template <>
__device__ __forceinline__ float load_elem<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_elem<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

template <typename Elem>
__global__ __launch_bounds__(64) void verify_attn_valu_kernel(AttnArgs a) {
  __shared__ float qs[kValuMaxT * kValuMaxD];  // queries, pre-scaled
  __shared__ float ps[kValuMaxT * kWave];      // probabilities of the current 64 keys
  const int sp = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const SplitRange r = split_range(a, b, sp);
  if (sp >= r.nact) return;
  const int lane = threadIdx.x;
  const int T = a.T, D = a.D;
  const Elem* kbase = reinterpret_cast<const Elem*>(a.k) + b * a.s_row + h * a.s_head;
  const Elem* vbase = reinterpret_cast<const Elem*>(a.v) + b * a.s_row + h * a.s_head;
  const Elem* qb = reinterpret_cast<const Elem*>(a.q);
  for (int idx = lane; idx < T * D; idx += kWave) {
    const int t = idx / D, d = idx - t * D;
    qs[t * D + d] = load_elem<Elem>(qb + ((int64_t)(b * T + t) * a.H + h) * D + d) * a.scale_log2;
  }
  __syncthreads();

  float m_run[kValuMaxT], l_run[kValuMaxT], acc[kValuMaxT][kValuDPL];
#pragma unroll
  for (int t = 0; t < kValuMaxT; ++t) {
    m_run[t] = -INFINITY;
    l_run[t] = 0.f;
#pragma unroll
    for (int dd = 0; dd < kValuDPL; ++dd) acc[t][dd] = 0.f;
  }
  const int64_t last_key = a.cache_len - 1;
  for (int64_t kb = r.start; kb < r.stop; kb += kWave) {
    const int64_t key = kb + lane;
    const int64_t kl = key < last_key ? key : last_key;
    const Elem* krow = kbase + kl * a.s_pos;
    float s[kValuMaxT];
#pragma unroll
    for (int t = 0; t < kValuMaxT; ++t) s[t] = 0.f;
    for (int d = 0; d < D; ++d) {
      const float kd = load_elem<Elem>(krow + d);
#pragma unroll
      for (int t = 0; t < kValuMaxT; ++t)
        if (t < T) s[t] = fmaf(qs[t * D + d], kd, s[t]);
    }
#pragma unroll
    for (int t = 0; t < kValuMaxT; ++t) {
      if (t >= T) continue;  // T is uniform: the whole wave skips together
      const int64_t lim = (r.n + t) < r.stop ? (r.n + t) : r.stop;
      const float sc = key < lim ? s[t] : -INFINITY;
      const float m_new = fmaxf(m_run[t], wave_max(sc));
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m_run[t] - m_use);
      const float pr = exp2f(sc - m_use);
      l_run[t] = l_run[t] * alpha + pr;
      m_run[t] = m_new;
      ps[t * kWave + lane] = pr;
#pragma unroll
      for (int dd = 0; dd < kValuDPL; ++dd) acc[t][dd] *= alpha;
    }
    __syncthreads();
    const int64_t kend = (r.stop - kb) < kWave ? (r.stop - kb) : kWave;
    for (int kk = 0; kk < kend; ++kk) {
      const Elem* vrow = vbase + (kb + kk) * a.s_pos;
#pragma unroll
      for (int dd = 0; dd < kValuDPL; ++dd) {
        const int d = dd * kWave + lane;
        if (d < D) {
          const float vd = load_elem<Elem>(vrow + d);
#pragma unroll
          for (int t = 0; t < kValuMaxT; ++t)
            if (t < T) acc[t][dd] = fmaf(ps[t * kWave + kk], vd, acc[t][dd]);
        }
      }
    }
    __syncthreads();
  }

  const bool direct = r.nact == 1 && !a.separate;
  const int64_t base = (((int64_t)b * a.H + h) * a.splits + sp) * T;
  Elem* out = reinterpret_cast<Elem*>(a.out);
#pragma unroll
  for (int t = 0; t < kValuMaxT; ++t) {
    if (t >= T) continue;
    const float l_tot = wave_sum(l_run[t]);
    const float div = l_tot > 0.f ? l_tot : 1.f;
#pragma unroll
    for (int dd = 0; dd < kValuDPL; ++dd) {
      const int d = dd * kWave + lane;
      if (d >= D) continue;
      if (direct) {
        const float v = acc[t][dd] / div;
        if constexpr (sizeof(Elem) == 2)
          out[((int64_t)(b * T + t) * a.H + h) * D + d] = (uint16_t)f32_to_bf16_rne(v);
        else
          out[((int64_t)(b * T + t) * a.H + h) * D + d] = v;
      } else {
        a.part_o[(base + t) * D + d] = acc[t][dd];
      }
    }
    if (!direct && lane == 0) {
      a.part_ml[(base + t) * 2] = m_run[t];
      a.part_ml[(base + t) * 2 + 1] = l_tot;
    }
  }
  if (direct) return;
  finish_split<Elem>(a, b, h, r.nact);
}

// ---------------------------------------------------------------------------------------------- combine

template <typename OutT>
__global__ __launch_bounds__(64) void verify_attn_combine_kernel(AttnArgs a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const SplitRange r = split_range(a, b, 0);
  merge_splits<OutT>(a, b, h, r.nact);
}

}  // namespace omni

using namespace omni;

static int attn_splits(int32_t keys, int32_t chunk) { return (int)((keys + chunk - 1) / chunk); }

extern "C" int32_t omni_verify_attention_chunk(int32_t rows, int32_t tokens, int32_t heads,
                                               int32_t head_dim, int32_t keys) {
  (void)tokens;
  (void)head_dim;
  if (rows <= 0 || heads <= 0 || keys <= 0) return 64;
  // About 2048 waves over the chip's 256 CUs (8 per CU) when the rows are full, at least 64 keys
  // per split so that a wave's fixed cost (its queries, its partial) stays small.
  const int64_t items = (int64_t)rows * heads;
  int64_t want = (2048 + items - 1) / items;
  int64_t chunk = (keys + want - 1) / want;
  chunk = (chunk + 63) / 64 * 64;
  if (chunk < 64) chunk = 64;
  const int64_t whole = ((int64_t)keys + 31) / 32 * 32;
  if (chunk > whole) chunk = whole;
  return (int32_t)chunk;
}

static size_t align256(size_t n) { return (n + 255) / 256 * 256; }

extern "C" size_t omni_verify_attention_workspace(int32_t rows, int32_t tokens, int32_t heads,
                                                  int32_t head_dim, int32_t keys, int32_t chunk) {
  if (rows <= 0 || tokens <= 0 || heads <= 0 || head_dim <= 0 || keys <= 0) return 0;
  if (chunk <= 0) chunk = omni_verify_attention_chunk(rows, tokens, heads, head_dim, keys);
  const size_t splits = (size_t)attn_splits(keys, chunk);
  const size_t units = (size_t)rows * heads * splits * tokens;
  return align256(units * head_dim * sizeof(float)) + align256(units * 2 * sizeof(float));
}

extern "C" int omni_verify_attention(const void* q, const void* k_cache, const void* v_cache,
                                     int64_t stride_row, int64_t stride_head, int64_t stride_pos,
                                     int64_t cache_len, const int64_t* lengths, int32_t rows,
                                     int32_t tokens, int32_t heads, int32_t head_dim, int32_t keys,
                                     int32_t chunk, float scale, void* out, void* workspace,
                                     size_t workspace_bytes, int32_t* counters, int32_t flags,
                                     int32_t dtype, void* stream) {
  if (rows < 0 || heads <= 0 || head_dim <= 0 || keys <= 0 || cache_len <= 0) return OMNI_ERR_INVALID;
  if (rows == 0) return OMNI_OK;
  if (!q || !k_cache || !v_cache || !lengths || !out || !workspace || !counters) return OMNI_ERR_INVALID;
  if (tokens < 1 || tokens > 16) return OMNI_ERR_SHAPE;
  if (dtype != OMNI_BF16 && dtype != OMNI_F32) return OMNI_ERR_DTYPE;
  if (head_dim % 8 != 0 || head_dim > kValuMaxD) return OMNI_ERR_SHAPE;
  if (chunk == 0) chunk = omni_verify_attention_chunk(rows, tokens, heads, head_dim, keys);
  if (chunk <= 0 || chunk % 64 != 0) return OMNI_ERR_INVALID;
  if (workspace_bytes < omni_verify_attention_workspace(rows, tokens, heads, head_dim, keys, chunk))
    return OMNI_ERR_WORKSPACE;
  if (((uintptr_t)workspace & 255u) != 0) return OMNI_ERR_WORKSPACE;
  const bool mfma = dtype == OMNI_BF16 && head_dim % 128 == 0;
  // Vector accesses: q, out (and, on MFMA, every row / head / position start) 16-byte aligned.
  if (((uintptr_t)q | (uintptr_t)out) & 15u) return OMNI_ERR_INVALID;
  if (mfma) {
    if (((uintptr_t)k_cache | (uintptr_t)v_cache) & 15u) return OMNI_ERR_INVALID;
    if ((stride_row | stride_head | stride_pos) % 8 != 0) return OMNI_ERR_INVALID;
  }
  const int splits = attn_splits(keys, chunk);
  const size_t units = (size_t)rows * heads * splits * tokens;
  AttnArgs a;
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.s_row = stride_row;
  a.s_head = stride_head;
  a.s_pos = stride_pos;
  a.cache_len = cache_len;
  a.lengths = lengths;
  a.T = tokens;
  a.H = heads;
  a.D = head_dim;
  a.chunk = chunk;
  a.splits = splits;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.part_o = (float*)workspace;
  a.part_ml = (float*)((char*)workspace + align256(units * head_dim * sizeof(float)));
  a.counters = counters;
  a.out = out;
  a.separate = (flags & OMNI_ATTN_SEPARATE_COMBINE) ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid(splits, heads, rows);
  if (mfma) {
    switch (head_dim) {
      case 128: verify_attn_mfma_kernel<128><<<grid, 64, 0, s>>>(a); break;
      case 256: verify_attn_mfma_kernel<256><<<grid, 64, 0, s>>>(a); break;
      case 512: verify_attn_mfma_kernel<512><<<grid, 64, 0, s>>>(a); break;
      default: verify_attn_valu_kernel<uint16_t><<<grid, 64, 0, s>>>(a); break;
    }
  } else if (dtype == OMNI_BF16) {
    verify_attn_valu_kernel<uint16_t><<<grid, 64, 0, s>>>(a);
  } else {
    verify_attn_valu_kernel<float><<<grid, 64, 0, s>>>(a);
  }
  int st = omni_launch_status();
  if (st != OMNI_OK || !a.separate) return st;
  dim3 cgrid(heads, rows);
  if (dtype == OMNI_BF16) verify_attn_combine_kernel<uint16_t><<<cgrid, 64, 0, s>>>(a);
  else verify_attn_combine_kernel<float><<<cgrid, 64, 0, s>>>(a);
  return omni_launch_status();
}
