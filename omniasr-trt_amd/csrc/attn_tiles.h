// The MFMA tile math shared by the attention kernels (verify, beams, prefill) on gfx950.
//
// One 32-key tile of K and V per wave, both products on v_mfma_f32_16x16x32_bf16 with up to 16 queries padded to
// the 16-wide MFMA dimension:
//   S^T = K Q^T  -- A = K (16 keys x 32 dims), B = Q^T.  Lane (c = lane%16, g = lane/16) holds key
//                   kb + 8*(c/4) + 4*mb + c%4 (mb = 0, 1), so the two output blocks leave lane (c, g) the scores
//                   of query c for keys kb + 8g .. kb + 8g + 7;
//   O  = P V     -- A = P (those 8 scores as probabilities, rounded to bf16: exactly lane (c, g)'s A operand),
//                   B = V (32 keys x 16 dims).  Output column c of block (gg, e) is dimension 128*gg + 8c + e, so
//                   lane (c, g) holds 8 consecutive dimensions of 8 keys and builds the B operands with one byte
//                   permute per dword.
// Softmax is online with a lazy reference max (kLazyLog2) in the log2 domain.
#pragma once

#include <math.h>

#include "common.h"

namespace omni {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Scores are kept relative to a reference max m_ref (log2 domain) that only moves when a score exceeds it by
// more than 2^kLazyLog2: the cross-lane max and the rescale of O are skipped for almost every tile, and
// probabilities stay <= 2^kLazyLog2 (exact in fp32, and bf16 keeps its relative precision at any scale).
constexpr float kLazyLog2 = 8.0f;

// One 32-key tile of K and V in MFMA operand layout (see the file comment).
template <int D>
struct KVTile {
  static constexpr int KS = D / 32, NG = D / 128;
  u32x4_t k[2][KS];
  u32x4_t v[NG][8];
};

__device__ __forceinline__ u32x4_t ld16(const char* p) { return *reinterpret_cast<const u32x4_t*>(p); }

// One 32-key tile of K and V into MFMA operand layout.  Key rows are kRow bytes apart (contiguous rows of D elements
// by default; a 128-dimension slice of a wider head otherwise), so each load is the wave-uniform tile base plus a
// 32-bit lane offset.  K rows past ``kmax`` (the last cache position, relative to
// the tile's first key; 31 inside the cache) are read at kmax; their scores are masked.  V rows at or past
// ``vstop`` (the end of the keys in use, relative; 32 for a full tile, >= 1 for a tile that is attended) are read
// at vstop - 1, a key in use: every query's probability of those keys is 0, and 0 times a finite value of a key in
// use adds nothing (stale memory past the keys could hold NaN).  Only addresses are clamped, never loaded data, so
// nothing waits for a tile's loads before its math.
template <int D, uint32_t kRow = D * 2>
__device__ __forceinline__ void load_tile_clamped(KVTile<D>& t, const char* kt, const char* vt, int kmax, int vstop,
                                                  int c, int g) {
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    int rk = 8 * (c >> 2) + 4 * mb + (c & 3);
    rk = rk < kmax ? rk : kmax;
    const uint32_t ko = (uint32_t)rk * kRow + g * 16;
#pragma unroll
    for (int s = 0; s < KVTile<D>::KS; ++s) t.k[mb][s] = ld16(kt + ko + s * 64);
  }
  int vmax = vstop - 1 < kmax ? vstop - 1 : kmax;
  vmax = vmax > 0 ? vmax : 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int rv = 8 * g + j;
    const uint32_t vo = (uint32_t)(rv < vmax ? rv : vmax) * kRow + c * 16;
#pragma unroll
    for (int gg = 0; gg < KVTile<D>::NG; ++gg) t.v[gg][j] = ld16(vt + vo + gg * 256);
  }
}

// A tile of 32 gathered key rows into MFMA operand layout: ``rows`` (in LDS) holds the byte offset of each of the
// tile's 32 keys from ``kt`` / ``vt`` (the same offset in K and V); every offset is a key in use.
template <int D>
__device__ __forceinline__ void load_tile_rows(KVTile<D>& t, const char* kt, const char* vt, const uint32_t* rows, int c,
                                               int g) {
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const uint32_t ko = rows[8 * (c >> 2) + 4 * mb + (c & 3)] + g * 16;
#pragma unroll
    for (int s = 0; s < KVTile<D>::KS; ++s) t.k[mb][s] = ld16(kt + ko + s * 64);
  }
  const u32x4_t r0 = *reinterpret_cast<const u32x4_t*>(rows + 8 * g);
  const u32x4_t r1 = *reinterpret_cast<const u32x4_t*>(rows + 8 * g + 4);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t vo = (j < 4 ? r0[j] : r1[j - 4]) + c * 16;
#pragma unroll
    for (int gg = 0; gg < KVTile<D>::NG; ++gg) t.v[gg][j] = ld16(vt + vo + gg * 256);
  }
}

// S^T for the tile: lane (c, g) gets query c's raw scores for keys kb + 8g + j, j = 0..7.
template <int D>
__device__ __forceinline__ void tile_scores(const KVTile<D>& t, const u32x4_t (&qop)[D / 32], float (&sv)[8]) {
  f32x4_t sacc[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    sacc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
      sacc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, t.k[mb][s]),
                                                         __builtin_bit_cast(bf16x8_t, qop[s]), sacc[mb], 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) sv[j] = sacc[j >> 2][j & 3];
}

// Move the reference max of every row to ``m_new`` (rows 4g + i of O live in this lane; their alphas in lanes
// 4g + i), rescaling O and this lane's share of the probability sum.
template <int NB>
__device__ __forceinline__ void rescale(float m_old, float m_new_use, float& l_run, f32x4_t (&o)[NB], int g) {
  const float alpha = __builtin_amdgcn_exp2f(m_old - m_new_use);  // m_old = -inf: 0
  l_run *= alpha;
  float al[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i, kWave);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[nb][i] *= al[i];
  }
}

// O += P V for the tile: P from this lane's 8 probabilities (its A operand), V transposed in registers.
template <int D>
__device__ __forceinline__ void tile_pv(const KVTile<D>& t, const float (&p)[8], f32x4_t (&o)[D / 16]) {
  u32x4_t pop;
#pragma unroll
  for (int w = 0; w < 4; ++w)
    pop[w] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{p[2 * w], p[2 * w + 1]}), bf16x2_t));
#pragma unroll
  for (int gg = 0; gg < D / 128; ++gg) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      u32x4_t bop;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo = t.v[gg][2 * w][e >> 1];
        const uint32_t hi = t.v[gg][2 * w + 1][e >> 1];
        // element e of rows 2w and 2w+1: one byte permute
        bop[w] = __builtin_amdgcn_perm(hi, lo, (e & 1) ? 0x07060302u : 0x05040100u);
      }
      o[gg * 8 + e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, pop),
                                                              __builtin_bit_cast(bf16x8_t, bop), o[gg * 8 + e], 0,
                                                              0, 0);
    }
  }
}

struct SoftmaxState {
  float m_ref;  // reference max of query c (log2 domain), equal over g
  float thr;    // raw-score threshold above which m_ref must move
  float l_run;  // this lane's share of query c's probability sum (relative to m_ref)
};

// A tile with its raw scores ``sv`` (lane (c, g): query c, keys key0 + j): the causal / end-of-row mask (key0 + j >=
// lim: query c does not see key j of this lane), the lazy reference max, probabilities, O += P V.  The mask is a no-op
// on tiles every query sees whole.  kBits: ``lim`` holds this lane's mask instead, bit j set when query c sees key
// key0 + j (key0 unused).
template <int D, bool kBits = false>
__device__ __forceinline__ void attend_scored(const KVTile<D>& t, float (&sv)[8], float c_scale, SoftmaxState& st,
                                              f32x4_t (&o)[D / 16], int g, int key0, int lim) {
  bool over = false;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool seen = kBits ? ((lim >> j) & 1) != 0 : key0 + j < lim;
    sv[j] = seen ? sv[j] : -INFINITY;
    over |= sv[j] > st.thr;
  }
  if (__any(over)) {
    float mx = sv[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mx = fmaxf(mx, sv[j]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(st.m_ref, mx * c_scale);
    rescale<D / 16>(st.m_ref, m_new == -INFINITY ? 0.f : m_new, st.l_run, o, g);
    st.m_ref = m_new;
    st.thr = m_new == -INFINITY ? -INFINITY : (m_new + kLazyLog2) / c_scale;
  }
  const float m_use = st.m_ref == -INFINITY ? 0.f : st.m_ref;  // no key seen yet: every probability is 0
  float p[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[j], c_scale, -m_use));
    st.l_run += p[j];
  }
  tile_pv<D>(t, p, o);
}

// One tile: scores, then attend_scored.
template <int D>
__device__ __forceinline__ void attend(const KVTile<D>& t, const u32x4_t (&qop)[D / 32], float c_scale,
                                       SoftmaxState& st, f32x4_t (&o)[D / 16], int g, int key0, int lim) {
  float sv[8];
  tile_scores<D>(t, qop, sv);
  attend_scored<D>(t, sv, c_scale, st, o, g, key0, lim);
}

// One tile whose keys each query sees by a mask: bit j of ``bits`` says whether query c sees key 8g + j.
template <int D>
__device__ __forceinline__ void attend_bits(const KVTile<D>& t, const u32x4_t (&qop)[D / 32], float c_scale,
                                            SoftmaxState& st, f32x4_t (&o)[D / 16], int g, int bits) {
  float sv[8];
  tile_scores<D>(t, qop, sv);
  attend_scored<D, true>(t, sv, c_scale, st, o, g, 0, bits);
}

// A workgroup barrier ordering LDS accesses only: global loads in flight stay in flight across it (a full
// __syncthreads waits for every outstanding memory access of the wave).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace omni
