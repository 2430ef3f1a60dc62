// Causal attention over whole contexts for gfx950: the prefill's
//     F.scaled_dot_product_attention(q, k, v, is_causal=True)
// (src/omniasr_trt/decode.py:163-164) over the cache rows ``kernels.rope_kv`` has just written.  Query p of context
// b attends to keys [0, p] of its cache row; fp32 accumulation, bf16 in and out, head_dim 128, 256 or 512.
#include <math.h>

#include "attn_tiles.h"
#include "common.h"

namespace omni {

// Causal attention over whole contexts (the prefill): query p of context b attends to keys [0, p] of its cache row.
// One workgroup of kPfWaves waves per (query block, head, context), the longest blocks first.  The block's 32-key
// tiles go through LDS once for all of its waves (double-buffered: tile t + 1's global loads are in flight during
// tile t's math).  Each wave holds kPfSub groups of 16 queries: per tile it reads the K fragments and, by LDS
// transpose reads, the V operands once, then runs S^T = K Q^T, the lazy softmax (causal limit as the key limit,
// skipped on tiles the whole group sees) and O += P V for every group that sees the tile.
constexpr int kPfWaves = 4;
constexpr int kPfSub = 3;  // 16-query groups per wave (3: 255 VGPRs, two waves per SIMD; measured fastest of 1-4)
constexpr int kPfQueries = 16 * kPfSub * kPfWaves;
constexpr int kPfRow = 128 * 2 + 16;  // LDS bytes per key row: 256 B of data, padded against bank conflicts
constexpr int kPfStage = 32;          // keys per LDS stage (one barrier each), a multiple of the 32-key MFMA tile
constexpr int kPfThreads = 64 * kPfWaves;
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16;
typedef __attribute__((address_space(3))) const char lds_char;
constexpr int kPfChunks = kPfStage * 16 / kPfThreads;  // 16-byte chunks of K (and of V) per thread per stage
static_assert(kPfChunks * kPfThreads == kPfStage * 16, "a stage is whole chunks per thread");

struct PrefillArgs {
  const uint16_t* q;    // [B * width, H, D] bf16
  const uint16_t* k;    // cache rows: element strides s_row / s_head, key rows contiguous (D elements)
  const uint16_t* v;
  const int64_t* slots;  // [B] cache row of each context
  int64_t s_row, s_head, cache_rows;
  int width, H;
  float scale_log2;
  uint16_t* out;  // [B * width, H, D] bf16
};

// Workgroup -> (query block j counted from the longest, head h, context b).  The dispatcher hands consecutive
// workgroups to the 8 XCDs in turn; when heads x contexts is a multiple of 8, XCD x gets units (head, context)
// x, x + 8, ... one after another, all query blocks of a unit together (longest first), so each unit's K / V rows
// are brought into one XCD's L2 rather than into all eight.  Only speed depends on the dispatch order.
constexpr bool kPfXcd = true;
struct PfBlock {
  int j, h, b;
};
__device__ __forceinline__ PfBlock pf_block(int nqb, int H, int B) {
  if (!kPfXcd || (H * B) % 8 != 0) return PfBlock{(int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z};
  const int L = (int)blockIdx.x + nqb * ((int)blockIdx.y + H * (int)blockIdx.z);
  const int x = L % 8, k = L / 8;
  const int unit = (k / nqb) * 8 + x;
  return PfBlock{k % nqb, unit % H, unit / H};
}

// The softmax step of one 16-query group for one tile: mask (key0 + j >= lim), lazy reference max, this lane's
// 8 probabilities packed as the P operand.  (The same arithmetic as attend().)
template <int NB>
__device__ __forceinline__ u32x4_t softmax_tile(float (&sv)[8], float c_scale, SoftmaxState& st, f32x4_t (&o)[NB],
                                                int g, int key0, int lim, bool whole) {
  bool over = false;
  if (!whole) {  // whole (wave-uniform): every query of the group sees every key of the tile
#pragma unroll
    for (int j = 0; j < 8; ++j) sv[j] = key0 + j < lim ? sv[j] : -INFINITY;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) over |= sv[j] > st.thr;
  if (__any(over)) {
    float mx = sv[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mx = fmaxf(mx, sv[j]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(st.m_ref, mx * c_scale);
    rescale<NB>(st.m_ref, m_new == -INFINITY ? 0.f : m_new, st.l_run, o, g);
    st.m_ref = m_new;
    st.thr = m_new == -INFINITY ? -INFINITY : (m_new + kLazyLog2) / c_scale;
  }
  const float m_use = st.m_ref == -INFINITY ? 0.f : st.m_ref;
  float p[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[j], c_scale, -m_use));
    st.l_run += p[j];
  }
  u32x4_t pop;
#pragma unroll
  for (int w = 0; w < 4; ++w)
    pop[w] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{p[2 * w], p[2 * w + 1]}), bf16x2_t));
  return pop;
}

__global__ __launch_bounds__(64 * kPfWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_attn_kernel(
    PrefillArgs a) {
  constexpr int D = 128, KS = D / 32;
  __shared__ __attribute__((aligned(16))) char lds[2][2][kPfStage * kPfRow];  // [buffer][K, V][key rows]
  const int nqb = (a.width + kPfQueries - 1) / kPfQueries;
  const PfBlock blk = pf_block(nqb, a.H, (int)gridDim.z);
  const int qb = (nqb - 1 - blk.j) * kPfQueries;  // the longest blocks first
  const int h = blk.h, b = blk.b;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t slot = clamp64(a.slots[b], 0, a.cache_rows - 1);
  const uint16_t* kbase = a.k + slot * a.s_row + h * a.s_head;
  const uint16_t* vbase = a.v + slot * a.s_row + h * a.s_head;
  const int kend = min(qb + kPfQueries, a.width);  // keys the block's last query sees
  const int nt = (kend + kPfStage - 1) / kPfStage;

  // Global -> LDS: thread tid moves 16-byte chunks tid, tid + kPfThreads, ... of the stage's K and of its V (kPfStage rows x
  // 256 B each).  Rows past the context read its last key (finite: masked by the causal limit, never NaN).
  u32x4_t stage[2 * kPfChunks];
  auto fetch = [&](int t) {
#pragma unroll
    for (int e = 0; e < kPfChunks; ++e) {
      const int ci = tid + e * kPfThreads, r = ci >> 4, col = ci & 15;
      const int key = min(t * kPfStage + r, a.width - 1);
      stage[e] = *reinterpret_cast<const u32x4_t*>(kbase + (int64_t)key * D + col * 8);
      stage[kPfChunks + e] = *reinterpret_cast<const u32x4_t*>(vbase + (int64_t)key * D + col * 8);
    }
  };
  auto put = [&](int buf) {
#pragma unroll
    for (int e = 0; e < kPfChunks; ++e) {
      const int ci = tid + e * kPfThreads, r = ci >> 4, col = ci & 15;
      *reinterpret_cast<u32x4_t*>(&lds[buf][0][r * kPfRow + col * 16]) = stage[e];
      *reinterpret_cast<u32x4_t*>(&lds[buf][1][r * kPfRow + col * 16]) = stage[kPfChunks + e];
    }
  };

  // The wave's groups: queries q0[u] + c, u < kPfSub (group u of wave w: block rows 16 (w + kPfWaves u)).
  int q0[kPfSub];
  u32x4_t qop[kPfSub][KS];  // B operand of S^T = K Q^T: lane (c, g) holds q[q0 + c][32s + 8g .. +7] (0 past the end)
  SoftmaxState st[kPfSub];
  f32x4_t o[kPfSub][D / 16];
#pragma unroll
  for (int u = 0; u < kPfSub; ++u) {
    q0[u] = qb + 16 * (w + kPfWaves * u);
    const bool live = q0[u] + c < a.width;
    const uint16_t* qrow = a.q + ((int64_t)(b * a.width + (live ? q0[u] + c : 0)) * a.H + h) * D + g * 8;
#pragma unroll
    for (int s2 = 0; s2 < KS; ++s2)
      qop[u][s2] = live ? *reinterpret_cast<const u32x4_t*>(qrow + s2 * 32) : u32x4_t{0u, 0u, 0u, 0u};
    st[u] = SoftmaxState{-INFINITY, -INFINITY, 0.f};
#pragma unroll
    for (int nb = 0; nb < D / 16; ++nb) o[u][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  fetch(0);
  put(0);
  __syncthreads();
  for (int t = 0; t < nt; ++t) {
    fetch(t + 1 < nt ? t + 1 : t);  // unconditional: the last iteration re-reads its own tile (cache hit)
    // The stage's 32-key MFMA tiles in turn.
#pragma unroll
    for (int sub = 0; sub < kPfStage / 32; ++sub) {
    const int key0 = t * kPfStage + sub * 32;
    // Groups that see the tile (wave-uniform): a live group whose last query reaches the tile's first key.
    bool act[kPfSub];
    bool any = false;
#pragma unroll
    for (int u = 0; u < kPfSub; ++u) {
      act[u] = q0[u] < a.width && key0 <= q0[u] + 15;
      any |= act[u];
    }
    if (any) {
      const char* kl = lds[t & 1][0] + sub * 32 * kPfRow;
      const char* vl = lds[t & 1][1] + sub * 32 * kPfRow;
      u32x4_t pop[kPfSub];
      {
        u32x4_t kf[2][KS];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          const int rk = 8 * (c >> 2) + 4 * mb + (c & 3);
#pragma unroll
          for (int s2 = 0; s2 < KS; ++s2) kf[mb][s2] = *reinterpret_cast<const u32x4_t*>(kl + rk * kPfRow + g * 16 + s2 * 64);
        }
#pragma unroll
        for (int u = 0; u < kPfSub; ++u) {
          if (!act[u]) continue;
          f32x4_t sacc[2];
#pragma unroll
          for (int mb = 0; mb < 2; ++mb) {
            sacc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s2 = 0; s2 < KS; ++s2)
              sacc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf[mb][s2]),
                                                                 __builtin_bit_cast(bf16x8_t, qop[u][s2]), sacc[mb],
                                                                 0, 0, 0);
          }
          float sv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) sv[j] = sacc[j >> 2][j & 3];
          pop[u] = softmax_tile<D / 16>(sv, a.scale_log2, st[u], o[u], g, key0 + 8 * g, q0[u] + c + 1,
                                        key0 + 31 <= q0[u]);
        }
      }
      {
        // V operands by transpose reads: in lane group g (keys 8g .. 8g + 7) lane 4r + q points at key
        // 8g + 4h + r, dimensions 16e + 4q .. 16e + 4q + 3 (h = 0, 1), and ds_read_b64_tr_b16 hands lane c the
        // four keys' dimension 16e + c: block e's B operand, output column c = dimension 16e + c.
        const int rr = c >> 2, q4 = c & 3;
        const lds_char* vls = (const lds_char*)vl;  // vl points into LDS
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int off = (8 * g + rr) * kPfRow + (16 * e + 4 * q4) * 2;
          const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vls + off));
          const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vls + off + 4 * kPfRow));
          u32x4_t bop;
          bop[0] = (uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
          bop[1] = (uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
          bop[2] = (uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
          bop[3] = (uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
#pragma unroll
          for (int u = 0; u < kPfSub; ++u) {
            if (!act[u]) continue;
            o[u][e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, pop[u]),
                                                              __builtin_bit_cast(bf16x8_t, bop), o[u][e], 0, 0, 0);
          }
        }
      }
    }
    }
    put((t + 1) & 1);
    __syncthreads();
  }

  // ---- each group's 16 output rows: O / l, rounded to bf16
#pragma unroll
  for (int u = 0; u < kPfSub; ++u) {
    float l_tot = st[u].l_run + __shfl_xor(st[u].l_run, 16, kWave);
    l_tot += __shfl_xor(l_tot, 32, kWave);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float li = __shfl(l_tot, 4 * g + i, kWave);
      const int qq = q0[u] + 4 * g + i;
      if (qq >= a.width) continue;
      const float div = li > 0.f ? li : 1.f;
      uint16_t* orow = a.out + ((int64_t)(b * a.width + qq) * a.H + h) * D;
#pragma unroll
      for (int e = 0; e < 8; ++e) orow[16 * e + c] = (uint16_t)pack_bf16x2(o[u][e][i] / div, 0.f);  // dim 16e + c
    }
  }
}

// Wide heads (D = 256, 512): one workgroup of kPwWaves waves per (query block, head, context).  The block's
// NG = kPwSub * M groups of 16 queries (M = kPwWaves / (D/128)): group gi holds queries qb + 16 gi .. + 15.  Wave w
// holds the 128-dimension slice sl = w % (D/128) of q and O for the groups m + M u (m = w / (D/128), u < kPwSub).
// Per 32-key tile (K and V through LDS once for all waves):
//   1. each wave writes its slice's partial scores S^T = K_sl Q_sl^T of its groups to LDS;  barrier;
//   2. wave w runs the softmax of groups w, w + kPwWaves, ...: adds the D/128 partials in slice order, moves the
//      lazy reference max when needed, and publishes the group's P operand (bf16) and, when the reference max
//      moved, its 16 rescale factors;  barrier;
//   3. each wave rescales its O_sl of a group when told to and adds P V_sl.
// So each group's softmax runs once, not once per slice.  K has one LDS buffer (the next tile's goes in after
// barrier 1, when every wave has read this one), V two (the next tile's goes in during step 3 of this one, into the
// buffer the previous tile's P V read before barrier 1).
constexpr int kPwWaves = 8;
constexpr int kPwSub = 3;  // 16-query groups per wave

template <int D>
__global__ __launch_bounds__(64 * kPwWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_attn_wide_kernel(
    PrefillArgs a) {
  constexpr int NSL = D / 128, M = kPwWaves / NSL, NG = kPwSub * M, QW = 16 * NG;
  constexpr int OWN = (NG + kPwWaves - 1) / kPwWaves;  // groups whose softmax one wave runs, at most
  constexpr int kRowB = D * 2 + 16;                     // LDS bytes per key row, padded against bank conflicts
  constexpr int kRowChunks = D / 8;                     // 16-byte chunks per key row
  constexpr int kChunks = 32 * kRowChunks / (64 * kPwWaves);  // chunks of K (or of V) per thread per tile
  static_assert(NSL * M == kPwWaves && kChunks * 64 * kPwWaves == 32 * kRowChunks, "whole slices and chunks");
  __shared__ __attribute__((aligned(16))) char kl[32 * kRowB];     // K: 32 key rows
  __shared__ __attribute__((aligned(16))) char vl[2][32 * kRowB];  // V: two tiles
  __shared__ f32x4_t part[NG][NSL][2][64];  // partial scores: [group][slice][block mb][lane]
  __shared__ u32x4_t pex[NG][64];           // P operand of each group: [group][lane]
  __shared__ float alx[NG][16];             // rescale factor of each query of a group (when rflag)
  __shared__ int rflag[NG];                 // the group's reference max moved on this tile
  __shared__ float lsum[NG][16];            // probability sum of each query, at the end
  const int nqb = (a.width + QW - 1) / QW;
  const PfBlock blk = pf_block(nqb, a.H, (int)gridDim.z);
  const int qb = (nqb - 1 - blk.j) * QW;  // the longest blocks first
  const int h = blk.h, b = blk.b;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sl = w % NSL, m = w / NSL;
  const int64_t slot = clamp64(a.slots[b], 0, a.cache_rows - 1);
  const uint16_t* kbase = a.k + slot * a.s_row + h * a.s_head;
  const uint16_t* vbase = a.v + slot * a.s_row + h * a.s_head;
  const int kend = min(qb + QW, a.width);
  const int nt = (kend + 31) / 32;

  // Global -> LDS through one set of staging registers: thread tid moves 16-byte chunks tid, tid + 64 kPwWaves, ...
  // of a tile's K or V rows.  Rows past the context read its last key (finite: masked by the causal limit).
  u32x4_t stage[kChunks];
  auto fetch = [&](int t, const uint16_t* base) {
#pragma unroll
    for (int e = 0; e < kChunks; ++e) {
      const int ci = tid + e * 64 * kPwWaves, r = ci / kRowChunks, col = ci % kRowChunks;
      const int key = min(t * 32 + r, a.width - 1);
      stage[e] = *reinterpret_cast<const u32x4_t*>(base + (int64_t)key * D + col * 8);
    }
  };
  auto put = [&](char* dst) {
#pragma unroll
    for (int e = 0; e < kChunks; ++e) {
      const int ci = tid + e * 64 * kPwWaves, r = ci / kRowChunks, col = ci % kRowChunks;
      *reinterpret_cast<u32x4_t*>(dst + r * kRowB + col * 16) = stage[e];
    }
  };
  // Whether group gi sees the tile starting at key0: a live group whose last query reaches the tile's first key.
  auto sees = [&](int gi, int key0) { return qb + 16 * gi < a.width && key0 <= qb + 16 * gi + 15; };

  u32x4_t qop[kPwSub][4];  // lane (c, g): q[qb + 16 gi + c][128 sl + 32 s2 + 8g .. +7] (0 past the end)
  f32x4_t o[kPwSub][8];    // output column c of block e: dimension 128 sl + 16 e + c
#pragma unroll
  for (int u = 0; u < kPwSub; ++u) {
    const int row = qb + 16 * (m + M * u) + c;
    const bool live = row < a.width;
    const uint16_t* qrow = a.q + ((int64_t)(b * a.width + (live ? row : 0)) * a.H + h) * D + 128 * sl + g * 8;
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
      qop[u][s2] = live ? *reinterpret_cast<const u32x4_t*>(qrow + s2 * 32) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) o[u][e] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  SoftmaxState st[OWN];  // the softmax state of groups w + kPwWaves r
#pragma unroll
  for (int r = 0; r < OWN; ++r) st[r] = SoftmaxState{-INFINITY, -INFINITY, 0.f};

  fetch(0, kbase);
  put(kl);
  fetch(0, vbase);
  put(vl[0]);
  if (nt > 1) fetch(1, kbase);
  lds_barrier();
  for (int t = 0; t < nt; ++t) {
    const int key0 = t * 32;
    // 1. partial scores of this wave's groups over its slice
    {
      u32x4_t kf[2][4];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const int rk = 8 * (c >> 2) + 4 * mb + (c & 3);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
          kf[mb][s2] = *reinterpret_cast<const u32x4_t*>(&kl[rk * kRowB + 256 * sl + g * 16 + s2 * 64]);
      }
#pragma unroll
      for (int u = 0; u < kPwSub; ++u) {
        const int gi = m + M * u;
        if (!sees(gi, key0)) continue;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf[mb][s2]),
                                                          __builtin_bit_cast(bf16x8_t, qop[u][s2]), acc, 0, 0, 0);
          part[gi][sl][mb][lane] = acc;
        }
      }
    }
    lds_barrier();
    if (t + 1 < nt) {
      put(kl);             // every wave has read this tile's K
      fetch(t + 1, vbase);  // the next V, in flight during steps 2 and 3
    }
    // 2. the softmax of this wave's own groups
#pragma unroll
    for (int r = 0; r < OWN; ++r) {
      const int gi = w + kPwWaves * r;
      if (gi >= NG || !sees(gi, key0)) continue;
      const int q0 = qb + 16 * gi;
      f32x4_t sum[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        sum[mb] = part[gi][0][mb][lane];
#pragma unroll
        for (int s3 = 1; s3 < NSL; ++s3) sum[mb] += part[gi][s3][mb][lane];
      }
      float sv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) sv[j] = sum[j >> 2][j & 3];
      const int lim = q0 + c + 1;
      if (!(key0 + 31 <= q0)) {  // not every query of the group sees the whole tile
#pragma unroll
        for (int j = 0; j < 8; ++j) sv[j] = key0 + 8 * g + j < lim ? sv[j] : -INFINITY;
      }
      bool over = false;
#pragma unroll
      for (int j = 0; j < 8; ++j) over |= sv[j] > st[r].thr;
      const bool moved = __any(over);
      if (moved) {
        float mx = sv[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) mx = fmaxf(mx, sv[j]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float m_new = fmaxf(st[r].m_ref, mx * a.scale_log2);
        const float alpha = __builtin_amdgcn_exp2f(st[r].m_ref - (m_new == -INFINITY ? 0.f : m_new));  // -inf: 0
        st[r].l_run *= alpha;
        if (g == 0) alx[gi][c] = alpha;
        st[r].m_ref = m_new;
        st[r].thr = m_new == -INFINITY ? -INFINITY : (m_new + kLazyLog2) / a.scale_log2;
      }
      if (lane == 0) rflag[gi] = moved ? 1 : 0;
      const float m_use = st[r].m_ref == -INFINITY ? 0.f : st[r].m_ref;
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[j], a.scale_log2, -m_use));
        st[r].l_run += p[j];
      }
      u32x4_t pop;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        pop[q] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{p[2 * q], p[2 * q + 1]}), bf16x2_t));
      pex[gi][lane] = pop;
    }
    lds_barrier();
    // 3. O_sl += P V_sl for this wave's groups (rescaled first when the group's reference max moved)
    {
      u32x4_t pop[kPwSub];
#pragma unroll
      for (int u = 0; u < kPwSub; ++u) {
        const int gi = m + M * u;
        if (!sees(gi, key0)) continue;
        if (rflag[gi]) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float al = alx[gi][4 * g + i];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[u][e][i] *= al;
          }
        }
        pop[u] = pex[gi][lane];
      }
      // V operands by transpose reads, as in prefill_attn_kernel, from this wave's slice of the rows.
      const int rr = c >> 2, q4 = c & 3;
      const lds_char* vls = (const lds_char*)vl[t & 1];  // vl lives in LDS
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int off = (8 * g + rr) * kRowB + 256 * sl + (16 * e + 4 * q4) * 2;
        const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vls + off));
        const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vls + off + 4 * kRowB));
        u32x4_t bop;
        bop[0] = (uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
        bop[1] = (uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
        bop[2] = (uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
        bop[3] = (uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
#pragma unroll
        for (int u = 0; u < kPwSub; ++u) {
          if (!sees(m + M * u, key0)) continue;
          o[u][e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, pop[u]),
                                                            __builtin_bit_cast(bf16x8_t, bop), o[u][e], 0, 0, 0);
        }
      }
    }
    if (t + 1 < nt) {
      put(vl[(t + 1) & 1]);  // read last by tile t - 1's P V, before this tile's first barrier
      if (t + 2 < nt) fetch(t + 2, kbase);
    }
  }

  // ---- probability sums from the softmax owners, then each group's 16 output rows of this wave's slice
#pragma unroll
  for (int r = 0; r < OWN; ++r) {
    const int gi = w + kPwWaves * r;
    if (gi >= NG) continue;
    float l_tot = st[r].l_run + __shfl_xor(st[r].l_run, 16, kWave);
    l_tot += __shfl_xor(l_tot, 32, kWave);
    if (g == 0) lsum[gi][c] = l_tot;
  }
  lds_barrier();
#pragma unroll
  for (int u = 0; u < kPwSub; ++u) {
    const int gi = m + M * u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qq = qb + 16 * gi + 4 * g + i;
      if (qq >= a.width) continue;
      const float li = lsum[gi][4 * g + i];
      const float div = li > 0.f ? li : 1.f;
      uint16_t* orow = a.out + ((int64_t)(b * a.width + qq) * a.H + h) * D + 128 * sl;
#pragma unroll
      for (int e = 0; e < 8; ++e) orow[16 * e + c] = (uint16_t)pack_bf16x2(o[u][e][i] / div, 0.f);
    }
  }
}

}  // namespace omni

extern "C" int omni_prefill_attention(const void* q, const void* k_cache, const void* v_cache, int64_t stride_row,
                                      int64_t stride_head, int64_t stride_pos, int64_t cache_len,
                                      int64_t cache_rows, const int64_t* slots, int32_t contexts, int32_t width,
                                      int32_t heads, int32_t head_dim, float scale, void* out, int32_t dtype,
                                      void* stream) {
  if (contexts < 0 || width < 0 || heads <= 0 || cache_rows <= 0) return OMNI_ERR_INVALID;
  if (dtype != OMNI_BF16) return OMNI_ERR_DTYPE;
  if ((head_dim != 128 && head_dim != 256 && head_dim != 512) || stride_pos != head_dim) return OMNI_ERR_SHAPE;
  if (!(scale > 0.f) || width > cache_len) return OMNI_ERR_INVALID;
  if (contexts == 0 || width == 0) return OMNI_OK;
  if (!q || !k_cache || !v_cache || !slots || !out) return OMNI_ERR_INVALID;
  if (((uintptr_t)q | (uintptr_t)out | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u) return OMNI_ERR_INVALID;
  if ((stride_row | stride_head) % 8 != 0) return OMNI_ERR_INVALID;
  if ((int64_t)contexts * width * heads >= (int64_t{1} << 31) / head_dim) return OMNI_ERR_INVALID;
  omni::PrefillArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k_cache;
  a.v = (const uint16_t*)v_cache;
  a.slots = slots;
  a.s_row = stride_row;
  a.s_head = stride_head;
  a.cache_rows = cache_rows;
  a.width = width;
  a.H = heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = (uint16_t*)out;
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128) {
    dim3 grid((width + omni::kPfQueries - 1) / omni::kPfQueries, heads, contexts);
    omni::prefill_attn_kernel<<<grid, 64 * omni::kPfWaves, 0, s>>>(a);
  } else {
    const int qw = 16 * omni::kPwSub * (omni::kPwWaves / (head_dim / 128));  // queries per workgroup
    dim3 grid((width + qw - 1) / qw, heads, contexts);
    if (head_dim == 256)
      omni::prefill_attn_wide_kernel<256><<<grid, 64 * omni::kPwWaves, 0, s>>>(a);
    else
      omni::prefill_attn_wide_kernel<512><<<grid, 64 * omni::kPwWaves, 0, s>>>(a);
  }
  return omni_launch_status();
}
