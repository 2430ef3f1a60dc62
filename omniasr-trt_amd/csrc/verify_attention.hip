// Multi-query split-K flash-decode verification attention for gfx950.
//
// Semantics of ``kernels.draft_attention`` (``_beam_ctx`` CAUSAL=True + ``_beam_combine``,
// src/omniasr_trt/kernels.py:338-358, 56-113, 146-161) and, with one query per row, of
// ``kernels.decode_attention`` (src/omniasr_trt/kernels.py:406-423, 163-211): query i of row b
// attends to keys [0, lengths[b] + i); softmax in fp32; split partials (acc, m, l) are merged by
// log-sum-exp with w_s = exp(m_s - max m) (0 for an empty split) and out = sum w_s acc_s /
// sum w_s l_s (0 when that sum is 0).
//
// Work decompositions.  The unit of work is a (head, row) pair; its T <= 16 queries share one read of K and V,
// 32 keys at a time (the tile math of attn_tiles.h).
//  * Halves (bf16, head_dim 128, T <= 11, rows <= 256, rows x heads >= 128; verify_attn_pair_kernel): one 8-wave
//    workgroup per unit, taking the first half of a long unit and the second half of a short one (units ranked by
//    length on the device), so every CU streams about the same number of tiles -- a CU reads at most ~30 GB/s, so
//    HBM runs at full rate only while nearly all CUs are busy.  The waves' tiles run through both halves in one
//    pipeline; a unit's two halves meet through partials written through to the coherence point and a ticket per
//    unit, and the workgroup of the second half fetches the first while its waves finish.  One launch; results
//    do not depend on timing.
//  * Split-K (every other shape; verify_attn_mfma_kernel / verify_attn_slice_kernel / verify_attn_valu_kernel):
//    one wavefront per (key split, head, row), grid (splits, heads, rows) -- for head dims 256 and 512 one
//    workgroup of D/128 waves per split, a wave per 128-dimension slice, the partial scores added through LDS (the
//    tile registers of the 128-dimension kernel, two tiles in flight, two waves per SIMD).  A row's 32-key tiles are
//    dealt round-robin over its splits.
//    Splits beyond a row's last key exit at once, so the grid depends on the key bucket only (graph capture)
//    while ragged rows read just their own keys.  The splits' partials are merged by a second launch or by the
//    last split to finish (ticket per (row, head)); a row with one split writes its output directly.
// bf16 with head_dim a multiple of 128 runs on MFMA with every K/V element loaded straight into the operand layout
// (128-bit loads, no LDS); fp32, or bf16 with another head_dim, runs a vector-ALU wave with fp32 products (the
// reference's IEEE path for fp32 agreement checks).  The beams' attention (context by these kernels, generated
// keys through pointers) is at the end of the file.
#include <math.h>

#include <mutex>

#include "attn_tiles.h"
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
  int causal;        // 1: query i sees lengths + i keys (drafted step); 0: every query sees lengths keys (beams)
  int ctx_splits;    // key splits of the grid (= splits, or splits - 1 with a generated-keys split)
  int gen_split;     // partial slot of the beams' generated keys (merged with the key splits), or -1
  int balanced;      // wide-head split-K with a fixed number of workgroups per head (see balanced_split)
  int rows;          // rows of the launch (balanced split-K)
  // The beams' generated keys as tiles of the halves kernel (verify_attn_pair_kernel<D, true>): key j of row r (the
  // unit's group g = r / T, beam r - g T) is position j of generated-cache row ptr[r, j], j < gen_len[r] <= gen_cap.
  const char* kg = nullptr;  // generated K / V, [gen_rows, H, gen_cap, D] with key rows of D elements
  const char* vg = nullptr;
  int64_t g_row = 0, g_head = 0;  // element strides of a generated-cache row and head
  const int32_t* ptr = nullptr;
  int64_t ptr_stride = 0;
  const int64_t* gen_len = nullptr;
  int gen_cap = 0, gen_rows = 0;
  int gen_table = 0;  // LDS entries of a unit's table of generated-key offsets (a multiple of 32)
  // Optional: each group's generated keys listed once per distinct (row, position) by beam_gen_list_kernel --
  // offsets (row and position only), beam masks, lengths; row stride glist_stride.  nullptr: every beam's own keys.
  const uint32_t* glist = nullptr;
  const uint16_t* gmask = nullptr;
  const int32_t* gcount = nullptr;
  int64_t glist_stride = 0;
};

struct SplitRange {
  int64_t n;      // keys every query of the row sees (lengths[b], clamped to the cache)
  int64_t total;  // keys the row's last query sees (clamped to the cache and the grid)
  int64_t stop;   // end of this split's keys (contiguous ranges)
  int64_t start;  // first key of this split (contiguous ranges)
  int nact;       // splits holding keys of this row (>= 1: an empty row still writes zeros)
};

__device__ __forceinline__ SplitRange split_range(const AttnArgs& a, int b, int sp) {
  SplitRange r;
  r.n = clamp64(a.lengths[b], 0, a.cache_len);
  int64_t total = r.n + (a.causal ? a.T - 1 : 0);  // keys the last query sees
  total = total < a.cache_len ? total : a.cache_len;
  const int64_t covered = (int64_t)a.ctx_splits * a.chunk;
  total = total < covered ? total : covered;
  r.total = total;
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

// The in-kernel merge reads partials written by waves on other XCDs, whose L2s are not coherent with each other.
// Those partials are stored and loaded with agent-scope (relaxed atomic) accesses, which go through the L2 to the
// device's coherence point: no L2 writeback or invalidate of the whole cache is needed, only the wave's own stores
// completing before its ticket.
__device__ __forceinline__ void put_partial(float* p, float v, bool through) {
  if (through) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

// Memory order of the merge tickets' fetch-adds.  Relaxed: the ordering rests on each wave's s_waitcnt before its
// ticket (its write-through partial stores acknowledged at the coherence point) and on the merger's loads being
// issued only after its ticket returned.  OMNI_TICKET_ACQ_REL=1 builds them as agent-scope acquire-release
// operations instead (an L2 write-back before and an L2 invalidate after each, on gfx950).
#ifndef OMNI_TICKET_ACQ_REL
#define OMNI_TICKET_ACQ_REL 0
#endif
constexpr int kTicketOrder = OMNI_TICKET_ACQ_REL ? __ATOMIC_ACQ_REL : __ATOMIC_RELAXED;

// Two floats (m, l) written through in one 8-byte agent-scope store.
__device__ __forceinline__ void put_through2(float* p, float x, float y) {
  const uint64_t v = (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Four floats of a partial written through to the coherence point: element ``at`` of the partial buffer ``base``
// (wave-uniform).  One 16-byte store with the agent-scope cache policy (SC1: through the L2 to the device's
// coherence point), issued through a buffer resource over ``base``; the offset is 32-bit (the launchers refuse
// workspaces of 4 GiB and more).  OMNI_THROUGH16=0 builds the earlier form, two 8-byte agent-scope atomic stores.
#ifndef OMNI_THROUGH16
#define OMNI_THROUGH16 1
#endif
constexpr int kPolicySc1 = 16;  // buffer instruction cache policy bits: SC1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(const float* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, -1, 0x00020000);
}

__device__ __forceinline__ void put_through4(float* base, int64_t at, f32x4_t v) {
#if OMNI_THROUGH16
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), partial_rsrc(base), (uint32_t)at * 4u, 0,
                                         kPolicySc1);
#else
  put_through2(base + at, v[0], v[1]);
  put_through2(base + at + 2, v[2], v[3]);
#endif
}

// Partial slot of the q-th partial to merge: the row's key splits, then the generated-keys slot if any.
__device__ __forceinline__ int merge_slot(const AttnArgs& a, int nact, int q) {
  return q < nact ? q : a.gen_split;
}

// Log-sum-exp merge of the partials of (row b, head h) by one wave (the merge launch, after the split kernel);
// writes the output.
template <typename OutT>
__device__ void merge_splits(const AttnArgs& a, int b, int h, int nact) {
  const int lane = lane_id();
  const int nq = nact + (a.gen_split >= 0 ? 1 : 0);
  const int64_t split0 = ((int64_t)b * a.H + h) * a.splits;
  OutT* out = reinterpret_cast<OutT*>(a.out);
  auto get = [](const float* p) { return *p; };
  for (int t = 0; t < a.T; ++t) {
    float top = -INFINITY;
    for (int q = lane; q < nq; q += kWave)
      top = fmaxf(top, get(a.part_ml + ((split0 + merge_slot(a, nact, q)) * a.T + t) * 2));
    top = wave_max(top);
    float den = 0.f;
    for (int q = lane; q < nq; q += kWave) {
      const int64_t ml = ((split0 + merge_slot(a, nact, q)) * a.T + t) * 2;
      const float m = get(a.part_ml + ml);
      const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - top);
      den += w * get(a.part_ml + ml + 1);
    }
    den = wave_sum(den);
    const float div = den > 0.f ? den : 1.f;
    OutT* orow = out + ((int64_t)(b * a.T + t) * a.H + h) * a.D;
    for (int d = lane * 4; d < a.D; d += kWave * 4) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      for (int q = 0; q < nq; ++q) {
        const int64_t slot = (split0 + merge_slot(a, nact, q)) * a.T + t;
        const float m = get(a.part_ml + slot * 2);
        const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - top);
        acc += w * *reinterpret_cast<const f32x4_t*>(a.part_o + slot * a.D + d);
      }
      store4<OutT>(orow + d, acc / div);
    }
  }
}

// The in-kernel merge by the row's last split: lane l owns the floats f = 1024p + 256r + 4l (query f / D) of the
// row's T x D output block, and every load of a batch of up to 8 partials x 1024 floats is in flight at once (the
// tile registers are free by then), so a typical merge is one memory round trip.
__device__ __forceinline__ f32x4_t get_through4(const float* base, int64_t at) {
#if OMNI_THROUGH16
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(partial_rsrc(base), (uint32_t)at * 4u, 0,
                                                                           kPolicySc1));
#else
  const float* p = base + at;
  const uint64_t lo = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t hi = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)) + 1, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
  return f32x4_t{__uint_as_float((uint32_t)lo), __uint_as_float((uint32_t)(lo >> 32)),
                 __uint_as_float((uint32_t)hi), __uint_as_float((uint32_t)(hi >> 32))};
#endif
}

// The partials of (row b, head h) merged by one wave, each read at the coherence point: the row's ``nact`` key
// splits from slot ``first_slot`` on (default: the unit's own slots), then the generated keys' partial if any (slot
// ``gen_slot``; default: gen_split past the unit's first slot).
template <typename OutT>
__device__ void merge_splits_fast(const AttnArgs& a, int b, int h, int nact, int d0 = 0, int dw = -1,
                                  int64_t first_slot = -1, int64_t gen_slot = -1) {
  constexpr int kS = 8, kR = 3;
  const int lane = lane_id();
  const int T = a.T, D = a.D;
  if (dw < 0) dw = D;  // dimensions d0 .. d0 + dw - 1 of every query (dw a multiple of 4)
  const int nf = T * dw;
  const int nq = nact + (a.gen_split >= 0 ? 1 : 0);
  const int64_t split0 = first_slot >= 0 ? first_slot : ((int64_t)b * a.H + h) * a.splits;
  const int64_t gslot = gen_slot >= 0 ? gen_slot : split0 + a.gen_split;
  OutT* out = reinterpret_cast<OutT*>(a.out);
  for (int f0 = 0; f0 < nf; f0 += kR * 256) {
    float top[kR], den[kR];
    f32x4_t acc[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      top[r] = -INFINITY;
      den[r] = 0.f;
      acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    for (int q0 = 0; q0 < nq; q0 += kS) {
      f32x4_t ov[kS][kR];
      float mv[kS][kR], lv[kS][kR];
#pragma unroll
      for (int sq = 0; sq < kS; ++sq) {
#pragma unroll
        for (int r = 0; r < kR; ++r) {
          const int f = f0 + r * 256 + 4 * lane;
          mv[sq][r] = -INFINITY;
          lv[sq][r] = 0.f;
          ov[sq][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          if (q0 + sq < nq && f < nf) {
            const int t = f / dw;
            const int64_t slot = (q0 + sq < nact ? split0 + q0 + sq : gslot) * T + t;
            const uint64_t ml = __hip_atomic_load(reinterpret_cast<uint64_t*>(a.part_ml + slot * 2), __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
            mv[sq][r] = __uint_as_float((uint32_t)ml);
            lv[sq][r] = __uint_as_float((uint32_t)(ml >> 32));
            ov[sq][r] = get_through4(a.part_o, slot * D + d0 + (f - t * dw));
          }
        }
      }
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        float t2 = top[r];
#pragma unroll
        for (int sq = 0; sq < kS; ++sq) t2 = fmaxf(t2, mv[sq][r]);
        const float rs = top[r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(top[r] - t2);
        den[r] *= rs;
        acc[r] *= rs;
#pragma unroll
        for (int sq = 0; sq < kS; ++sq) {
          const float wt = mv[sq][r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv[sq][r] - t2);
          den[r] += wt * lv[sq][r];
          acc[r] += wt * ov[sq][r];
        }
        top[r] = t2;
      }
    }
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const int f = f0 + r * 256 + 4 * lane;
      if (f >= nf) continue;
      const int t = f / dw;
      const float div = den[r] > 0.f ? den[r] : 1.f;
      store4<OutT>(out + ((int64_t)(b * T + t) * a.H + h) * D + d0 + (f - t * dw), acc[r] / div);
    }
  }
}

// After a split wrote its partial: the last of the row's ``nact`` splits merges them all.
template <typename OutT>
__device__ __forceinline__ void finish_split(const AttnArgs& a, int b, int h, int nact) {
  if (a.separate) return;
  // This wave's partial stores (agent scope, written through) have reached the coherence point before its ticket
  // is taken; the compiler barriers keep them on their side of the wait.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  int* counter = &a.counters[b * a.H + h];
  int ticket = 0;
  if (lane_id() == 0) ticket = __hip_atomic_fetch_add(counter, 1, kTicketOrder, __HIP_MEMORY_SCOPE_AGENT);
  ticket = __shfl(ticket, 0, kWave);
  if (ticket != nact - 1) return;
  merge_splits_fast<OutT>(a, b, h, nact);  // every split's partial, read at the coherence point
  if (lane_id() == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------- MFMA

// One split's share of row b, head h: tiles sp, sp + nact, sp + 2 nact, ... of the row (r.nact splits).  Leaves
// the split's unnormalised output rows in ``o`` and its softmax state in ``st``.
// Two tiles of registers: the next tile's loads are in flight during the current tile's math.
template <int D>
__device__ __forceinline__ void attend_split(const AttnArgs& a, int b, int h, int sp, const SplitRange& r,
                                             SoftmaxState& st, f32x4_t (&o)[D / 16], int64_t t0 = 0,
                                             int64_t t1 = -1) {
  constexpr int KS = D / 32;  // k-steps of S^T = K Q^T
  constexpr int NG = D / 128;  // 128-wide output groups
  const int lane = lane_id(), c = lane & 15, g = lane >> 4;
  const int T = a.T;

  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(a.k) + b * a.s_row + h * a.s_head;
  const uint16_t* vbase = reinterpret_cast<const uint16_t*>(a.v) + b * a.s_row + h * a.s_head;
  const int64_t last_key = a.cache_len - 1;
  const float c_scale = a.scale_log2;

  // B operand of S^T = K Q^T: lane (c, g) holds q[c][32s + 8g .. 32s + 8g + 7].
  u32x4_t qop[KS];
  {
    const u32x4_t zero = {0u, 0u, 0u, 0u};
    const uint16_t* qrow =
        reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)(b * T + c) * a.H + h) * D + g * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) qop[s] = c < T ? *reinterpret_cast<const u32x4_t*>(qrow + s * 32) : zero;
  }

  st = SoftmaxState{-INFINITY, -INFINITY, 0.f};
#pragma unroll
  for (int nb = 0; nb < NG * 8; ++nb) o[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};  // row 4g + i, dimension 128gg + 8c + e

  // The row's 32-key tiles t0, t0 + 1, ... < t1 (default: all of them) are dealt out round-robin over the nact
  // splits: split sp takes tiles t0 + sp, t0 + sp + nact, ...  Each split gets the same number of tiles (give or
  // take one), and at any moment the splits read neighbouring tiles (DRAM locality), unlike contiguous ranges.
  // One branch-free loader and one attend routine serve whole tiles and those reaching past some query's last
  // key, so the only branches around the loads are the loop's own: the wait before a tile's math then leaves the
  // next tile's loads in flight (a load under a condition makes the compiler wait for every outstanding load
  // where the branches join).
  const int64_t row_tiles = (r.total + 31) >> 5;
  const int64_t end = t1 < 0 || t1 > row_tiles ? row_tiles : t1;
  const int64_t first = t0 + sp;
  const int64_t ntot = first < end ? (end - first + r.nact - 1) / r.nact : 0;
  // The launcher sends only caches with contiguous key rows (s_pos == D) here.
  const char* kt = reinterpret_cast<const char*>(kbase) + first * 32 * a.s_pos * 2;
  const char* vt = reinterpret_cast<const char*>(vbase) + first * 32 * a.s_pos * 2;
  const int64_t tile_bytes = (int64_t)r.nact * 32 * a.s_pos * 2;  // stride between this split's tiles
  const int64_t own = r.n + (a.causal ? c : 0);
  const int lim_c = (int)(own < r.total ? own : r.total);  // query c's key limit (keys fit in 32 bits)
  auto load_k = [&](KVTile<D>& t, int64_t k) {
    const int64_t kb = (first + k * r.nact) * 32;  // < total <= cache_len
    const int64_t kmax = last_key - kb, vstop = r.total - kb;
    load_tile_clamped<D>(t, kt + k * tile_bytes, vt + k * tile_bytes, kmax < 31 ? (int)kmax : 31,
                         vstop < 32 ? (int)vstop : 32, c, g);
  };
  auto attend_k = [&](const KVTile<D>& t, int64_t k) {
    attend<D>(t, qop, c_scale, st, o, g, (int)((first + k * r.nact) * 32) + 8 * g, lim_c);
  };
  if (ntot > 0) {
    KVTile<D> A, B;
    load_k(A, 0);
    int64_t k = 0;
    for (; k + 2 < ntot; k += 2) {
      load_k(B, k + 1);
      attend_k(A, k);
      load_k(A, k + 2);
      attend_k(B, k + 1);
    }
    if (k + 1 < ntot) {
      load_k(B, k + 1);
      attend_k(A, k);
      attend_k(B, k + 1);
    } else {
      attend_k(A, k);
    }
  }

}

// Split-K: one wave per (split, head, row); the split's partial (or, for a row with one split, the output) goes to
// HBM and a second launch (or the row's last split) merges them.
template <int D>
__global__ __launch_bounds__(64, 2) void verify_attn_mfma_kernel(AttnArgs a) {
  constexpr int NG = D / 128;
  const int sp = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const SplitRange r = split_range(a, b, sp);
  if (sp >= r.nact) return;
  const int lane = threadIdx.x, c = lane & 15, g = lane >> 4;
  const int T = a.T;
  SoftmaxState st;
  f32x4_t o[NG * 8];
  attend_split<D>(a, b, h, sp, r, st, o);

  // ---- finish: per-query sums, then either the output or this split's partial
  float l_tot = st.l_run + __shfl_xor(st.l_run, 16, kWave);
  l_tot += __shfl_xor(l_tot, 32, kWave);
  float li[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) li[i] = __shfl(l_tot, 4 * g + i, kWave);
  if (r.nact == 1 && a.gen_split < 0) {
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
  const bool through = !a.separate;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * g + i;
    if (t >= T) continue;
#pragma unroll
    for (int gg = 0; gg < NG; ++gg) {
      float* po = a.part_o + (base + t) * D + gg * 128 + c * 8;
      if (through) {
        const int64_t at = (base + t) * D + gg * 128 + c * 8;
        put_through4(a.part_o, at, f32x4_t{o[gg * 8 + 0][i], o[gg * 8 + 1][i], o[gg * 8 + 2][i], o[gg * 8 + 3][i]});
        put_through4(a.part_o, at + 4, f32x4_t{o[gg * 8 + 4][i], o[gg * 8 + 5][i], o[gg * 8 + 6][i], o[gg * 8 + 7][i]});
      } else {
        reinterpret_cast<f32x4_t*>(po)[0] = f32x4_t{o[gg * 8 + 0][i], o[gg * 8 + 1][i], o[gg * 8 + 2][i],
                                                    o[gg * 8 + 3][i]};
        reinterpret_cast<f32x4_t*>(po)[1] = f32x4_t{o[gg * 8 + 4][i], o[gg * 8 + 5][i], o[gg * 8 + 6][i],
                                                    o[gg * 8 + 7][i]};
      }
    }
  }
  if (g == 0 && c < T) {
    put_partial(a.part_ml + (base + c) * 2, st.m_ref, through);
    put_partial(a.part_ml + (base + c) * 2 + 1, l_tot, through);
  }
  finish_split<uint16_t>(a, b, h, r.nact);
}

// Balanced split-K for wide heads: a fixed budget of ``a.splits`` workgroups per head (about two per CU in all) is
// dealt to the rows in proportion to their tile counts -- one to every row, the rest by the largest remainder of
// (budget - rows) x tiles / total tiles, ties to the lower row -- so every workgroup streams about the same number
// of tiles whatever the rows' lengths.  Workgroup j of a head works on split k of row b, one of the row's nact
// splits (tiles dealt round-robin over them, as in split-K); the partials of a head's workgroups take the head's
// a.splits slots in workgroup order, so a unit's splits have consecutive slots from ``first``.  Every workgroup
// computes the same deal from the rows' lengths (rows <= kBalancedMaxRows).  b < 0: no work (every row empty).
// GEN: a row's tiles are its context tiles and then its beams' generated keys (see verify_attn_slice_kernel), whose
// counts the deal leaves in gl[row][beam].
constexpr int kBalancedMaxRows = 64;
constexpr int kWideMaxBeams = 16;
constexpr int kWideMaxGenTable = 4096;  // generated keys of a unit taken as tiles of the balanced wide-head kernel

// The generated keys of row ``row`` (a beam) in use.
__device__ __forceinline__ int gen_count(const AttnArgs& a, int64_t row) {
  return (int)clamp64(a.gen_len[row], 0, a.gen_cap);
}

struct BalancedSplit {
  int b, k, nact, first;
};

// Bit j: whether query c sees key 8g + j of a tile of a generated-key list (its keys' beam masks at msk8, in LDS).
__device__ __forceinline__ int gen_bits(const uint16_t* msk8, int c) {
  const u32x4_t m = *reinterpret_cast<const u32x4_t*>(msk8);
  int bits = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) bits |= (int)((m[j >> 1] >> (16 * (j & 1) + c)) & 1u) << j;
  return bits;
}

// A unit's table of generated keys in LDS (group b's ng keys; cnt: its beams' key counts, LDS): the byte offset of
// key f from the head's base and the beams that see it, padded to whole tiles with the list's last key (a key in use,
// so the padding reads finite values) seen by none.  With a.glist the keys are the group's list (each distinct (row,
// position) once); otherwise beam 0's keys, then beam 1's, ... (key j of beam e at row ptr[e, j]).  Every thread of
// the workgroup (nt of them) calls it; the caller's barrier follows.
__device__ __forceinline__ void fill_gen_table(const AttnArgs& a, int b, int ng, const int* cnt, uint32_t* tab,
                                               uint16_t* msk, int nt, int D) {
  const int T = a.T;
  for (int f = threadIdx.x; f < ((ng + 31) & ~31); f += nt) {
    const int ff = f < ng ? f : ng - 1;
    if (a.glist) {
      const int64_t at = (int64_t)b * a.glist_stride + ff;
      tab[f] = a.glist[at];
      msk[f] = f < ng ? a.gmask[at] : (uint16_t)0;
      continue;
    }
    int e = 0, base = 0;
    for (; e < T - 1; ++e) {
      const int ne = cnt[e];
      if (ff < base + ne) break;
      base += ne;
    }
    const int j = ff - base;
    const int64_t src = clamp64(a.ptr[(int64_t)(b * T + e) * a.ptr_stride + j], 0, a.gen_rows - 1);
    tab[f] = (uint32_t)((src * a.g_row + (int64_t)j * D) * 2);
    msk[f] = f < ng ? (uint16_t)(1u << e) : (uint16_t)0;
  }
}

// One workgroup per group: the group's generated keys listed once per distinct (row, position).  Beams share most of
// their history, so a key several beams reach through their pointers is read once per launch and seen by all of
// them.  Order: by position, then by the first beam that reaches the key (the same list every call).  list[f]: the
// byte offset of key f from a generated cache's (layer's) head base, row ptr[r, j] and position j; mask[f]: the beams
// that see it; count: the list's length.  Thread t lists positions t, t + 256, ...: one round trip for the pointers
// and one scan per round.  Built once per search step, read by every layer's launch.
struct GenListArgs {
  const int32_t* ptr;
  int64_t ptr_stride;
  const int64_t* gen_len;
  int64_t gen_cap, gen_rows, g_row, g_pos;
  int beams;
  uint32_t* list;
  uint16_t* mask;
  int32_t* count;
  int64_t stride;
};

__global__ __launch_bounds__(256) void beam_gen_list_kernel(GenListArgs a) {
  constexpr int NT = 256, NW = NT / 64, MAXB = kWideMaxBeams;
  __shared__ int wsum[NW];
  const int grp = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, T = a.beams;
  const int32_t* prow = a.ptr + (int64_t)grp * T * a.ptr_stride;
  // The beams' key counts (the same for every thread) and the first round's pointers load together: a pointer's
  // address does not depend on the count (positions clamped into the capacity).
  int cnt[MAXB], raw[MAXB];
  int longest = 0;
#pragma unroll
  for (int e = 0; e < MAXB; ++e) {
    cnt[e] = e < T ? (int)clamp64(a.gen_len[(int64_t)grp * T + e], 0, a.gen_cap) : 0;
    raw[e] = e < T ? prow[(int64_t)e * a.ptr_stride + min((int64_t)tid, a.gen_cap - 1)] : 0;
    longest = max(longest, cnt[e]);
  }
  uint32_t* list = a.list + (int64_t)grp * a.stride;
  uint16_t* mask = a.mask + (int64_t)grp * a.stride;
  int total = 0;
  for (int j0 = 0; j0 < longest; j0 += NT) {
    const int j = j0 + tid;
    int src[MAXB];
#pragma unroll
    for (int e = 0; e < MAXB; ++e) {  // beam e's row for position j (clamped), -1 where the beam has no key j
      const int p = j0 == 0 ? raw[e] : (e < T && j < cnt[e] ? prow[(int64_t)e * a.ptr_stride + j] : 0);
      src[e] = e < T && j < cnt[e] ? (int)clamp64(p, 0, a.gen_rows - 1) : -1;
    }
    auto first = [&](int e) {  // beam e reaches a key no earlier beam reaches
      bool f = src[e] >= 0;
#pragma unroll
      for (int e2 = 0; e2 < MAXB; ++e2) f &= !(e2 < e && src[e2] == src[e]);
      return f;
    };
    int mine = 0;
#pragma unroll
    for (int e = 0; e < MAXB; ++e) mine += first(e) ? 1 : 0;
    int incl = mine;  // inclusive scan within the wave, then over the waves' totals
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o, kWave);
      incl += lane >= o ? v : 0;
    }
    if (lane == 63) wsum[wv] = incl;
    __syncthreads();
    int f = total + incl - mine;
    for (int q = 0; q < NW; ++q) {
      const int x = wsum[q];
      f += q < wv ? x : 0;
      total += x;
    }
#pragma unroll
    for (int e = 0; e < MAXB; ++e) {
      if (!first(e)) continue;
      uint32_t m = 0;
#pragma unroll
      for (int e2 = 0; e2 < MAXB; ++e2) m |= src[e2] == src[e] ? 1u << e2 : 0u;
      list[f] = (uint32_t)(((int64_t)src[e] * a.g_row + (int64_t)j * a.g_pos) * 2);
      mask[f] = (uint16_t)m;
      ++f;
    }
    __syncthreads();  // wsum is written again in the next round
  }
  if (tid == 0) a.count[grp] = total;
}

template <bool GEN = false>
__device__ BalancedSplit balanced_split(const AttnArgs& a, int j, int* gl = nullptr) {
  __shared__ int nt[kBalancedMaxRows], wk[kBalancedMaxRows], rem[kBalancedMaxRows];
  __shared__ int s_total, s_given;
  const int tid = threadIdx.x, rows = a.rows, budget = a.splits;  // the launcher ensures rows <= blockDim.x
  if (tid < rows) {
    int n = (int)((split_range(a, tid, 0).total + 31) >> 5);
    if constexpr (GEN) {
      int ng = 0;
      for (int e = 0; e < a.T; ++e) {
        const int ne = gen_count(a, (int64_t)tid * a.T + e);
        gl[tid * a.T + e] = ne;
        ng += ne;
      }
      n += ((a.glist ? min(a.gcount[tid], a.gen_table) : ng) + 31) >> 5;
    }
    nt[tid] = n;
  }
  __syncthreads();
  if (tid == 0) {
    int total = 0;
    for (int b = 0; b < rows; ++b) total += nt[b];
    s_total = total;
  }
  __syncthreads();
  const int total = s_total, spare = budget - rows;
  if (tid < rows) {
    const int64_t share = total > 0 ? (int64_t)spare * nt[tid] : 0;
    wk[tid] = 1 + (total > 0 ? (int)(share / total) : 0);
    rem[tid] = total > 0 ? (int)(share % total) : 0;
  }
  __syncthreads();
  if (tid == 0) {
    int given = 0;
    for (int b = 0; b < rows; ++b) given += wk[b];
    s_given = given;
  }
  __syncthreads();
  const int left = total > 0 ? budget - s_given : 0;  // < rows: one more to the rows of the largest remainders
  int extra = 0;
  if (tid < rows) {
    int rank = 0;
    for (int o = 0; o < rows; ++o) rank += rem[o] > rem[tid] || (rem[o] == rem[tid] && o < tid);
    extra = rank < left;
  }
  __syncthreads();
  if (tid < rows) wk[tid] += extra;
  __syncthreads();
  BalancedSplit out{-1, 0, 1, 0};
  int first = 0;
  for (int b = 0; b < rows; ++b) {
    if (j < first + wk[b]) {
      out = BalancedSplit{b, j - first, wk[b], first};
      break;
    }
    first += wk[b];
  }
  return out;
}

// Split-K for head dims past 128 (256, 512): one workgroup of D/128 waves per (split, head, row), wave w holding
// dimensions 128w .. 128w + 127 of q, K, V and O.  Each wave reads its slice of a tile (32 keys x 256 bytes of K
// and of V; two tiles in flight, the register budget of the 128-dimension kernel), its partial scores go to LDS,
// and after one barrier every wave adds the D/128 partials in slice order, so all waves hold the same scores and
// the same softmax state; each then accumulates its own slice of P V.  Tiles are dealt to the splits as in
// attend_split; the partials and the last split's merge are those of verify_attn_mfma_kernel.
//
// GEN (beams, balanced): a row's tiles are its context tiles followed by its group's generated keys as one list cut
// into 32-key tiles -- the step's list of distinct (row, position) keys (a.glist), or beam 0's keys, then beam 1's,
// ... -- key f at the byte offset the workgroup's table in LDS gives and seen by the beams of its mask, so the deal,
// the pipeline and the merge treat the generated keys like any other tile.
template <int D, int G, bool GEN = false>
__global__ __launch_bounds__(64 * (D / 128), G == 1 ? 2 : 1) void verify_attn_slice_kernel(AttnArgs a) {
  constexpr int NSL = D / 128;
  __shared__ float sx[2][NSL][G][kWave * 8];  // partial scores of a tile by slice and query group, double-buffered
  __shared__ int s_ticket;
  // GEN: the rows' generated-key counts [rows][T] and the unit's table of key offsets
  __shared__ int s_gl[GEN ? kBalancedMaxRows * kWideMaxBeams : 1];
  __shared__ __align__(16) uint32_t s_tab[GEN ? kWideMaxGenTable : 4];
  __shared__ __align__(16) uint16_t s_msk[GEN ? kWideMaxGenTable : 8];
  const int h = blockIdx.y;
  int sp, b;
  SplitRange r;
  int64_t slot0;  // partial slot of the unit's first split
  if (a.balanced) {
    const BalancedSplit bs = balanced_split<GEN>(a, blockIdx.x, s_gl);
    if (bs.b < 0) return;  // uniform over the workgroup
    b = bs.b;
    sp = bs.k;
    r = split_range(a, b, 0);
    r.nact = bs.nact;
    slot0 = (int64_t)h * a.splits + bs.first;
  } else {
    sp = blockIdx.x;
    b = blockIdx.z;
    r = split_range(a, b, sp);
    if (sp >= r.nact) return;  // uniform over the workgroup
    slot0 = ((int64_t)b * a.H + h) * a.splits;
  }
  const int lane = lane_id(), sl = threadIdx.x / kWave, c = lane & 15, g = lane >> 4;  // sl: this wave's slice
  const int T = a.T;

  // Query group u holds queries 16u .. 16u + 15 of the row.  B operand of the slice's S^T = K Q^T: lane (c, g) holds
  // q[16u + c][128 sl + 32s + 8g .. + 7].
  u32x4_t qop[G][4];
  SoftmaxState st[G];
  f32x4_t o[G][8];
  int lim_c[G];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int qi = 16 * u + c;
    const uint16_t* qrow =
        reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)(b * T + qi) * a.H + h) * D + sl * 128 + g * 8;
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
      qop[u][s2] = qi < T ? *reinterpret_cast<const u32x4_t*>(qrow + s2 * 32) : u32x4_t{0u, 0u, 0u, 0u};
    st[u] = SoftmaxState{-INFINITY, -INFINITY, 0.f};
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[u][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int64_t own = r.n + (a.causal ? qi : 0);
    lim_c[u] = (int)(own < r.total ? own : r.total);
  }

  // The split's tiles are k = 0 .. ntot - 1: tile first + k nact of the row.
  const int ctx_tiles = (int)((r.total + 31) >> 5);
  int64_t row_tiles = ctx_tiles;
  // GEN: the row's generated keys after its context tiles, their offsets and beam masks in LDS
  const char* kgb = nullptr;
  const char* vgb = nullptr;
  if constexpr (GEN) {
    int ng = 0;
    for (int e = 0; e < T; ++e) ng += s_gl[b * T + e];
    ng = __builtin_amdgcn_readfirstlane(a.glist ? min(a.gcount[b], a.gen_table) : ng);  // a list holds at most the table
    row_tiles += (ng + 31) >> 5;
    kgb = a.kg + h * a.g_head * 2 + sl * 256;
    vgb = a.vg + h * a.g_head * 2 + sl * 256;
    fill_gen_table(a, b, ng, s_gl + b * T, s_tab, s_msk, 64 * NSL, D);
    __syncthreads();
  }
  const int64_t first = sp;
  const int64_t ntot = first < row_tiles ? (row_tiles - first + r.nact - 1) / r.nact : 0;
  // The launcher sends only caches with contiguous key rows (s_pos == D) here.
  const char* kt = reinterpret_cast<const char*>(a.k) + (b * a.s_row + h * a.s_head + first * 32 * D) * 2 + sl * 256;
  const char* vt = reinterpret_cast<const char*>(a.v) + (b * a.s_row + h * a.s_head + first * 32 * D) * 2 + sl * 256;
  const int64_t tile_bytes = (int64_t)r.nact * 32 * D * 2;
  const int64_t last_key = a.cache_len - 1;
  auto load_k = [&](KVTile<128>& t, int64_t k) {
    if constexpr (GEN) {
      const int ti = (int)(first + k * r.nact);
      if (ti >= ctx_tiles) {  // a tile of generated keys (wave-uniform)
        load_tile_rows<128>(t, kgb, vgb, s_tab + (ti - ctx_tiles) * 32, c, g);
        return;
      }
    }
    const int64_t kb = (first + k * r.nact) * 32;
    const int64_t kmax = last_key - kb, vstop = r.total - kb;
    load_tile_clamped<128, D * 2>(t, kt + k * tile_bytes, vt + k * tile_bytes, kmax < 31 ? (int)kmax : 31,
                                  vstop < 32 ? (int)vstop : 32, c, g);
  };
  auto attend_k = [&](const KVTile<128>& t, int64_t k) {
#pragma unroll
    for (int u = 0; u < G; ++u) {
      float sv[8];
      tile_scores<128>(t, qop[u], sv);
      float* mine = &sx[k & 1][sl][u][lane * 8];
      *reinterpret_cast<f32x4_t*>(mine) = f32x4_t{sv[0], sv[1], sv[2], sv[3]};
      *reinterpret_cast<f32x4_t*>(mine + 4) = f32x4_t{sv[4], sv[5], sv[6], sv[7]};
    }
    lds_barrier();
#pragma unroll
    for (int u = 0; u < G; ++u) {
      float tot[8];
#pragma unroll
      for (int ww = 0; ww < NSL; ++ww) {
        const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(&sx[k & 1][ww][u][lane * 8]);
        const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(&sx[k & 1][ww][u][lane * 8 + 4]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          tot[j] = ww == 0 ? lo[j] : tot[j] + lo[j];
          tot[j + 4] = ww == 0 ? hi[j] : tot[j + 4] + hi[j];
        }
      }
      const int ti = (int)(first + k * r.nact);
      if (GEN && ti >= ctx_tiles)  // generated keys: the beams that see each key
        attend_scored<128, true>(t, tot, a.scale_log2, st[u], o[u], g, 0,
                                 u == 0 ? gen_bits(s_msk + (ti - ctx_tiles) * 32 + 8 * g, c) : 0);
      else
        attend_scored<128>(t, tot, a.scale_log2, st[u], o[u], g, ti * 32 + 8 * g, lim_c[u]);
    }
  };
  // The buffer written for tile k was last read for tile k - 2, before every wave passed tile k - 1's barrier.
  if (ntot > 0) {
    KVTile<128> A, B;
    load_k(A, 0);
    int64_t k = 0;
    for (; k + 2 < ntot; k += 2) {
      load_k(B, k + 1);
      attend_k(A, k);
      load_k(A, k + 2);
      attend_k(B, k + 1);
    }
    if (k + 1 < ntot) {
      load_k(B, k + 1);
      attend_k(A, k);
      attend_k(B, k + 1);
    } else {
      attend_k(A, k);
    }
  }

  // ---- finish: per-query sums (the same in every wave), then the output slice or this split's partial slice
  const bool direct = r.nact == 1 && a.gen_split < 0;
  const int64_t base = (slot0 + sp) * T;
#pragma unroll
  for (int u = 0; u < G; ++u) {
    float l_tot = st[u].l_run + __shfl_xor(st[u].l_run, 16, kWave);
    l_tot += __shfl_xor(l_tot, 32, kWave);
    float li[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) li[i] = __shfl(l_tot, 4 * g + i, kWave);
    if (direct) {
      uint16_t* out = reinterpret_cast<uint16_t*>(a.out);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * u + 4 * g + i;
        if (t >= T) continue;
        const float div = li[i] > 0.f ? li[i] : 1.f;
        u32x4_t wv;
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) wv[q2] = pack_bf16x2(o[u][2 * q2][i] / div, o[u][2 * q2 + 1][i] / div);
        *reinterpret_cast<u32x4_t*>(out + ((int64_t)(b * T + t) * a.H + h) * D + sl * 128 + c * 8) = wv;
      }
      continue;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * u + 4 * g + i;
      if (t >= T) continue;
      float* po = a.part_o + (base + t) * D + sl * 128 + c * 8;
      const f32x4_t x0 = f32x4_t{o[u][0][i], o[u][1][i], o[u][2][i], o[u][3][i]};
      const f32x4_t x1 = f32x4_t{o[u][4][i], o[u][5][i], o[u][6][i], o[u][7][i]};
      if (a.separate) {
        reinterpret_cast<f32x4_t*>(po)[0] = x0;
        reinterpret_cast<f32x4_t*>(po)[1] = x1;
      } else {
        const int64_t at = (base + t) * D + sl * 128 + c * 8;
        put_through4(a.part_o, at, x0);
        put_through4(a.part_o, at + 4, x1);
      }
    }
    const int tc = 16 * u + c;
    if (sl == 0 && g == 0 && tc < T) {
      if (a.separate) {
        a.part_ml[(base + tc) * 2] = st[u].m_ref;
        a.part_ml[(base + tc) * 2 + 1] = l_tot;
      } else {
        put_through2(a.part_ml + (base + tc) * 2, st[u].m_ref, l_tot);
      }
    }
  }
  if (direct || a.separate) return;
  // Every wave's partial stores have reached the coherence point before the split's ticket is taken.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  int* counter = &a.counters[b * a.H + h];
  if (threadIdx.x == 0) s_ticket = __hip_atomic_fetch_add(counter, 1, kTicketOrder, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_ticket != r.nact - 1) return;
  // The last split merges; each wave its slice.  Balanced beams: the generated keys' partials follow the heads'
  // workgroup slots, one per (group, head).
  const int64_t gen_slot = a.balanced ? (int64_t)a.H * a.splits + (int64_t)b * a.H + h : -1;
  merge_splits_fast<uint16_t>(a, b, h, r.nact, sl * 128, 128, slot0, gen_slot);
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------- workgroup per row

constexpr int kWgWaves = 8;
constexpr int kWgMaxT = 11;  // the waves' states, the fetched partials and the ranking stay within 64 KB of LDS
constexpr int64_t kWgMinUnits = 128;  // rows x heads from which one workgroup per (head, row) beats split-K

constexpr int kPairMaxRows = 256;
constexpr int64_t kPairMaxGenTable = 4096;  // generated keys of a unit taken as tiles of the halves kernel
constexpr size_t kPairMaxLds = 64 * 1024;   // dynamic LDS of the halves kernel
constexpr int64_t kPairMaxQueryRows = int64_t{1} << 30;  // query rows x heads: 32-bit row indices in the kernel

// The row's tile count: 32-key tiles up to the keys its last query sees.
__device__ __forceinline__ int row_tile_count(const AttnArgs& a, int b) {
  const SplitRange r = split_range(a, b, 0);
  return (int)((r.total + 31) >> 5);
}

// One partial (m, l, O[t][d .. d + 3]) read at the coherence point.
struct PartialItem {
  float m, l;
  f32x4_t o;
};

__device__ __forceinline__ PartialItem get_partial(const AttnArgs& a, int64_t slot_base, int t, int d) {
  const uint64_t ml = __hip_atomic_load(reinterpret_cast<uint64_t*>(a.part_ml + (slot_base * a.T + t) * 2),
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return PartialItem{__uint_as_float((uint32_t)ml), __uint_as_float((uint32_t)(ml >> 32)),
                     get_through4(a.part_o, (slot_base * a.T + t) * a.D + d)};
}

// Up to three partials of one output item merged and written (bf16).
__device__ __forceinline__ void write_merged(const AttnArgs& a, int b, int h, int t, int d, const PartialItem (&p)[3],
                                             int np) {
  float top = -INFINITY;
#pragma unroll
  for (int e = 0; e < 3; ++e) top = e < np ? fmaxf(top, p[e].m) : top;
  float den = 0.f;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 3; ++e) {
    const float wt = e >= np || p[e].m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(p[e].m - top);
    den += wt * (e < np ? p[e].l : 0.f);
    acc += wt * (e < np ? p[e].o : f32x4_t{0.f, 0.f, 0.f, 0.f});
  }
  const float div = den > 0.f ? den : 1.f;
  store4<uint16_t>(reinterpret_cast<uint16_t*>(a.out) + (int64_t)((b * a.T + t) * a.H + h) * a.D + d, acc / div);
}

// The wave's n >= 1 tiles of one sequence: X holds (is loading) tile 0, Y is free.  Tile k + 1 loads while tile k's
// math runs, and during the last tile's math ``ldn`` loads the next sequence's first tile.  Every load is
// unconditional (the loop's own branches only), so each wait is for one tile's loads.  Returns 0 if the next
// sequence's first tile is in X, 1 if in Y.
template <int D, class LD, class AT, class LDN>
__device__ __forceinline__ int run_tiles(KVTile<D>& X, KVTile<D>& Y, int n, LD ld, AT at, LDN ldn) {
  int k = 0;
  for (; k + 2 < n; k += 2) {
    ld(Y, k + 1);
    at(X, k);
    ld(X, k + 2);
    at(Y, k + 1);
  }
  if (k + 1 < n) {
    ld(Y, k + 1);
    at(X, k);
    ldn(X);
    at(Y, k + 1);
    return 0;
  }
  ldn(Y);
  at(X, k);
  return 1;
}

// NS softmax states in LDS (NS x [T][D] O, [T] m, [T] l) merged into this thread's item (t, d) of a partial.
template <int NS>
__device__ __forceinline__ PartialItem merge_slots(const float* po, const float* pm, const float* pl, int T, int D,
                                                   int t, int d) {
  // Every read is issued before the first use, so that their LDS latencies overlap.
  float mv[NS], lv[NS];
  f32x4_t ov[NS];
#pragma unroll
  for (int v = 0; v < NS; ++v) {
    mv[v] = pm[v * T + t];
    lv[v] = pl[v * T + t];
    ov[v] = *reinterpret_cast<const f32x4_t*>(po + (v * T + t) * D + d);
  }
  float top = -INFINITY;
#pragma unroll
  for (int v = 0; v < NS; ++v) top = fmaxf(top, mv[v]);
  float den = 0.f;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int v = 0; v < NS; ++v) {
    const float wt = mv[v] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv[v] - top);
    den += wt * lv[v];
    acc += wt * ov[v];
  }
  return PartialItem{top, den, acc};
}

// Unit tickets of the halves (one int per unit, zero between launches).  The first half's workgroup publishes its
// partial, then adds kTicketFirst.  The second half's workgroup adds kTicketClaim before publishing anything: an
// old value of kTicketFirst means the first half is out and it merges at once from its own registers.  Otherwise it
// publishes its partial and adds kTicketSecond: an old value of kTicketClaim + kTicketFirst means the first half
// came out in between and it merges; an old value of kTicketClaim means the first half's workgroup will find
// kTicketClaim + kTicketSecond and merge.  Exactly one workgroup merges, after the last add, and it resets the
// ticket to zero.
constexpr int kTicketFirst = 1, kTicketClaim = 2, kTicketSecond = 4;

// Dynamic LDS of the halves kernel: the waves' states, the two fetched partials of unit 1, half 1's queries (bf16);
// with generated keys (beams) also every row's generated-key count and the two units' tables of key offsets.
__host__ __device__ constexpr size_t pair_lds_bytes(int T, int D, int rows = 0, int gen_table = 0) {
  return (size_t)(kWgWaves + 2) * T * (D + 2) * sizeof(float) + (size_t)T * D * 2 +
         (((size_t)rows * T + 3) / 4 * 4 + 2 * (size_t)gen_table) * sizeof(int32_t) +
         2 * (size_t)gen_table * sizeof(uint16_t);
}

// One 8-wave workgroup per (head, row) unit, working on halves: units are ranked by length, and workgroup i takes
// the first half of the i-th longest unit ("half 0") and the second half of the i-th shortest ("half 1"), so the
// workgroups (one per CU) stream about the same number of tiles.  That balance is what the HBM needs: a CU reads
// at most ~30 GB/s, so the GPU streams at full rate only while nearly every CU is busy.
//
// The workgroup's tiles (half 0's, then half 1's) are dealt round-robin over its 8 waves in one sequence, and each
// wave's tiles run through both halves in one pipeline (half 1's first tile loads during half 0's last).  At the
// switch the waves' half-0 states merge in LDS and the partial is written through to the coherence point while the
// next tiles load.  The first wave to finish half 1 claims unit 1 (see kTicketFirst) and, if its first half is out,
// fetches it into LDS while the other waves finish, so the common end is an LDS merge and the output store.  The
// dealing is static, so results do not depend on timing.
//
// GEN (beams): each unit's tiles are its context tiles followed by its group's generated keys as one list cut into
// 32-key tiles -- the step's list of distinct (row, position) keys (a.glist), or beam 0's keys, then beam 1's, ... --
// key f at the byte offset the workgroup's table in LDS gives and seen by the beams of its mask, so the halves deal,
// the pipeline and the merges treat the generated keys like any other tile.
template <int D, bool GEN = false>
__global__ __launch_bounds__(64 * kWgWaves, 1) void verify_attn_pair_kernel(AttnArgs a, int rows, int slots) {
  static_assert(D == 128, "the halves kernel serves head dim 128");
  constexpr int KS = D / 32;
  constexpr int kFetched = kWgWaves;  // LDS state slots of the fetched partials: unit 1's first half, its generated keys
  constexpr int kSlots = kWgWaves + 2;
  extern __shared__ float smem[];  // [10][T][D] O, [10][T] m, [10][T] l, then [T][D] bf16 queries
  __shared__ int ntl[kPairMaxRows];
  __shared__ int order[kPairMaxRows];  // rows by tile count, longest first (ties: lower row first)
  __shared__ int s_tk[2];
  __shared__ int s_done;  // waves done with their tiles
  const int tid = threadIdx.x, lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int T = a.T, H = a.H, U = rows * H;
  // GEN: every row's generated-key counts [rows][T], then the two units' offset tables, after half 1's queries
  int* s_gl = reinterpret_cast<int*>(smem + (kWgWaves + 2) * T * (D + 2) + T * D / 2);
  uint32_t* tab = reinterpret_cast<uint32_t*>(s_gl + ((rows * T + 3) & ~3));  // 16-byte aligned (row reads)
  uint16_t* msk = reinterpret_cast<uint16_t*>(tab + 2 * a.gen_table);
  if (tid == 0) s_done = 0;
  for (int b = tid; b < rows; b += 64 * kWgWaves) {
    int nt = row_tile_count(a, b);
    if constexpr (GEN) {
      int ng = 0;
      for (int e = 0; e < T; ++e) {
        const int n = gen_count(a, (int64_t)b * T + e);
        s_gl[b * T + e] = n;
        ng += n;
      }
      nt += ((a.glist ? min(a.gcount[b], a.gen_table) : ng) + 31) >> 5;
    }
    ntl[b] = nt;
  }
  __syncthreads();
  for (int b = tid; b < rows; b += 64 * kWgWaves) {
    const int nb = ntl[b];
    int rank = 0;
    for (int b2 = 0; b2 < rows; ++b2) rank += (ntl[b2] > nb) || (ntl[b2] == nb && b2 < b);
    order[rank] = b;
  }
  __syncthreads();
  const int i = blockIdx.x;
  const int u0 = __builtin_amdgcn_readfirstlane(order[i / H] * H + i % H);
  const int u1 = __builtin_amdgcn_readfirstlane(order[(U - 1 - i) / H] * H + (U - 1 - i) % H);
  const int b0 = u0 / H, h0 = u0 - b0 * H, b1 = u1 / H, h1 = u1 - b1 * H;
  const SplitRange r0 = split_range(a, b0, 0), r1 = split_range(a, b1, 0);
  const int nc0 = (int)((r0.total + 31) >> 5), nc1 = (int)((r1.total + 31) >> 5);  // context tiles
  // GEN: the units' generated keys (wave-uniform)
  auto gen_total = [&](int bu) {
    int n = 0;
    for (int e = 0; e < T; ++e) n += s_gl[bu * T + e];
    return __builtin_amdgcn_readfirstlane(a.glist ? min(a.gcount[bu], a.gen_table) : n);  // at most the table
  };
  const int ng0 = GEN ? gen_total(b0) : 0, ng1 = GEN ? gen_total(b1) : 0;
  const int nt0 = nc0 + ((ng0 + 31) >> 5), nt1 = nc1 + ((ng1 + 31) >> 5);
  const int e0 = (nt0 + 1) >> 1, s1 = (nt1 + 1) >> 1;  // half 0: tiles [0, e0) of u0; half 1: [s1, nt1) of u1
  // Wave w takes half 0's tiles w, w + 8, ...  Half 1's tiles go to waves 0..6 only (the last wave publishes half
  // 0 at the switch), round-robin from wave e0 mod 8 on (the waves without an extra half-0 tile first): wave w < 7
  // takes s1 + j1, s1 + j1 + 7, ..., j1 = (w - start) mod 7.
  constexpr int kHalf1Waves = kWgWaves - 1;
  const int start1 = e0 % kWgWaves < kHalf1Waves ? e0 % kWgWaves : 0;
  const int j1 = ((w - start1) % kHalf1Waves + kHalf1Waves) % kHalf1Waves;
  const int n0 = e0 > w ? (e0 - w + kWgWaves - 1) / kWgWaves : 0;
  const int n1 = w < kHalf1Waves && nt1 - s1 > j1 ? (nt1 - s1 - j1 + kHalf1Waves - 1) / kHalf1Waves : 0;

  float* po = smem;
  float* pm = po + kSlots * T * D;
  float* pl = pm + kSlots * T;
  uint16_t* qs1 = reinterpret_cast<uint16_t*>(pl + kSlots * T);
  const uint16_t* qg = reinterpret_cast<const uint16_t*>(a.q);
  for (int idx = tid; idx < T * (D / 8); idx += 64 * kWgWaves) {
    const int t = idx / (D / 8), d8 = (idx - t * (D / 8)) * 8;
    *reinterpret_cast<u32x4_t*>(qs1 + t * D + d8) =
        *reinterpret_cast<const u32x4_t*>(qg + (int64_t)((b1 * T + t) * H + h1) * D + d8);
  }
  // B operand of S^T = K Q^T for half 0: lane (c, g) holds q[c][32s + 8g .. 32s + 8g + 7].
  u32x4_t qop[KS];
  const u32x4_t zero = {0u, 0u, 0u, 0u};
  {
    const uint16_t* qrow = qg + (int64_t)((b0 * T + c) * H + h0) * D + g * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) qop[s] = c < T ? *reinterpret_cast<const u32x4_t*>(qrow + s * 32) : zero;
  }
  const char* kgb0 = nullptr;
  const char* vgb0 = nullptr;
  const char* kgb1 = nullptr;
  const char* vgb1 = nullptr;
  if constexpr (GEN) {
    kgb0 = a.kg + h0 * a.g_head * 2;
    vgb0 = a.vg + h0 * a.g_head * 2;
    kgb1 = a.kg + h1 * a.g_head * 2;
    vgb1 = a.vg + h1 * a.g_head * 2;
    fill_gen_table(a, b0, ng0, s_gl + b0 * T, tab, msk, 64 * kWgWaves, D);
    fill_gen_table(a, b1, ng1, s_gl + b1 * T, tab + a.gen_table, msk + a.gen_table, 64 * kWgWaves, D);
    __syncthreads();
  }

  const char* kb0 = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(a.k) + b0 * a.s_row + h0 * a.s_head);
  const char* vb0 = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(a.v) + b0 * a.s_row + h0 * a.s_head);
  const char* kb1 = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(a.k) + b1 * a.s_row + h1 * a.s_head);
  const char* vb1 = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(a.v) + b1 * a.s_row + h1 * a.s_head);
  const int64_t last_key = a.cache_len - 1;
  // A tile of a unit's keys (see load_tile_clamped).  The launcher sends only caches with contiguous key rows
  // (s_pos == D) here.
  auto ld_tile = [&](KVTile<D>& t, const char* kb, const char* vb, int tile, int64_t total) {
    const int64_t k0 = (int64_t)tile * 32;
    const int64_t kmax = last_key - k0, vstop = total - k0;
    load_tile_clamped<D>(t, kb + k0 * D * 2, vb + k0 * D * 2, kmax < 31 ? (int)kmax : 31,
                         vstop < 32 ? (int)vstop : 32, c, g);
  };
  // Query c's key limit in the current half (keys fit in 32 bits); half 1's is set at the switch.
  auto key_limit = [&](const SplitRange& r) {
    const int64_t own = r.n + (a.causal ? c : 0);
    return (int)(own < r.total ? own : r.total);
  };
  int lim = key_limit(r0);
  const float c_scale = a.scale_log2;
  SoftmaxState st{-INFINITY, -INFINITY, 0.f};
  f32x4_t o[D / 16];
#pragma unroll
  for (int nb = 0; nb < D / 16; ++nb) o[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // The wave's k-th tile: the unit's base, tile index and key limit are scalar selects, so every load stays
  // unconditional.
  auto tile_of = [&](int k) { return k < n0 ? w + kWgWaves * k : s1 + j1 + kHalf1Waves * (k - n0); };
  auto ld = [&](KVTile<D>& t, int k) {
    const bool first = k < n0;
    const int tile = tile_of(k);
    if constexpr (GEN) {
      const int nc = first ? nc0 : nc1;
      if (tile >= nc) {  // a tile of generated keys (wave-uniform)
        load_tile_rows<D>(t, first ? kgb0 : kgb1, first ? vgb0 : vgb1,
                          tab + (first ? 0 : a.gen_table) + (tile - nc) * 32, c, g);
        return;
      }
    }
    ld_tile(t, first ? kb0 : kb1, first ? vb0 : vb1, tile, first ? r0.total : r1.total);
  };
  auto flush = [&]() {
    float l_tot = st.l_run + __shfl_xor(st.l_run, 16, kWave);
    l_tot += __shfl_xor(l_tot, 32, kWave);
    // The lane's LDS addresses are computed here, not kept in registers through the tile loops.
    int lx = lane;
    asm volatile("" : "+v"(lx));
    const int fc = lx & 15, fg = lx >> 4;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int t = 4 * fg + ii;
      if (t >= T) continue;
      f32x4_t* dst = reinterpret_cast<f32x4_t*>(po + (w * T + t) * D + fc * 8);
      dst[0] = f32x4_t{o[0][ii], o[1][ii], o[2][ii], o[3][ii]};
      dst[1] = f32x4_t{o[4][ii], o[5][ii], o[6][ii], o[7][ii]};
    }
    if (g == 0 && c < T) {
      pm[w * T + c] = st.m_ref;
      pl[w * T + c] = l_tot;
    }
  };
  // Thread tid's item of a merged partial: query item_t, dimensions item_d .. item_d + 3 (T x D / 4 <= 352 items).
  // Computed where used (from an opaque copy of tid), not kept in registers through the tile loops.
  int item_t = 0, item_d = 0;
  bool has_item = false;
  auto set_item = [&]() {
    int tx = tid;
    asm volatile("" : "+v"(tx));
    item_t = tx / (D / 4);
    item_d = (tx - item_t * (D / 4)) * 4;
    has_item = item_t < T;
  };
  // The switch, once per wave after its last half-0 tile (before its first tile if it has none): the waves' half-0
  // states go to LDS; the last wave merges them, writes the partial through, waits for its stores and takes unit
  // 0's first ticket (kept for the end), while the other waves go on with half 1's queries.
  int tk0 = 0;
  auto to_half1 = [&]() {
    flush();
    __syncthreads();
    if (w == kWgWaves - 1) {
      const int64_t sb = (int64_t)u0 * slots;
      for (int idx = lane; idx < T * (D / 4); idx += kWave) {
        const int t = idx / (D / 4), d = (idx - t * (D / 4)) * 4;
        const PartialItem m0 = merge_slots<kWgWaves>(po, pm, pl, T, D, t, d);
        put_through4(a.part_o, (sb * T + t) * D + d, m0.o);
        if (d == 0) put_through2(a.part_ml + (sb * T + t) * 2, m0.m, m0.l);
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      int v = 0;
      if (lane == 0)
        v = __hip_atomic_fetch_add(&a.counters[u0], kTicketFirst, kTicketOrder, __HIP_MEMORY_SCOPE_AGENT);
      tk0 = __builtin_amdgcn_readfirstlane(v);
    }
    st = SoftmaxState{-INFINITY, -INFINITY, 0.f};
#pragma unroll
    for (int nb = 0; nb < D / 16; ++nb) o[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qop[s] = c < T ? *reinterpret_cast<const u32x4_t*>(qs1 + c * D + s * 32 + g * 8) : zero;
    lim = key_limit(r1);
  };
  auto at = [&](const KVTile<D>& t, int k) {
    const int tile = tile_of(k);
    if constexpr (GEN) {
      const bool first = k < n0;
      const int nc = first ? nc0 : nc1;
      const bool gt = tile >= nc;  // generated keys: the beams that see each key; context: the key limit
      // the masks are read on every tile (a clamped index), so that no load waits under a branch
      const int gb = gen_bits(msk + (first ? 0 : a.gen_table) + (gt ? tile - nc : 0) * 32 + 8 * g, c);
      int cb = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) cb |= tile * 32 + 8 * g + j < lim ? 1 << j : 0;
      attend_bits<D>(t, qop, c_scale, st, o, g, gt ? gb : cb);
    } else {
      attend<D>(t, qop, c_scale, st, o, g, tile * 32 + 8 * g, lim);
    }
    if (k == n0 - 1) to_half1();
  };
  if (n0 == 0) to_half1();
  const int n = n0 + n1;
  if (n > 0) {
    KVTile<D> A, B;
    ld(A, 0);
    run_tiles<D>(A, B, n, ld, at, [&](KVTile<D>&) {});
  }

  // ---- the end.  The first of waves 0..6 done claims unit 1 and, when its first half is out, copies it (and the
  // beams' generated-keys partial) into the LDS slots kFetched, kFetched + 1 while the other waves finish.
  const bool gen = a.gen_split >= 0;  // beams: a third partial, written by the previous launch at slot gen_split
  if (w < kHalf1Waves) {
    int first = 0;
    if (lane == 0) first = __hip_atomic_fetch_add(&s_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(first) == 0) {
      int tk = 0;
      if (lane == 0)
        tk = __hip_atomic_fetch_add(&a.counters[u1], kTicketClaim, kTicketOrder, __HIP_MEMORY_SCOPE_AGENT);
      tk = __builtin_amdgcn_readfirstlane(tk);
      if (lane == 0) s_tk[1] = tk;
      if (tk == kTicketFirst) {
        constexpr int kRounds = (kWgMaxT * (D / 4) + kWave - 1) / kWave;
        PartialItem p[kRounds][2];
#pragma unroll
        for (int r = 0; r < kRounds; ++r) {  // every load in flight at once
          const int idx = lane + r * kWave, t = idx / (D / 4), d = (idx - t * (D / 4)) * 4;
          if (t < T) {
            p[r][0] = get_partial(a, (int64_t)u1 * slots, t, d);
            if (gen) p[r][1] = get_partial(a, (int64_t)u1 * slots + a.gen_split, t, d);
          }
        }
#pragma unroll
        for (int r = 0; r < kRounds; ++r) {
          const int idx = lane + r * kWave, t = idx / (D / 4), d = (idx - t * (D / 4)) * 4;
          if (t < T) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              if (e == 1 && !gen) continue;
              const int sl = kFetched + e;
              *reinterpret_cast<f32x4_t*>(po + (sl * T + t) * D + d) = p[r][e].o;
              if (d == 0) {
                pm[sl * T + t] = p[r][e].m;
                pl[sl * T + t] = p[r][e].l;
              }
            }
          }
        }
      }
    }
  }
  __syncthreads();  // the last wave is done with half 0's states; the fetched slots are written
  flush();
  if (w == kWgWaves - 1 && lane == 0) s_tk[0] = tk0;
  __syncthreads();
  const int tk1 = s_tk[1];
  set_item();
  // Every merger of a unit combines (first half, second half, generated keys) in that order with the same
  // arithmetic, so the output does not depend on which workgroup merges.
  if (tk1 == kTicketFirst) {  // unit 1: the fetched first half + the waves' second half (+ generated keys)
    if (has_item) {
      PartialItem p[3];
      p[0] = merge_slots<1>(po + kFetched * T * D, pm + kFetched * T, pl + kFetched * T, T, D, item_t, item_d);
      p[1] = merge_slots<kWgWaves>(po, pm, pl, T, D, item_t, item_d);
      p[2] = p[1];
      if (gen)
        p[2] = merge_slots<1>(po + (kFetched + 1) * T * D, pm + (kFetched + 1) * T, pl + (kFetched + 1) * T, T, D,
                              item_t, item_d);
      write_merged(a, b1, h1, item_t, item_d, p, gen ? 3 : 2);
    }
    if (tid == 0) __hip_atomic_store(&a.counters[u1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {  // half 1 claimed first: publish it, then the second add decides who merges
    PartialItem m1{-INFINITY, 0.f, f32x4_t{0.f, 0.f, 0.f, 0.f}};
    if (has_item) {
      m1 = merge_slots<kWgWaves>(po, pm, pl, T, D, item_t, item_d);
      const int64_t sb = (int64_t)u1 * slots + 1;
      put_through4(a.part_o, (sb * T + item_t) * D + item_d, m1.o);
      if (item_d == 0) put_through2(a.part_ml + (sb * T + item_t) * 2, m1.m, m1.l);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) s_tk[1] = __hip_atomic_fetch_add(&a.counters[u1], kTicketSecond, kTicketOrder,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_tk[1] == kTicketClaim + kTicketFirst) {  // the first half came out in between: merge here
      if (has_item) {
        PartialItem p[3];
        p[0] = get_partial(a, (int64_t)u1 * slots, item_t, item_d);
        p[1] = m1;
        p[2] = m1;
        if (gen) p[2] = get_partial(a, (int64_t)u1 * slots + a.gen_split, item_t, item_d);
        write_merged(a, b1, h1, item_t, item_d, p, gen ? 3 : 2);
      }
      if (tid == 0) __hip_atomic_store(&a.counters[u1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (s_tk[0] == kTicketClaim + kTicketSecond) {  // unit 0: both halves published
    if (has_item) {
      PartialItem p[3];
      p[0] = get_partial(a, (int64_t)u0 * slots, item_t, item_d);
      p[1] = get_partial(a, (int64_t)u0 * slots + 1, item_t, item_d);
      p[2] = p[1];
      if (gen) p[2] = get_partial(a, (int64_t)u0 * slots + a.gen_split, item_t, item_d);
      write_merged(a, b0, h0, item_t, item_d, p, gen ? 3 : 2);
    }
    if (tid == 0) __hip_atomic_store(&a.counters[u0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
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
      const int64_t own = r.n + (a.causal ? t : 0);
      const int64_t lim = own < r.stop ? own : r.stop;
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

  const bool direct = r.nact == 1 && a.gen_split < 0;
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
        put_partial(a.part_o + (base + t) * D + d, acc[t][dd], !a.separate);
      }
    }
    if (!direct && lane == 0) {
      put_partial(a.part_ml + (base + t) * 2, m_run[t], !a.separate);
      put_partial(a.part_ml + (base + t) * 2 + 1, l_tot, !a.separate);
    }
  }
  if (direct) return;
  finish_split<Elem>(a, b, h, r.nact);
}

// ---------------------------------------------------------------------------------------------- combine

// Second launch of the split merge: one wave per (query row t, head, row b), every load issued at once (one
// memory round trip).  Lane s holds split s's (m, l); each lane keeps D/64 output dimensions of every split.

template <typename OutT, int DPL>
__global__ __launch_bounds__(64) void verify_attn_combine_kernel(AttnArgs a) {
  const int t = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const SplitRange r = split_range(a, b, 0);
  const int nact = r.nact;
  if (nact == 1 && a.gen_split < 0) return;  // written directly by its only split
  const int nq = nact + (a.gen_split >= 0 ? 1 : 0);  // partials to merge
  const int lane = threadIdx.x;
  const int T = a.T, D = a.D;
  const int64_t split0 = ((int64_t)b * a.H + h) * a.splits;
  OutT* orow = reinterpret_cast<OutT*>(a.out) + ((int64_t)(b * T + t) * a.H + h) * D;
  if (nq > kWave) {  // more partials than lanes to hold their (m, l): the generic merge
    if (t == 0) merge_splits<OutT>(a, b, h, nact);
    return;
  }
  const bool has_d = lane * DPL < D;
  const int d0 = has_d ? lane * DPL : 0;  // lanes past the head's dimensions read dimension 0 and store nothing
  // The splits' rows in batches of kB, every load of a batch in flight at once (addresses clamped to the last
  // split; the clamped repeats are not added), added in split order.  The first batch is issued before the
  // splits' (m, l), which the weights need, so a merge of up to kB splits is one memory round trip.
  constexpr int kB = 16;  // one batch for up to 16 splits (the default chunk gives at most 10 at 2560 keys)
  float po[kB][DPL];
  auto load_batch = [&](int s0) {
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const int sj = s0 + j < nq ? s0 + j : nq - 1;
      const float* src = a.part_o + ((split0 + merge_slot(a, nact, sj)) * T + t) * D + d0;
      if constexpr (DPL % 4 == 0) {
#pragma unroll
        for (int e4 = 0; e4 < DPL; e4 += 4) {
          const f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(src + e4);
#pragma unroll
          for (int e = 0; e < 4; ++e) po[j][e4 + e] = v4[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < DPL; ++e) po[j][e] = src[e];
      }
    }
  };
  load_batch(0);
  float m = -INFINITY, l = 0.f;
  if (lane < nq) {
    const int64_t ml = ((split0 + merge_slot(a, nact, lane)) * T + t) * 2;
    m = a.part_ml[ml];
    l = a.part_ml[ml + 1];
  }
  const float top = wave_max(m);
  const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - top);
  const float den = wave_sum(w * l);
  const float div = den > 0.f ? den : 1.f;
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
  for (int s0 = 0;; s0 += kB) {
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (s0 + j < nq) {
        const float ws = __shfl(w, s0 + j, kWave);
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[e] += ws * po[j][e];
      }
    }
    if (s0 + kB >= nq) break;
    load_batch(s0 + kB);
  }
  if (!has_d) return;
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const float v = acc[e] / div;
    if constexpr (sizeof(OutT) == 2)
      orow[d0 + e] = (uint16_t)f32_to_bf16_rne(v);
    else
      orow[d0 + e] = v;
  }
}

}  // namespace omni

using namespace omni;

static int attn_splits(int32_t keys, int32_t chunk) { return (int)((keys + chunk - 1) / chunk); }

extern "C" int32_t omni_verify_attention_chunk(int32_t rows, int32_t tokens, int32_t heads,
                                               int32_t head_dim, int32_t keys) {
  (void)tokens;
  if (rows <= 0 || heads <= 0 || keys <= 0) return 64;
  // About 2048 waves (8 per CU) when the rows are full, at most 8 tiles (256 keys) per split: measured on
  // config 3 (8 rows x 32 heads, 750-2400 keys), 224-256 keys per split are among the fastest and longer
  // splits leave too few waves in flight; at least 64 keys so that a split's fixed cost stays small.  Head dims
  // of 256 and more: 256 keys per split (measured at the real checkpoint's 8 slots x 8 heads x 512, T = 5, with the
  // merge launch: 45.6 us against 49.0 us for 128-key splits).
  const int64_t items = (int64_t)rows * heads;
  int64_t chunk = ((int64_t)keys * items + 2047) / 2048;
  chunk = (chunk + 31) / 32 * 32;
  if (head_dim >= 256) chunk = 256;
  if (chunk > 256) chunk = 256;
  if (chunk < 64) chunk = 64;
  return (int32_t)chunk;
}

static size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Partials are addressed with 32-bit byte offsets from the workspace base.
static constexpr size_t kMaxWorkspace = (size_t)1 << 32;

// Partial slots per unit in the workspace: split-K at this chunk, or a unit's two halves.
static size_t attn_slots(int keys, int chunk) {
  const int splits = attn_splits(keys, chunk);
  return (size_t)(splits > 2 ? splits : 2);
}

// Balanced split-K for wide heads (bf16, head dim 256 / 512): workgroups per head.  OMNI_WIDE_WGS in all, one per CU
// (measured at 8 rows x 8 heads x 512, T = 5: 42.1 us against 49.5 us with two per CU and 58.2 us with four), and
// at least one per row.
#ifndef OMNI_WIDE_WGS
#define OMNI_WIDE_WGS 256
#endif
static int balanced_budget(int rows, int heads) {
  const int per_head = OMNI_WIDE_WGS / heads;
  return per_head > rows ? per_head : rows;
}

static bool balanced_shape(int32_t rows, int32_t heads, int32_t head_dim) {
  // rows <= kBalancedMaxRows <= the workgroup's threads (one per row while the deal is computed)
  return (head_dim == 256 || head_dim == 512) && rows <= kBalancedMaxRows && balanced_budget(rows, heads) <= 65535;
}

// The balanced wide-head launch (bf16, head dim 256 / 512, balanced_shape): grid (budget, heads), every key of a row
// in its one range (the deal splits it), the partials merged in the kernel -- with the generated keys' partial when
// a.gen_split >= 0 (beams; see verify_attn_slice_kernel).  a.T > 16 runs two query groups per wave.
static void launch_balanced_wide(AttnArgs& a, int32_t rows, int32_t heads, int32_t head_dim, int32_t keys,
                                 hipStream_t s) {
  a.balanced = 1;
  a.rows = rows;
  a.splits = balanced_budget(rows, heads);
  a.ctx_splits = 1;
  a.chunk = (keys + 31) / 32 * 32;
  a.separate = 0;
  dim3 grid(a.splits, heads, 1);
  if (a.kg) {  // beams with their generated keys as tiles (T <= kWideMaxBeams <= 16: one query group)
    if (head_dim == 256) verify_attn_slice_kernel<256, 1, true><<<grid, 128, 0, s>>>(a);
    else verify_attn_slice_kernel<512, 1, true><<<grid, 256, 0, s>>>(a);
  } else if (head_dim == 256) {
    if (a.T > 16) verify_attn_slice_kernel<256, 2><<<grid, 128, 0, s>>>(a);
    else verify_attn_slice_kernel<256, 1><<<grid, 128, 0, s>>>(a);
  } else {
    if (a.T > 16) verify_attn_slice_kernel<512, 2><<<grid, 256, 0, s>>>(a);
    else verify_attn_slice_kernel<512, 1><<<grid, 256, 0, s>>>(a);
  }
}

// Partial items (T x D floats and their (m, l)) the workspace holds: split-K slots per (row, head) -- a unit's splits
// or its two halves -- or, for the balanced wide-head split-K, the heads' workgroup slots.
static size_t attn_partial_items(int32_t rows, int32_t tokens, int32_t heads, int32_t head_dim, int32_t keys,
                                 int32_t chunk) {
  size_t units = (size_t)rows * heads * attn_slots(keys, chunk) * tokens;
  if (balanced_shape(rows, heads, head_dim)) {
    const size_t wide = (size_t)heads * balanced_budget(rows, heads) * tokens;
    units = units > wide ? units : wide;
  }
  return units;
}

extern "C" size_t omni_verify_attention_workspace(int32_t rows, int32_t tokens, int32_t heads,
                                                  int32_t head_dim, int32_t keys, int32_t chunk) {
  if (rows <= 0 || tokens <= 0 || heads <= 0 || head_dim <= 0 || keys <= 0) return 0;
  if (chunk <= 0) chunk = omni_verify_attention_chunk(rows, tokens, heads, head_dim, keys);
  const size_t units = attn_partial_items(rows, tokens, heads, head_dim, keys, chunk);
  return align256(units * head_dim * sizeof(float)) + align256(units * 2 * sizeof(float));
}

// Key-split kernel and (when asked) the merge launch for filled-in arguments.
static int launch_attention(const AttnArgs& a, int rows, int dtype, hipStream_t s) {
  const bool mfma = dtype == OMNI_BF16 && a.D % 128 == 0 && a.s_pos == a.D;  // contiguous key rows
  dim3 grid(a.ctx_splits, a.H, rows);
  if (mfma) {
    switch (a.D) {
      case 128: verify_attn_mfma_kernel<128><<<grid, 64, 0, s>>>(a); break;
      case 256:
        if (a.T > 16) verify_attn_slice_kernel<256, 2><<<grid, 128, 0, s>>>(a);
        else verify_attn_slice_kernel<256, 1><<<grid, 128, 0, s>>>(a);
        break;
      case 512:
        if (a.T > 16) verify_attn_slice_kernel<512, 2><<<grid, 256, 0, s>>>(a);
        else verify_attn_slice_kernel<512, 1><<<grid, 256, 0, s>>>(a);
        break;
      default: verify_attn_valu_kernel<uint16_t><<<grid, 64, 0, s>>>(a); break;
    }
  } else if (dtype == OMNI_BF16) {
    verify_attn_valu_kernel<uint16_t><<<grid, 64, 0, s>>>(a);
  } else {
    verify_attn_valu_kernel<float><<<grid, 64, 0, s>>>(a);
  }
  return omni_launch_status();
}

static int launch_combine(const AttnArgs& a, int rows, int dtype, hipStream_t s) {
  dim3 cgrid(a.T, a.H, rows);
  const int dpl = (a.D + 63) / 64;  // output dimensions per lane
#define OMNI_COMBINE(T_, DPL_) verify_attn_combine_kernel<T_, DPL_><<<cgrid, 64, 0, s>>>(a)
  if (dtype == OMNI_BF16) {
    if (dpl == 1) OMNI_COMBINE(uint16_t, 1);
    else if (dpl == 2) OMNI_COMBINE(uint16_t, 2);
    else if (dpl <= 4) OMNI_COMBINE(uint16_t, 4);
    else OMNI_COMBINE(uint16_t, 8);
  } else {
    if (dpl == 1) OMNI_COMBINE(float, 1);
    else if (dpl == 2) OMNI_COMBINE(float, 2);
    else if (dpl <= 4) OMNI_COMBINE(float, 4);
    else OMNI_COMBINE(float, 8);
  }
#undef OMNI_COMBINE
  return omni_launch_status();
}

static int check_attention_shape(int32_t tokens, int32_t heads, int32_t head_dim, int32_t dtype, float scale,
                                 int64_t stride_pos) {
  if (heads <= 0 || head_dim <= 0) return OMNI_ERR_INVALID;
  if (!(scale > 0.f)) return OMNI_ERR_INVALID;  // a softmax scale is positive (head_dim^-1/2)
  // Up to 16 queries per row; up to 32 on the wide-head MFMA kernel (two query groups per wave).
  const bool wide = dtype == OMNI_BF16 && (head_dim == 256 || head_dim == 512) && stride_pos == head_dim;
  if (tokens < 1 || tokens > (wide ? 32 : 16)) return OMNI_ERR_SHAPE;
  if (dtype != OMNI_BF16 && dtype != OMNI_F32) return OMNI_ERR_DTYPE;
  if (head_dim % 8 != 0 || head_dim > kValuMaxD) return OMNI_ERR_SHAPE;
  return OMNI_OK;
}

// 128-bit operand loads: q and out, and on the MFMA path every row / head / position start, 16-byte aligned.
static bool attention_aligned(const void* q, const void* out, const void* k, const void* v, int64_t s_row,
                              int64_t s_head, int64_t s_pos, int32_t head_dim, int32_t dtype) {
  if (((uintptr_t)q | (uintptr_t)out) & 15u) return false;
  if (dtype == OMNI_BF16 && head_dim % 128 == 0) {
    if (((uintptr_t)k | (uintptr_t)v) & 15u) return false;
    if ((s_row | s_head | s_pos) % 8 != 0) return false;
  }
  return true;
}

extern "C" int omni_verify_attention(const void* q, const void* k_cache, const void* v_cache,
                                     int64_t stride_row, int64_t stride_head, int64_t stride_pos,
                                     int64_t cache_len, const int64_t* lengths, int32_t rows,
                                     int32_t tokens, int32_t heads, int32_t head_dim, int32_t keys,
                                     int32_t chunk, float scale, void* out, void* workspace,
                                     size_t workspace_bytes, int32_t* counters, int32_t flags,
                                     int32_t dtype, void* stream) {
  if (rows < 0 || keys <= 0 || cache_len <= 0) return OMNI_ERR_INVALID;
  int st = check_attention_shape(tokens, heads, head_dim, dtype, scale, stride_pos);
  if (st != OMNI_OK) return st;
  if (rows == 0) return OMNI_OK;
  if (!q || !k_cache || !v_cache || !lengths || !out || !workspace || !counters) return OMNI_ERR_INVALID;
  if (chunk == 0) chunk = omni_verify_attention_chunk(rows, tokens, heads, head_dim, keys);
  if (chunk <= 0 || chunk % 32 != 0) return OMNI_ERR_INVALID;
  const size_t need = omni_verify_attention_workspace(rows, tokens, heads, head_dim, keys, chunk);
  if (need >= kMaxWorkspace) return OMNI_ERR_SHAPE;  // partial offsets are 32-bit
  if (workspace_bytes < need) return OMNI_ERR_WORKSPACE;
  if (((uintptr_t)workspace & 255u) != 0) return OMNI_ERR_WORKSPACE;
  if (!attention_aligned(q, out, k_cache, v_cache, stride_row, stride_head, stride_pos, head_dim, dtype))
    return OMNI_ERR_INVALID;
  const int splits = attn_splits(keys, chunk);
  const size_t units = attn_partial_items(rows, tokens, heads, head_dim, keys, chunk);
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
  a.causal = 1;
  a.ctx_splits = splits;
  a.gen_split = -1;
  a.balanced = 0;
  a.rows = rows;
  hipStream_t s = (hipStream_t)stream;
  const bool wg = dtype == OMNI_BF16 && head_dim == 128 && stride_pos == head_dim && tokens <= kWgMaxT &&
                  rows <= kPairMaxRows && !(flags & OMNI_ATTN_SPLIT_K) && (int64_t)rows * heads >= kWgMinUnits &&
                  (int64_t)rows * tokens * heads < kPairMaxQueryRows;
  if (wg) {  // one workgroup per (head, row): the whole key range is one split of kWgWaves waves
    a.chunk = (keys + 31) / 32 * 32;
    a.ctx_splits = 1;
    a.splits = 1;
    const int slots = (int)attn_slots(keys, chunk);
    verify_attn_pair_kernel<128><<<rows * heads, 64 * kWgWaves, pair_lds_bytes(tokens, head_dim), s>>>(a, rows,
                                                                                                     slots);
    return omni_launch_status();
  }
  if (dtype == OMNI_BF16 && stride_pos == head_dim && balanced_shape(rows, heads, head_dim) &&
      !(flags & OMNI_ATTN_SPLIT_K)) {
    // wide heads: a fixed budget of workgroups per head dealt to the rows by length, merged in the kernel
    launch_balanced_wide(a, rows, heads, head_dim, keys, s);
    return omni_launch_status();
  }
  st = launch_attention(a, rows, dtype, s);
  if (st != OMNI_OK || !a.separate) return st;
  return launch_combine(a, rows, dtype, s);
}

// ---------------------------------------------------------------------------------------------- static scratch

// The verify attention for callers that cannot allocate: its split partials and merge tickets live in this
// file-scope array, one copy per GPU for the life of the process.  Host code never passes ``scratch`` itself to
// a kernel (on the host the name is a stand-in, not a device address): it passes the device address that
// hipGetSymbolAddress returns for the current device, looked up once per device and kept in g_scratch.
static __device__ __align__(256) unsigned char scratch[OMNI_STATIC_WORKSPACE_BYTES +
                                                       OMNI_STATIC_MAX_UNITS * sizeof(int32_t)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices];

// This device's copy of ``scratch``: looked up by omni_verify_attention_static_init, or by the entry point's first
// call with the device current when that call's stream is not being captured (the lookup may load the code object,
// which a capture must not record).  ``stream`` null: the caller is the init call, nothing is being captured.
int scratch_address(void** ptr, hipStream_t stream, bool check_capture) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return OMNI_ERR_INVALID;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    if (check_capture) {
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      e = hipStreamIsCapturing(stream, &cap);
      if (e != hipSuccess) return (int)e;
      if (cap != hipStreamCaptureStatusNone) return OMNI_ERR_INVALID;  // omni_verify_attention_static_init first
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return OMNI_ERR_INVALID;
    g_scratch[dev] = p;
  }
  *ptr = g_scratch[dev];
  return OMNI_OK;
}

__global__ __launch_bounds__(256) void zero_tickets_kernel(int32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

}  // namespace

extern "C" int omni_verify_attention_static_init(void) {
  void* base = nullptr;
  return scratch_address(&base, nullptr, false);
}

extern "C" int omni_verify_attention_static(const void* q, const void* k_cache, const void* v_cache,
                                            int64_t stride_row, int64_t stride_head, int64_t stride_pos,
                                            int64_t cache_len, const int64_t* lengths, int32_t rows,
                                            int32_t tokens, int32_t heads, int32_t head_dim, int32_t keys,
                                            int32_t chunk, float scale, void* out, int32_t flags, int32_t dtype,
                                            void* stream) {
  // The checks omni_verify_attention makes on its own arguments come first, so that this entry point answers a
  // bad shape with the same status.
  if (rows < 0 || keys <= 0 || cache_len <= 0) return OMNI_ERR_INVALID;
  int st = check_attention_shape(tokens, heads, head_dim, dtype, scale, stride_pos);
  if (st != OMNI_OK) return st;
  if (rows == 0) return OMNI_OK;
  if (chunk == 0) chunk = omni_verify_attention_chunk(rows, tokens, heads, head_dim, keys);
  if (chunk <= 0 || chunk % 32 != 0) return OMNI_ERR_INVALID;
  const size_t need = omni_verify_attention_workspace(rows, tokens, heads, head_dim, keys, chunk);
  const int64_t units = (int64_t)rows * heads;
  if (need > OMNI_STATIC_WORKSPACE_BYTES || units > OMNI_STATIC_MAX_UNITS) return OMNI_ERR_WORKSPACE;
  void* base = nullptr;
  st = scratch_address(&base, (hipStream_t)stream, true);
  if (st != OMNI_OK) return st;
  int32_t* tickets = reinterpret_cast<int32_t*>(static_cast<unsigned char*>(base) + OMNI_STATIC_WORKSPACE_BYTES);
  // The tickets must be zero when the attention starts.  Every call leaves them zero, but the array keeps whatever
  // the last call on this GPU left, so they are cleared here by a kernel (a fill kernel, not hipMemsetAsync, so
  // that a captured graph replays it correctly).
  hipStream_t s = (hipStream_t)stream;
  const int n = (int)units;
  zero_tickets_kernel<<<(n + 255) / 256, 256, 0, s>>>(tickets, n);
  st = omni_launch_status();
  if (st != OMNI_OK) return st;
  return omni_verify_attention(q, k_cache, v_cache, stride_row, stride_head, stride_pos, cache_len, lengths, rows,
                               tokens, heads, head_dim, keys, chunk, scale, out, base, OMNI_STATIC_WORKSPACE_BYTES,
                               tickets, flags, dtype, stream);
}

// ---------------------------------------------------------------------------------------------- beams

namespace omni {

struct BeamGenArgs {
  const void* q;  // [groups * beams, H, D]
  const void* kg;
  const void* vg;
  int64_t s_row, s_head, s_pos, gen_cap, gen_rows;
  const int32_t* ptr;  // [groups * beams, ptr_stride]: row that wrote position j of row r's history
  int64_t ptr_stride;
  const int64_t* gen_len;  // [groups * beams]
  int beams, H, D;
  float scale_log2;
  float* part_o;
  float* part_ml;
  int splits, gen_split;
};

template <typename Elem>
__device__ __forceinline__ void load8(const Elem* p, float (&x)[8]);

template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float (&x)[8]) {
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = bf16x8_elem(v, e);
}

template <>
__device__ __forceinline__ void load8<float>(const float* p, float (&x)[8]) {
  const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(p);
  const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = lo[e];
    x[e + 4] = hi[e];
  }
}

// Row r's generated keys j < gen_len[r], each read from the row that wrote it (ptr[r, j]): one wave per
// (head, row), 64 keys per pass.  Scores: one key per lane, 16-byte loads along its row.  P V: D/8 lanes per
// key (8 dimensions each, 16-byte loads), 64/(D/8) keys at once, summed over the key groups at the end.  The
// result is a partial in the generated-keys slot, merged with the context splits by the merge launch.
// (``_beam_gen``, src/omniasr_trt/kernels.py:115-144.)
template <typename Elem>
__global__ __launch_bounds__(64) void beam_gen_kernel(BeamGenArgs a) {
  __shared__ float qs[kValuMaxD];
  __shared__ float ps[kWave];
  __shared__ int64_t off_sh[kWave];
  __shared__ float red[kWave * 8];  // kpar * D <= 64 * 8
  const int h = blockIdx.x, r = blockIdx.y;
  const int lane = threadIdx.x;
  const int D = a.D;
  const int64_t n = clamp64(a.gen_len[r], 0, a.gen_cap);
  const Elem* qrow = reinterpret_cast<const Elem*>(a.q) + ((int64_t)r * a.H + h) * D;
  for (int d = lane; d < D; d += kWave) qs[d] = load_elem<Elem>(qrow + d) * a.scale_log2;
  __syncthreads();
  const Elem* kb = reinterpret_cast<const Elem*>(a.kg) + h * a.s_head;
  const Elem* vb = reinterpret_cast<const Elem*>(a.vg) + h * a.s_head;
  const int lpk = D / 8;  // lanes per key in P V
  const int kpar = kWave / lpk;
  const int grp = lane / lpk, sub = lane - grp * lpk;
  const bool pv_lane = grp < kpar;
  float m_run = -INFINITY, l_run = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int64_t j0 = 0; j0 < n; j0 += kWave) {
    const int64_t j = j0 + lane;
    const bool valid = j < n;
    int64_t src = valid ? (int64_t)a.ptr[(int64_t)r * a.ptr_stride + j] : 0;
    src = clamp64(src, 0, a.gen_rows - 1);
    const int64_t off = src * a.s_row + (valid ? j : 0) * a.s_pos;
    float sc = 0.f;
    for (int d0 = 0; d0 < D; d0 += 8) {
      float x[8];
      load8<Elem>(kb + off + d0, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) sc = fmaf(qs[d0 + e], x[e], sc);
    }
    sc = valid ? sc : -INFINITY;
    const float m_new = fmaxf(m_run, wave_max(sc));
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // m_new is finite: key j0 is valid
    const float pr = __builtin_amdgcn_exp2f(sc - m_new);
    l_run = l_run * alpha + pr;
    m_run = m_new;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= alpha;
    ps[lane] = pr;
    off_sh[lane] = off;
    __syncthreads();
    const int kend = (int)((n - j0) < kWave ? (n - j0) : kWave);
    if (pv_lane) {
      for (int kk = grp; kk < kend; kk += kpar) {
        float x[8];
        load8<Elem>(vb + off_sh[kk] + sub * 8, x);
        const float p = ps[kk];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(p, x[e], acc[e]);
      }
    }
    __syncthreads();
  }
  const float l_tot = wave_sum(l_run);
  if (pv_lane) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[grp * D + sub * 8 + e] = acc[e];
  }
  __syncthreads();
  const int g = r / a.beams, i = r - g * a.beams;
  const int64_t slot = (((int64_t)g * a.H + h) * a.splits + a.gen_split) * a.beams + i;
  for (int d = lane; d < D; d += kWave) {
    float o = 0.f;
    for (int q = 0; q < kpar; ++q) o += red[q * D + d];
    a.part_o[slot * D + d] = o;
  }
  if (lane == 0) {
    a.part_ml[slot * 2] = m_run;
    a.part_ml[slot * 2 + 1] = l_tot;
  }
}

// The same for bf16 rows of 128 dimensions, both products' loads in one round trip per 64 keys once the pointers are
// in, K and V read as whole rows by 16 lanes each (4 rows per load instruction): lane (grp, sub) holds dimensions
// 8 sub .. 8 sub + 7 of keys grp + 4 ii; its partial dot products are summed over the group's 16 lanes, so every lane
// of a group holds its 16 keys' scores.  (One lane per key reading its whole K row was 2 us slower at config 5b:
// 64 rows per load instruction.)
__global__ __launch_bounds__(64) void beam_gen_kernel_d128(BeamGenArgs a) {
  constexpr int D = 128, kRow = D / 8;  // 16 lanes read a row
  const int h = blockIdx.x, r = blockIdx.y;
  const int lane = threadIdx.x, grp = lane / kRow, sub = lane - grp * kRow;
  // The first 64 keys' row pointers load beside the length (the index is clamped into the row's capacity, so the
  // load is in bounds whatever the length): one memory round trip less before the K / V loads.
  const int32_t ptr0 = a.ptr[(int64_t)r * a.ptr_stride + (lane < a.gen_cap ? lane : a.gen_cap - 1)];
  const int64_t n = clamp64(a.gen_len[r], 0, a.gen_cap);
  float qv[8];
  {
    const u32x4_t q4 =
        *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)r * a.H + h) * D + sub * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[e] = bf16x8_elem(q4, e) * a.scale_log2;
  }
  const char* kb = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(a.kg) + h * a.s_head);
  const char* vb = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(a.vg) + h * a.s_head);
  float m_run = -INFINITY, l_run = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int64_t j0 = 0; j0 < n; j0 += kWave) {
    const int64_t j = j0 + lane;
    const bool valid = j < n;
    int64_t src = valid ? (j0 == 0 ? (int64_t)ptr0 : (int64_t)a.ptr[(int64_t)r * a.ptr_stride + j]) : 0;
    src = clamp64(src, 0, a.gen_rows - 1);
    const int64_t off = (src * a.s_row + (valid ? j : 0) * a.s_pos) * 2;  // bytes; invalid lanes read key 0
    u32x4_t kx[kWave / 4], vx[kWave / 4];
#pragma unroll
    for (int ii = 0; ii < kWave / 4; ++ii) {
      const int sl = grp + 4 * ii;
      const int64_t o2 = (int64_t)(((uint64_t)__shfl((uint32_t)(off >> 32), sl, kWave) << 32) |
                                   __shfl((uint32_t)off, sl, kWave));
      kx[ii] = *reinterpret_cast<const u32x4_t*>(kb + o2 + sub * 16);
      vx[ii] = *reinterpret_cast<const u32x4_t*>(vb + o2 + sub * 16);
    }
    const int kend = (int)((n - j0) < kWave ? (n - j0) : kWave);
    float sc[kWave / 4];
    float mx = -INFINITY;
#pragma unroll
    for (int ii = 0; ii < kWave / 4; ++ii) {
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) part = fmaf(qv[e], bf16x8_elem(kx[ii], e), part);
#pragma unroll
      for (int o = 1; o < kRow; o <<= 1) part += __shfl_xor(part, o, kWave);
      sc[ii] = grp + 4 * ii < kend ? part : -INFINITY;
      mx = fmaxf(mx, sc[ii]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(m_run, mx);  // finite: key j0 is valid
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
    for (int ii = 0; ii < kWave / 4; ++ii) {
      const float p = __builtin_amdgcn_exp2f(sc[ii] - m_new);  // 0 for the keys past the end
      psum += p;
      const bool kv = grp + 4 * ii < kend;  // rows past the keys in use never reach the product (stale memory)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = kv ? fmaf(p, bf16x8_elem(vx[ii], e), acc[e]) : acc[e];
    }
    psum += __shfl_xor(psum, 16, kWave);
    psum += __shfl_xor(psum, 32, kWave);
    l_run = l_run * alpha + psum;
    m_run = m_new;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc[e] += __shfl_xor(acc[e], 16, kWave);
    acc[e] += __shfl_xor(acc[e], 32, kWave);
  }
  const int g = r / a.beams, i = r - g * a.beams;
  const int64_t slot = (((int64_t)g * a.H + h) * a.splits + a.gen_split) * a.beams + i;
  if (grp == 0) {
    *reinterpret_cast<f32x4_t*>(a.part_o + slot * D + sub * 8) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4_t*>(a.part_o + slot * D + sub * 8 + 4) = f32x4_t{acc[4], acc[5], acc[6], acc[7]};
  }
  if (lane == 0) {
    a.part_ml[slot * 2] = m_run;
    a.part_ml[slot * 2 + 1] = l_run;
  }
}

// Generated keys at head dim 512 (bf16, key rows contiguous): a workgroup of 4 waves per (beam row, head), wave w
// taking keys j0 + 16 w .. j0 + 16 w + 15 of every 64.  Each load instruction reads one whole 1 KB K (or V) row,
// lane l holding dimensions 8 l .. 8 l + 7, so a wave's 16 keys are one memory round trip once the pointers are in;
// the partial dot products are summed over the wave, and the 4 waves' (O, m, l) merge in LDS in wave order.
__global__ __launch_bounds__(256) void beam_gen_kernel_d512(BeamGenArgs a) {
  constexpr int D = 512, KW = 16, NW = 4;
  __shared__ float s_o[NW][D];
  __shared__ float s_m[NW], s_l[NW];
  const int h = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x, w = tid / kWave, lane = tid - w * kWave;
  // This wave's first 16 keys' row pointers load beside the length (index clamped into the row's capacity).
  const int jf = KW * w + (lane & (KW - 1));
  const int32_t ptr0 = a.ptr[(int64_t)r * a.ptr_stride + (jf < a.gen_cap ? jf : a.gen_cap - 1)];
  const int64_t n = clamp64(a.gen_len[r], 0, a.gen_cap);
  float qv[8];
  {
    const u32x4_t q4 =
        *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(a.q) + ((int64_t)r * a.H + h) * D + lane * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[e] = bf16x8_elem(q4, e) * a.scale_log2;
  }
  const char* kb = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(a.kg) + h * a.s_head);
  const char* vb = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(a.vg) + h * a.s_head);
  float m_run = -INFINITY, l_run = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int64_t j0 = 0; j0 < n; j0 += NW * KW) {
    const int64_t jb = j0 + KW * w;  // this wave's first key
    const int64_t j = jb + (lane & (KW - 1));
    const bool valid = j < n;
    int64_t src = valid ? (j0 == 0 ? (int64_t)ptr0 : (int64_t)a.ptr[(int64_t)r * a.ptr_stride + j]) : 0;
    src = clamp64(src, 0, a.gen_rows - 1);
    const int64_t off = (src * a.s_row + (valid ? j : 0) * a.s_pos) * 2;  // bytes; invalid keys read key 0
    u32x4_t kx[KW], vx[KW];
#pragma unroll
    for (int ii = 0; ii < KW; ++ii) {
      const int64_t o2 = (int64_t)(((uint64_t)__shfl((uint32_t)(off >> 32), ii, kWave) << 32) |
                                   __shfl((uint32_t)off, ii, kWave));
      kx[ii] = *reinterpret_cast<const u32x4_t*>(kb + o2 + lane * 16);
      vx[ii] = *reinterpret_cast<const u32x4_t*>(vb + o2 + lane * 16);
    }
    const int64_t left = n - jb;
    const int kend = (int)(left < 0 ? 0 : (left < KW ? left : KW));  // this wave's keys in use (wave-uniform)
    float sc[KW];
    float mx = -INFINITY;
#pragma unroll
    for (int ii = 0; ii < KW; ++ii) {
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) part = fmaf(qv[e], bf16x8_elem(kx[ii], e), part);
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) part += __shfl_xor(part, o, kWave);
      sc[ii] = ii < kend ? part : -INFINITY;
      mx = fmaxf(mx, sc[ii]);
    }
    if (kend > 0) {
      const float m_new = fmaxf(m_run, mx);  // finite: key jb is in use
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      float psum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
      for (int ii = 0; ii < KW; ++ii) {
        const float p = __builtin_amdgcn_exp2f(sc[ii] - m_new);  // 0 for the keys past the end
        psum += p;
        const bool kv = ii < kend;  // rows past the keys in use never reach the product (stale memory)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = kv ? fmaf(p, bf16x8_elem(vx[ii], e), acc[e]) : acc[e];
      }
      l_run = l_run * alpha + psum;
      m_run = m_new;
    }
  }
  *reinterpret_cast<f32x4_t*>(&s_o[w][lane * 8]) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
  *reinterpret_cast<f32x4_t*>(&s_o[w][lane * 8 + 4]) = f32x4_t{acc[4], acc[5], acc[6], acc[7]};
  if (lane == 0) {
    s_m[w] = m_run;
    s_l[w] = l_run;
  }
  __syncthreads();
  if (w != 0) return;
  float top = s_m[0];
#pragma unroll
  for (int q = 1; q < NW; ++q) top = fmaxf(top, s_m[q]);
  float wt[NW], l_tot = 0.f;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    wt[q] = s_m[q] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[q] - top);
    l_tot += wt[q] * s_l[q];
  }
  const int g = r / a.beams, i = r - g * a.beams;
  const int64_t slot = (((int64_t)g * a.H + h) * a.splits + a.gen_split) * a.beams + i;
#pragma unroll
  for (int e4 = 0; e4 < 8; e4 += 4) {
    f32x4_t o4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NW; ++q) o4 += wt[q] * *reinterpret_cast<const f32x4_t*>(&s_o[q][lane * 8 + e4]);
    *reinterpret_cast<f32x4_t*>(a.part_o + slot * D + lane * 8 + e4) = o4;
  }
  if (lane == 0) {
    a.part_ml[slot * 2] = top;
    a.part_ml[slot * 2 + 1] = l_tot;
  }
}

}  // namespace omni

extern "C" size_t omni_beam_attention_workspace(int32_t groups, int32_t beams, int32_t heads, int32_t head_dim,
                                                int32_t ctx_keys, int32_t chunk) {
  if (groups <= 0 || beams <= 0 || heads <= 0 || head_dim <= 0 || ctx_keys <= 0) return 0;
  if (chunk <= 0) chunk = omni_verify_attention_chunk(groups, beams, heads, head_dim, ctx_keys);
  size_t splits = (size_t)attn_splits(ctx_keys, chunk) + 1;
  if (splits < 3) splits = 3;  // or the two context halves and the generated keys
  size_t units = (size_t)groups * heads * splits * beams;
  if (balanced_shape(groups, heads, head_dim)) {  // the heads' workgroup slots, then one generated-keys slot per unit
    const size_t wide = ((size_t)heads * balanced_budget(groups, heads) + (size_t)groups * heads) * beams;
    units = units > wide ? units : wide;
  }
  return align256(units * head_dim * sizeof(float)) + align256(units * 2 * sizeof(float));
}

extern "C" int omni_beam_gen_list(int32_t groups, int32_t beams, const int32_t* ptr, int64_t ptr_stride,
                                  const int64_t* gen_len, int64_t gen_cap, int64_t gen_rows, int64_t gen_row,
                                  int64_t gen_pos, uint32_t* list, uint16_t* mask, int32_t* count, int64_t list_stride,
                                  void* stream) {
  if (groups < 0 || beams < 1 || beams > kWideMaxBeams || gen_cap <= 0 || gen_rows <= 0) return OMNI_ERR_INVALID;
  if (groups == 0) return OMNI_OK;
  if (!ptr || !gen_len || !list || !mask || !count || ptr_stride < gen_cap || list_stride < beams * gen_cap)
    return OMNI_ERR_INVALID;
  if (gen_row < 0 || gen_pos < 0 || ((gen_rows - 1) * gen_row + (gen_cap - 1) * gen_pos) * 2 > (int64_t)UINT32_MAX)
    return OMNI_ERR_SHAPE;  // byte offsets of 32 bits
  GenListArgs a;
  a.ptr = ptr;
  a.ptr_stride = ptr_stride;
  a.gen_len = gen_len;
  a.gen_cap = gen_cap;
  a.gen_rows = gen_rows;
  a.g_row = gen_row;
  a.g_pos = gen_pos;
  a.beams = beams;
  a.list = list;
  a.mask = mask;
  a.count = count;
  a.stride = list_stride;
  beam_gen_list_kernel<<<groups, 256, 0, (hipStream_t)stream>>>(a);
  return omni_launch_status();
}

static int beam_attention(const void* q, const void* k_ctx, const void* v_ctx, int64_t ctx_row, int64_t ctx_head,
                          int64_t ctx_pos, int64_t ctx_cap, const int64_t* ctx_len, const void* k_gen,
                          const void* v_gen, int64_t gen_row, int64_t gen_head, int64_t gen_pos, int64_t gen_cap,
                          int64_t gen_rows, const int32_t* ptr, int64_t ptr_stride, const int64_t* gen_len,
                          const uint32_t* gen_list, const uint16_t* gen_mask, const int32_t* gen_count,
                          int64_t list_stride, int32_t groups, int32_t beams, int32_t heads, int32_t head_dim,
                          int32_t ctx_keys, int32_t chunk, float scale, void* out, void* workspace,
                          size_t workspace_bytes, int32_t* counters, int32_t dtype, void* stream) {
  if (groups < 0 || ctx_keys <= 0 || ctx_cap <= 0 || gen_cap <= 0 || gen_rows <= 0) return OMNI_ERR_INVALID;
  const bool listed = gen_list != nullptr;
  if (listed && (!gen_mask || !gen_count || list_stride < (int64_t)beams * gen_cap)) return OMNI_ERR_INVALID;
  int st = check_attention_shape(beams, heads, head_dim, dtype, scale, 0);  // beams: 1..16
  if (st != OMNI_OK) return st;
  if (groups == 0) return OMNI_OK;
  if (!q || !k_ctx || !v_ctx || !ctx_len || !k_gen || !v_gen || !ptr || !gen_len || !out || !workspace)
    return OMNI_ERR_INVALID;
  if (ptr_stride < gen_cap) return OMNI_ERR_INVALID;
  // The generated-keys kernel reads 8 elements (16 or 32 bytes) at a time along every row.
  if ((((uintptr_t)k_gen | (uintptr_t)v_gen) & 15u) || (gen_row | gen_head | gen_pos) % 8 != 0)
    return OMNI_ERR_INVALID;
  if (chunk == 0) chunk = omni_verify_attention_chunk(groups, beams, heads, head_dim, ctx_keys);
  if (chunk <= 0 || chunk % 32 != 0) return OMNI_ERR_INVALID;
  const size_t need = omni_beam_attention_workspace(groups, beams, heads, head_dim, ctx_keys, chunk);
  if (need >= kMaxWorkspace) return OMNI_ERR_SHAPE;  // partial offsets are 32-bit
  if (workspace_bytes < need) return OMNI_ERR_WORKSPACE;
  if (((uintptr_t)workspace & 255u) != 0) return OMNI_ERR_WORKSPACE;
  if (!attention_aligned(q, out, k_ctx, v_ctx, ctx_row, ctx_head, ctx_pos, head_dim, dtype)) return OMNI_ERR_INVALID;
  const int ctx_splits = attn_splits(ctx_keys, chunk);
  const int splits = ctx_splits + 1 > 3 ? ctx_splits + 1 : 3;  // partial slots per unit (see the workspace)
  size_t units = (size_t)groups * heads * splits * beams;
  if (balanced_shape(groups, heads, head_dim)) {  // the workspace's layout (see omni_beam_attention_workspace)
    const size_t wide = ((size_t)heads * balanced_budget(groups, heads) + (size_t)groups * heads) * beams;
    units = units > wide ? units : wide;
  }
  AttnArgs a;
  a.q = q;
  a.k = k_ctx;
  a.v = v_ctx;
  a.s_row = ctx_row;
  a.s_head = ctx_head;
  a.s_pos = ctx_pos;
  a.cache_len = ctx_cap;
  a.lengths = ctx_len;
  a.T = beams;  // a group's beams are its queries, all over the same context keys
  a.H = heads;
  a.D = head_dim;
  a.chunk = chunk;
  a.splits = splits;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.part_o = (float*)workspace;
  a.part_ml = (float*)((char*)workspace + align256(units * head_dim * sizeof(float)));
  a.counters = nullptr;
  a.out = out;
  a.separate = 1;
  a.causal = 0;
  a.ctx_splits = ctx_splits;
  a.gen_split = ctx_splits;
  a.balanced = 0;
  a.rows = groups;
  hipStream_t s = (hipStream_t)stream;
  const bool halves = dtype == OMNI_BF16 && head_dim == 128 && ctx_pos == head_dim && beams <= kWgMaxT &&
                      groups <= kPairMaxRows && counters != nullptr && (int64_t)groups * heads >= kWgMinUnits &&
                      (int64_t)groups * beams * heads < kPairMaxQueryRows;
  const bool balanced = !halves && dtype == OMNI_BF16 && ctx_pos == head_dim && counters != nullptr &&
                        balanced_shape(groups, heads, head_dim);
  int gen_splits = splits, gen_slot = ctx_splits;  // where the generated keys' kernel writes: unit slot gen_slot
  // The generated keys as tiles of the context launch (halves or balanced wide heads): key rows of D elements, byte
  // offsets from a head's base within 32 bits, a unit's table of offsets (table entries) within the kernel's LDS.
  const int64_t table = ((int64_t)beams * gen_cap + 31) / 32 * 32;
  const bool gen_tiles = gen_pos == head_dim && ((gen_rows - 1) * gen_row + gen_cap * gen_pos) * 2 <= (int64_t)UINT32_MAX;
  auto take_gen = [&]() {
    a.gen_split = -1;
    a.kg = (const char*)k_gen;
    a.vg = (const char*)v_gen;
    a.g_row = gen_row;
    a.g_head = gen_head;
    a.ptr = ptr;
    a.ptr_stride = ptr_stride;
    a.gen_len = gen_len;
    a.gen_cap = (int)gen_cap;
    a.gen_rows = (int)gen_rows;
    a.gen_table = (int)table;
    if (listed) {  // each group's keys once per distinct (row, position): at most beams x gen_cap of them
      a.glist = gen_list;
      a.gmask = gen_mask;
      a.gcount = gen_count;
      a.glist_stride = list_stride;
    }
  };
  if (halves) {  // the generated keys' partial first, then the context halves, whose last merge includes it
    a.chunk = (ctx_keys + 31) / 32 * 32;
    a.ctx_splits = 1;
    a.gen_split = 2;
    a.splits = splits;  // >= 3 slots per unit (see omni_beam_attention_workspace)
    a.counters = counters;
    gen_slot = 2;
    if (gen_tiles && table <= kPairMaxGenTable && pair_lds_bytes(beams, head_dim, groups, (int)table) <= kPairMaxLds) {
      take_gen();
      verify_attn_pair_kernel<128, true><<<groups * heads, 64 * kWgWaves,
                                           pair_lds_bytes(beams, head_dim, groups, (int)table), s>>>(a, groups,
                                                                                                     a.splits);
      return omni_launch_status();
    }
  } else if (balanced) {  // the same order: the generated keys first, then the balanced context launch merging it
    a.counters = counters;
    if (gen_tiles && table <= kWideMaxGenTable && beams <= kWideMaxBeams) {
      take_gen();
      launch_balanced_wide(a, groups, heads, head_dim, ctx_keys, s);
      return omni_launch_status();
    }
    a.gen_split = 0;  // present; its slot is given by the kernel's balanced layout
    gen_splits = 1;
    gen_slot = heads * balanced_budget(groups, heads);  // slot heads x budget + (group x heads + head)
  } else {
    st = launch_attention(a, groups, dtype, s);
    if (st != OMNI_OK) return st;
  }
  BeamGenArgs gargs;
  gargs.q = q;
  gargs.kg = k_gen;
  gargs.vg = v_gen;
  gargs.s_row = gen_row;
  gargs.s_head = gen_head;
  gargs.s_pos = gen_pos;
  gargs.gen_cap = gen_cap;
  gargs.gen_rows = gen_rows;
  gargs.ptr = ptr;
  gargs.ptr_stride = ptr_stride;
  gargs.gen_len = gen_len;
  gargs.beams = beams;
  gargs.H = heads;
  gargs.D = head_dim;
  gargs.scale_log2 = a.scale_log2;
  gargs.part_o = a.part_o;
  gargs.part_ml = a.part_ml;
  dim3 ggrid(heads, groups * beams);
  gargs.splits = gen_splits;
  gargs.gen_split = gen_slot;
  if (dtype == OMNI_BF16 && head_dim == 128 && gen_pos == head_dim) beam_gen_kernel_d128<<<ggrid, 64, 0, s>>>(gargs);
  else if (dtype == OMNI_BF16 && head_dim == 512 && gen_pos == head_dim) beam_gen_kernel_d512<<<ggrid, 256, 0, s>>>(gargs);
  else if (dtype == OMNI_BF16) beam_gen_kernel<uint16_t><<<ggrid, 64, 0, s>>>(gargs);
  else beam_gen_kernel<float><<<ggrid, 64, 0, s>>>(gargs);
  st = omni_launch_status();
  if (st != OMNI_OK) return st;
  if (halves) {
    verify_attn_pair_kernel<128><<<groups * heads, 64 * kWgWaves, pair_lds_bytes(beams, head_dim), s>>>(a, groups,
                                                                                                         a.splits);
    return omni_launch_status();
  }
  if (balanced) {
    launch_balanced_wide(a, groups, heads, head_dim, ctx_keys, s);
    return omni_launch_status();
  }
  return launch_combine(a, groups, dtype, s);
}

extern "C" int omni_beam_attention(const void* q, const void* k_ctx, const void* v_ctx, int64_t ctx_row,
                                   int64_t ctx_head, int64_t ctx_pos, int64_t ctx_cap, const int64_t* ctx_len,
                                   const void* k_gen, const void* v_gen, int64_t gen_row, int64_t gen_head,
                                   int64_t gen_pos, int64_t gen_cap, int64_t gen_rows, const int32_t* ptr,
                                   int64_t ptr_stride, const int64_t* gen_len, int32_t groups, int32_t beams,
                                   int32_t heads, int32_t head_dim, int32_t ctx_keys, int32_t chunk, float scale,
                                   void* out, void* workspace, size_t workspace_bytes, int32_t* counters,
                                   int32_t dtype, void* stream) {
  return beam_attention(q, k_ctx, v_ctx, ctx_row, ctx_head, ctx_pos, ctx_cap, ctx_len, k_gen, v_gen, gen_row, gen_head,
                        gen_pos, gen_cap, gen_rows, ptr, ptr_stride, gen_len, nullptr, nullptr, nullptr, 0, groups,
                        beams, heads, head_dim, ctx_keys, chunk, scale, out, workspace, workspace_bytes, counters, dtype,
                        stream);
}

extern "C" int omni_beam_attention_listed(const void* q, const void* k_ctx, const void* v_ctx, int64_t ctx_row,
                                          int64_t ctx_head, int64_t ctx_pos, int64_t ctx_cap, const int64_t* ctx_len,
                                          const void* k_gen, const void* v_gen, int64_t gen_row, int64_t gen_head,
                                          int64_t gen_pos, int64_t gen_cap, int64_t gen_rows, const int32_t* ptr,
                                          int64_t ptr_stride, const int64_t* gen_len, const uint32_t* gen_list,
                                          const uint16_t* gen_mask, const int32_t* gen_count, int64_t list_stride,
                                          int32_t groups, int32_t beams, int32_t heads, int32_t head_dim,
                                          int32_t ctx_keys, int32_t chunk, float scale, void* out, void* workspace,
                                          size_t workspace_bytes, int32_t* counters, int32_t dtype, void* stream) {
  if (!gen_list) return OMNI_ERR_INVALID;
  return beam_attention(q, k_ctx, v_ctx, ctx_row, ctx_head, ctx_pos, ctx_cap, ctx_len, k_gen, v_gen, gen_row, gen_head,
                        gen_pos, gen_cap, gen_rows, ptr, ptr_stride, gen_len, gen_list, gen_mask, gen_count,
                        list_stride, groups, beams, heads, head_dim, ctx_keys, chunk, scale, out, workspace,
                        workspace_bytes, counters, dtype, stream);
}
