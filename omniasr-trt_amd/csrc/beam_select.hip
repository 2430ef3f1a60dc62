// The beam search step's choice, for gfx950: each group's N best offers over its N rows x V tokens, from the LM
// head's log-probabilities or logits (src/omniasr_trt/beam.py:165-175):
//   logp  = the input itself (OMNI_SELECT_LOGP: torch's own F.log_softmax output, so the choice is the reference's
//           bit for bit), or (OMNI_SELECT_LOGITS) log_softmax(logits) per row computed here in the model's dtype
//           (bf16): fp32 max, fp32 sum of exp(x - max) in this kernel's own order, logsum = log(sum),
//           logp = bf16((x - max) - logsum) -- the arithmetic of torch's kernel but not its summation order, so a
//           logp on a bf16 rounding boundary can round the other way;
//   offer = score + logp, or with length_norm, once the group's row 0 has tokens, (score * count + logp) / (count + 1),
//           each operation rounded to fp32 in that order (torch's element-wise kernels, no fused multiply-add);
//           a finished row offers -inf everywhere except EOS, at its frozen score;
//   best, flat = offers.view(S, N * V).topk(N), sorted best first: ties in value go to the lower flat index
//           (torch.topk leaves the order of equal values unspecified).
//
// Layout: one 256-thread workgroup per row (the log-softmax needs the whole row; a row is ~20 KB, so one workgroup
// per row spreads the group's reads over N CUs): the row's max and sum are two workgroup reductions in a fixed order;
// each offer and its flat index become one 64-bit key ordered as the choice is, so each wave takes its N best in N
// rounds of a branch-free scan and a wave-wide maximum, and wave 0 merges the waves' lists into the row's N best.
// The row writes them through to the device's coherence point (the rows of a group run on different XCDs, whose L2s
// are not coherent) and takes the group's ticket; the last row of the group reads the N rows' lists and merges them
// into the group's N best.  Every selection is by (value, index), so the result does not depend on which row
// finishes last.
#include <limits.h>
#include <math.h>

#include "common.h"

namespace omni {

constexpr int kSelThreads = 256;
constexpr int kSelWaves = kSelThreads / kWave;
constexpr int kSelMaxBeams = 16;

// An offer and its flat index as one 64-bit key whose unsigned order is the choice's order: the value's bits mapped
// to an order-preserving unsigned integer (negative values bit-inverted, positive ones with the sign bit set; -0 as
// +0, so equal values stay equal) above the index inverted (a lower index is the larger key).  Keys are unique, and 0
// is below every offer's key.
__device__ __forceinline__ uint64_t sel_key(float v, int i) {
  uint32_t b = v == 0.f ? 0u : __float_as_uint(v);
  const uint32_t u = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
}
__device__ __forceinline__ float sel_value(uint64_t k) {
  const uint32_t u = (uint32_t)(k >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
__device__ __forceinline__ int64_t sel_index(uint64_t k) { return (int64_t)(0xffffffffu - (uint32_t)k); }

__device__ __forceinline__ uint64_t sel_wave_max(uint64_t k) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)k, o, kWave), hi = __shfl_xor((uint32_t)(k >> 32), o, kWave);
    const uint64_t ok = ((uint64_t)hi << 32) | lo;
    k = ok > k ? ok : k;
  }
  return k;
}

// The wave's n largest of its lanes' E keys each, in order: lane j < n gets the j-th (0 past the keys there are).
template <int E>
__device__ __forceinline__ uint64_t sel_wave_top(const uint64_t (&keys)[E], int n) {
  uint64_t prev = ~0ull, mine = 0;
  for (int j = 0; j < n; ++j) {
    uint64_t best = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) best = keys[e] < prev && keys[e] > best ? keys[e] : best;
    best = sel_wave_max(best);
    if (lane_id() == j) mine = best;
    prev = best;
  }
  return mine;
}

__device__ __forceinline__ float sel_block_reduce(float v, float* red, bool is_max) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(v, o, kWave);
    v = is_max ? fmaxf(v, ov) : v + ov;
  }
  if (lane_id() == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < kSelWaves; ++w) t = is_max ? fmaxf(t, red[w]) : t + red[w];  // the same order in every thread
  __syncthreads();
  return t;
}

struct SelectArgs {
  const uint16_t* logits;
  int64_t logits_stride;
  int beams, vocab;
  const float* score;
  const int64_t* count;
  const uint8_t* ended;
  int length_norm;
  int64_t eos;
  float* best;
  int64_t* flat;
  uint64_t* cand;  // [rows][beams] keys of each row's best, written through
  int* tickets;    // [groups], zero before and after
  int logp_in;     // 1: the input rows are log-probabilities already (no log-softmax here)
};

// CPT: 8-logit chunks per thread (V <= 8 x 256 x CPT).
template <int CPT>
__global__ __launch_bounds__(kSelThreads) void beam_select_kernel(SelectArgs a) {
#pragma clang fp contract(off)
  __shared__ float red[kSelWaves];
  __shared__ uint64_t wk[kSelWaves][kSelMaxBeams];
  const int row = blockIdx.x, n = a.beams, V = a.vocab;
  const int g = row / n, b = row - g * n;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const uint16_t* lr = a.logits + (int64_t)row * a.logits_stride;
  u32x4_t x[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ci = tid + c * kSelThreads;
    x[c] = ci * 8 < V ? *reinterpret_cast<const u32x4_t*>(lr + ci * 8) : u32x4_t{0u, 0u, 0u, 0u};
  }
  const float score = a.score[row];
  const int64_t cnt = a.count[row];
  const bool ended = a.ended[row] != 0;
  const bool norm = a.length_norm && a.count[(int64_t)g * n] > 0;

  float m = 0.f, logsum = 0.f;
  if (!a.logp_in) {  // block-uniform
    m = -INFINITY;
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      if ((tid + c * kSelThreads) * 8 < V) {
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, bf16x8_elem(x[c], e));
      }
    m = sel_block_reduce(m, red, true);
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < CPT; ++c)
      if ((tid + c * kSelThreads) * 8 < V) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += expf(bf16x8_elem(x[c], e) - m);
      }
    sum = sel_block_reduce(sum, red, false);
    logsum = logf(sum);
  }

  // The row's offers as keys with their flat indices in the group's N x V (past V: key 0, never chosen).
  uint64_t keys[CPT * 8];
  const float cf = (float)cnt, c1 = (float)(cnt + 1);
#pragma unroll
  for (int c = 0; c < CPT; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int v = (tid + c * kSelThreads) * 8 + e;
      const float lp = a.logp_in ? bf16x8_elem(x[c], e) : round_through_bf16((bf16x8_elem(x[c], e) - m) - logsum);
      float o;
      if (norm) {
        const float t = score * cf;
        o = (t + lp) / c1;
      } else {
        o = score + lp;
      }
      if (ended) o = v == a.eos ? score : -INFINITY;
      keys[c * 8 + e] = v < V ? sel_key(o, b * V + v) : 0ull;
    }

  // Each wave's N best, then wave 0 merges the waves' lists into the row's.
  const uint64_t mine = sel_wave_top<CPT * 8>(keys, n);
  if (lane < n) wk[wave][lane] = mine;
  __syncthreads();
  if (wave != 0) return;
  uint64_t mk[1];
  {
    const int w = lane / kSelMaxBeams, j = lane - w * kSelMaxBeams;  // kSelWaves x kSelMaxBeams = 64 lanes
    mk[0] = j < n ? wk[w][j] : 0ull;
  }
  const uint64_t rowk = sel_wave_top<1>(mk, n);

  // The row's list, written through; then the group's ticket.
  uint64_t* crow = a.cand + (int64_t)row * n;
  if (lane < n) __hip_atomic_store(crow + lane, rowk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  int ticket = 0;
  if (lane == 0) ticket = __hip_atomic_fetch_add(a.tickets + g, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ticket = __shfl(ticket, 0, kWave);
  if (ticket != n - 1) return;

  // The group's last row: the N lists (N x N <= 256 keys, read at the coherence point), merged.
  const uint64_t* cg = a.cand + (int64_t)g * n * n;
  uint64_t gk[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int f = lane + q * kWave;
    const bool have = f < n * n;
    const uint64_t k = __hip_atomic_load(cg + (have ? f : 0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    gk[q] = have ? k : 0ull;
  }
  const uint64_t gkey = sel_wave_top<4>(gk, n);
  if (lane < n) {
    a.best[(int64_t)g * n + lane] = sel_value(gkey);
    a.flat[(int64_t)g * n + lane] = sel_index(gkey);
  }
  if (lane == 0) __hip_atomic_store(a.tickets + g, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace omni

extern "C" size_t omni_beam_select_workspace(int32_t groups, int32_t beams) {
  if (groups <= 0 || beams <= 0) return 0;
  return (size_t)groups * beams * beams * sizeof(uint64_t);
}

extern "C" int omni_beam_select(const void* logits, int64_t logits_stride, int32_t groups, int32_t beams,
                                int32_t vocab, const float* score, const int64_t* count, const uint8_t* ended,
                                int32_t length_norm, int64_t eos, float* best, int64_t* flat, void* workspace,
                                size_t workspace_bytes, int32_t* tickets, int32_t input_kind, int32_t dtype,
                                void* stream) {
  if (dtype != OMNI_BF16) return OMNI_ERR_DTYPE;
  if (input_kind != OMNI_SELECT_LOGP && input_kind != OMNI_SELECT_LOGITS) return OMNI_ERR_INVALID;
  if (groups < 0 || beams < 1 || beams > omni::kSelMaxBeams || vocab < beams) return OMNI_ERR_INVALID;
  if (vocab % 8 != 0 || vocab > 8 * omni::kSelThreads * 8) return OMNI_ERR_SHAPE;
  if (groups == 0) return OMNI_OK;
  if ((int64_t)beams * vocab >= INT_MAX) return OMNI_ERR_SHAPE;
  if (!logits || !score || !count || !ended || !best || !flat || !tickets || logits_stride < vocab ||
      logits_stride % 8)
    return OMNI_ERR_INVALID;
  if (!workspace || workspace_bytes < omni_beam_select_workspace(groups, beams)) return OMNI_ERR_WORKSPACE;
  omni::SelectArgs a{static_cast<const uint16_t*>(logits), logits_stride, beams, vocab, score, count, ended,
                     length_norm, eos, best, flat, static_cast<uint64_t*>(workspace), tickets,
                     input_kind == OMNI_SELECT_LOGP ? 1 : 0};
  const int rows = groups * beams, cpt = (vocab / 8 + omni::kSelThreads - 1) / omni::kSelThreads;
  hipStream_t s = (hipStream_t)stream;
  if (cpt <= 2)
    omni::beam_select_kernel<2><<<rows, omni::kSelThreads, 0, s>>>(a);
  else if (cpt <= 4)
    omni::beam_select_kernel<4><<<rows, omni::kSelThreads, 0, s>>>(a);
  else if (cpt <= 6)
    omni::beam_select_kernel<6><<<rows, omni::kSelThreads, 0, s>>>(a);
  else
    omni::beam_select_kernel<8><<<rows, omni::kSelThreads, 0, s>>>(a);
  return omni_launch_status();
}
