// Draft proposal (n-gram match against the draft and against the row's own tokens) for gfx950.
//
// Rules of ``_propose`` (src/omniasr_trt/kernels.py:214-268), the search of ``SpecDecoder``
// (src/omniasr_trt/spec.py:11-18, 35-40):
//   history   h_t = out[last - t] for t < ngram, valid while last - t >= first;
//   anchors   i < anchor_width: off = i - behind, anchor = next - 1 + off, live while off <= ahead
//             and anchor < draft_len; score = number of leading t with anchor - t >= 0, h_t valid
//             and draft[anchor - t] == h_t;
//   need      reach (distance, tokens) pairs in increasing distance, else ngram;
//   rank      score >= need and off <= ahead ? score*256 - |off| : -1; best = first maximum;
//   own       i < self_width: back = last - 1 - i, live while back >= first, same leading count
//             against out; j = last - 1 - (first maximum), period = max(last - j, 1);
//   choose    use_draft = mine < self_min or mine <= drafted;
//   propose   q < k: use_draft ? (start + q < draft_len ? draft[start + q] : 0)
//                              : out[j + 1 + q % period].
// Optionally also the drafted step's inputs (src/omniasr_trt/spec.py:85-95), see omni_spec_prepare.
//
// Layout: one 256-thread workgroup per row; thread i scores anchor i and own position i (and
// i + 256k beyond that), the newest tokens sit in LDS, and the two first-maximum searches are one
// 64-bit max each (rank in the high word, the complemented index in the low word) over wave
// shuffles and LDS.  About 4 KB of int32 history per row: latency-bound.
#include <limits.h>

#include "common.h"

namespace omni {

struct ProposeArgs {
  const int32_t* out;
  int64_t out_stride, out_cap;
  const int32_t* draft;
  int64_t draft_stride, draft_cap;
  const int64_t* draft_len;
  const int64_t* last;
  const int64_t* first;
  const int64_t* next;
  int64_t* prop;  // [rows, k] or NULL
  uint8_t* use_draft;
  int64_t* start;
  int k, ngram, behind, ahead, anchor_width, self_width, self_min;
  int reach[8];
  // step assembly (NULL tokens: none)
  const int64_t* tok;
  const uint8_t* done;
  int64_t capacity;
  int64_t* tokens;
  int64_t* pos;
  int64_t* slots;
  int64_t* lengths;
};

constexpr int kProposeThreads = 256;
constexpr int kProposeMaxWidth = 4096;

// Highest rank first, then the lowest index.
__device__ __forceinline__ long long rank_key(int rank, int i) {
  return ((long long)rank << 32) | (long long)(0xffffffffu - (uint32_t)i);
}
__device__ __forceinline__ int key_index(long long key) {
  return (int)(0xffffffffu - (uint32_t)(key & 0xffffffffll));
}
__device__ __forceinline__ int key_rank(long long key) { return (int)(key >> 32); }

__device__ long long block_max_i64(long long v, long long* red) {
  v = wave_max_i64(v);
  const int wave = threadIdx.x / kWave;
  if (lane_id() == 0) red[wave] = v;
  __syncthreads();
  long long r = red[0];
  for (int w = 1; w < kProposeThreads / kWave; ++w) r = red[w] > r ? red[w] : r;
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kProposeThreads) void propose_kernel(ProposeArgs a) {
  __shared__ int32_t hist[64];
  __shared__ uint8_t hvalid[64];
  __shared__ uint8_t score_sh[kProposeMaxWidth];
  __shared__ long long red[kProposeThreads / kWave];
  __shared__ int64_t bc[4];  // start, j, period, use_draft
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t lst = a.last[b], fst = a.first[b], nx = a.next[b], dl = a.draft_len[b];
  const int32_t* orow = a.out + (int64_t)b * a.out_stride;
  const int32_t* drow = a.draft + (int64_t)b * a.draft_stride;

  if (tid < a.ngram) {
    const int64_t hp = lst - tid;
    const bool hv = hp >= fst;
    hvalid[tid] = hv;
    hist[tid] = (hv && hp >= 0 && hp < a.out_cap) ? orow[hp] : -1;
  }
  __syncthreads();

  // ---- draft anchors
  long long best = LLONG_MIN;
  for (int i = tid; i < a.anchor_width; i += kProposeThreads) {
    const int off = i - a.behind;
    const int64_t anchor = nx - 1 + off;
    bool alive = off <= a.ahead && anchor < dl;
    int score = 0;
    for (int t = 0; t < a.ngram; ++t) {
      const int64_t at = anchor - t;
      alive = alive && at >= 0 && hvalid[t];
      if (alive) alive = (at < a.draft_cap ? drow[at] : -2) == hist[t];
      score += alive;
    }
    const int dist = off < 0 ? -off : off;
    int need = a.ngram;
    if (dist <= a.reach[6]) need = a.reach[7];
    if (dist <= a.reach[4]) need = a.reach[5];
    if (dist <= a.reach[2]) need = a.reach[3];
    if (dist <= a.reach[0]) need = a.reach[1];
    const int rank = (score >= need && off <= a.ahead) ? score * 256 - dist : -1;
    score_sh[i] = (uint8_t)score;
    const long long key = rank_key(rank, i);
    best = key > best ? key : best;
  }
  // ---- own earlier positions
  long long sbest = LLONG_MIN;
  for (int i = tid; i < a.self_width; i += kProposeThreads) {
    const int64_t back = lst - 1 - i;
    bool alive = back >= fst;
    int score = 0;
    for (int t = 0; t < a.ngram; ++t) {
      const int64_t at = back - t;
      alive = alive && at >= 0 && hvalid[t];
      if (alive) alive = (at < a.out_cap ? orow[at] : -2) == hist[t];
      score += alive;
    }
    const long long key = rank_key(score, i);
    sbest = key > sbest ? key : sbest;
  }
  best = block_max_i64(best, red);
  sbest = block_max_i64(sbest, red);

  if (tid == 0) {
    const int bi = key_index(best);
    const bool found = key_rank(best) >= 0;
    const int drafted = found ? score_sh[bi] : 0;
    const int64_t st = found ? nx + bi - a.behind : nx;
    const int mine = key_rank(sbest);
    const int64_t j = lst - 1 - key_index(sbest);
    const int64_t period = (lst - j) > 1 ? (lst - j) : 1;
    const bool ud = mine < a.self_min || mine <= drafted;
    bc[0] = st;
    bc[1] = j;
    bc[2] = period;
    bc[3] = ud;
    a.use_draft[b] = ud ? 1 : 0;
    a.start[b] = st;
  }
  __syncthreads();
  const int64_t st = bc[0], j = bc[1], period = bc[2];
  const bool ud = bc[3] != 0;
  const int width = a.k + 1;
  if (tid < a.k) {
    int64_t v;
    if (ud) {
      const int64_t at = st + tid;
      v = (at >= 0 && at < dl && at < a.draft_cap) ? drow[at] : 0;
    } else {
      const int64_t at = j + 1 + tid % period;
      v = (at >= 0 && at < a.out_cap) ? orow[at] : 0;
    }
    if (a.prop) a.prop[(int64_t)b * a.k + tid] = v;
    if (a.tokens) a.tokens[(int64_t)b * width + 1 + tid] = v;
  }
  if (a.tokens && tid < width) {
    const bool running = !a.done[b];
    const int64_t p = lst + (running ? 1 : 0);
    int64_t ps = running ? p + tid : lst;
    ps = ps < a.capacity - 1 ? ps : a.capacity - 1;
    a.pos[(int64_t)b * width + tid] = ps;
    a.slots[(int64_t)b * width + tid] = b;
    if (tid == 0) {
      a.tokens[(int64_t)b * width] = a.tok[b];
      a.lengths[b] = running ? p + 1 : 0;
    }
  }
}

}  // namespace omni

using namespace omni;

static int propose_check(const int32_t* out, int64_t out_stride, int64_t out_cap, const int32_t* draft,
                         int64_t draft_stride, int64_t draft_cap, const int64_t* draft_len,
                         const int64_t* last, const int64_t* first, const int64_t* next,
                         const uint8_t* use_draft, const int64_t* start, int32_t rows, int32_t k,
                         int32_t ngram, int32_t behind, int32_t ahead, int32_t anchor_width,
                         int32_t self_width, int32_t self_min, const int32_t* reach) {
  if (rows < 0) return OMNI_ERR_INVALID;
  if (rows == 0) return 0;
  if (!out || !draft || !draft_len || !last || !first || !next || !use_draft || !start || !reach)
    return OMNI_ERR_INVALID;
  if (out_cap <= 0 || out_stride < out_cap || draft_cap < 0 || draft_stride < draft_cap) return OMNI_ERR_INVALID;
  if (k < 1 || k > 64 || ngram < 1 || ngram > 64) return OMNI_ERR_SHAPE;
  if (anchor_width < 1 || anchor_width > kProposeMaxWidth || self_width < 1 || self_width > kProposeMaxWidth)
    return OMNI_ERR_SHAPE;
  if (behind < 0 || ahead < 0 || self_min < 0) return OMNI_ERR_INVALID;
  return 1;
}

static ProposeArgs make_propose_args(const int32_t* out, int64_t out_stride, int64_t out_cap,
                                     const int32_t* draft, int64_t draft_stride, int64_t draft_cap,
                                     const int64_t* draft_len, const int64_t* last, const int64_t* first,
                                     const int64_t* next, int64_t* prop, uint8_t* use_draft, int64_t* start,
                                     int32_t k, int32_t ngram, int32_t behind, int32_t ahead,
                                     int32_t anchor_width, int32_t self_width, int32_t self_min,
                                     const int32_t* reach) {
  ProposeArgs a = {};
  a.out = out;
  a.out_stride = out_stride;
  a.out_cap = out_cap;
  a.draft = draft;
  a.draft_stride = draft_stride;
  a.draft_cap = draft_cap;
  a.draft_len = draft_len;
  a.last = last;
  a.first = first;
  a.next = next;
  a.prop = prop;
  a.use_draft = use_draft;
  a.start = start;
  a.k = k;
  a.ngram = ngram;
  a.behind = behind;
  a.ahead = ahead;
  a.anchor_width = anchor_width;
  a.self_width = self_width;
  a.self_min = self_min;
  for (int i = 0; i < 8; ++i) a.reach[i] = reach[i];
  return a;
}

extern "C" int omni_propose(const int32_t* out, int64_t out_stride, int64_t out_cap, const int32_t* draft,
                            int64_t draft_stride, int64_t draft_cap, const int64_t* draft_len,
                            const int64_t* last, const int64_t* first, const int64_t* next, int64_t* prop,
                            uint8_t* use_draft, int64_t* start, int32_t rows, int32_t k, int32_t ngram,
                            int32_t behind, int32_t ahead, int32_t anchor_width, int32_t self_width,
                            int32_t self_min, const int32_t reach[8], void* stream) {
  int st = propose_check(out, out_stride, out_cap, draft, draft_stride, draft_cap, draft_len, last, first,
                         next, use_draft, start, rows, k, ngram, behind, ahead, anchor_width, self_width,
                         self_min, reach);
  if (st <= 0) return st;
  if (!prop) return OMNI_ERR_INVALID;
  ProposeArgs a = make_propose_args(out, out_stride, out_cap, draft, draft_stride, draft_cap, draft_len, last,
                                    first, next, prop, use_draft, start, k, ngram, behind, ahead, anchor_width,
                                    self_width, self_min, reach);
  propose_kernel<<<rows, kProposeThreads, 0, (hipStream_t)stream>>>(a);
  return omni_launch_status();
}

extern "C" int omni_spec_prepare(const int32_t* out, int64_t out_stride, int64_t out_cap,
                                 const int32_t* draft, int64_t draft_stride, int64_t draft_cap,
                                 const int64_t* draft_len, const int64_t* last, const int64_t* first,
                                 const int64_t* next, int64_t* prop, uint8_t* use_draft, int64_t* start,
                                 int32_t rows, int32_t k, int32_t ngram, int32_t behind, int32_t ahead,
                                 int32_t anchor_width, int32_t self_width, int32_t self_min,
                                 const int32_t reach[8], const int64_t* tok, const uint8_t* done,
                                 int64_t capacity, int64_t* tokens, int64_t* pos, int64_t* slots,
                                 int64_t* lengths, void* stream) {
  int st = propose_check(out, out_stride, out_cap, draft, draft_stride, draft_cap, draft_len, last, first,
                         next, use_draft, start, rows, k, ngram, behind, ahead, anchor_width, self_width,
                         self_min, reach);
  if (st <= 0) return st;
  if (!tok || !done || !tokens || !pos || !slots || !lengths || capacity <= 0) return OMNI_ERR_INVALID;
  ProposeArgs a = make_propose_args(out, out_stride, out_cap, draft, draft_stride, draft_cap, draft_len, last,
                                    first, next, prop, use_draft, start, k, ngram, behind, ahead, anchor_width,
                                    self_width, self_min, reach);
  a.tok = tok;
  a.done = done;
  a.capacity = capacity;
  a.tokens = tokens;
  a.pos = pos;
  a.slots = slots;
  a.lengths = lengths;
  propose_kernel<<<rows, kProposeThreads, 0, (hipStream_t)stream>>>(a);
  return omni_launch_status();
}
