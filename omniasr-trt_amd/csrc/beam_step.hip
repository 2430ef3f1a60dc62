// The beam search step's bookkeeping around the layers, for gfx950: what a step does before its layers (each row's
// input position, generated-cache position and key counts, and the row's own pointer at the position it writes) and
// after the per-group top-N of the offers (each row takes over its parent's history, pointers, score, token count and
// finished flag, extended by the chosen token; then the groups' step counters and finished flags).
//
// Rules (src/omniasr_trt/beam.py:127-187, the step and the parent reorder):
//   before   live_r = !group_done[g]; k_r = k_step[g]; pos_r = ctx[g] + k_r - 1; gen_pos_r = max(k_r - 1, 0);
//            gen_len_r = live_r ? k_r : 0; ctx_len[g] = group_done[g] ? 0 : ctx[g];
//            live_r: ptr[r][gen_pos_r] = r (the row reads the key it writes in this step);
//   after    parent_r = live_r ? g*N + flat[g][i] / V : r;  chosen_r = live_r ? flat[g][i] % V : tok[r];
//            chosen_r = ended[parent_r] ? EOS : chosen_r;  row r's ptr and hist rows := parent_r's;
//            live_r: hist[r][k_r] = chosen_r;  extends_r = live_r && !ended[parent_r];
//            score_r = extends_r ? best[g][i] : score[parent_r];
//            count_r = count[parent_r] + (extends_r && chosen_r != PAD && chosen_r != EOS);
//            ended_r = live_r ? chosen_r == EOS : ended[parent_r];  tok_r = chosen_r;
//            k_step[g] += !group_done[g];
//            group_done[g] |= all(ended of its rows) || ctx[g] + k_step[g] - 2 >= limit.
// Every value is copied or compared, never computed in floating point, so the results are the torch ops' bit for bit.
//
// Layout: the before-step is one thread per row.  The after-step is one 256-thread workgroup per group: the first N
// threads work out the rows' parents and new state from the old one (held in LDS until every thread has read it),
// then each thread moves whole columns of the group's ptr / hist rows -- it reads a column of all N old rows before
// it writes the column of the new ones, so the in-place reorder needs no second buffer.
#include "common.h"

namespace omni {

constexpr int kBeamMax = 16;  // beams per group

__global__ __launch_bounds__(256) void beam_prepare_kernel(int groups, int beams, const int64_t* ctx,
                                                           const int64_t* k_step, const uint8_t* gdone, int32_t* ptr,
                                                           int64_t ptr_stride, int64_t ptr_cols, int64_t* pos,
                                                           int64_t* gen_pos, int64_t* ctx_len, int64_t* gen_len) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= groups * beams) return;
  const int g = r / beams;
  const bool done = gdone[g] != 0;
  const int64_t k = k_step[g], c = ctx[g];
  const int64_t gp = k - 1 > 0 ? k - 1 : 0;
  pos[r] = c + k - 1;
  gen_pos[r] = gp;
  gen_len[r] = done ? 0 : k;
  if (r == g * beams) ctx_len[g] = done ? 0 : c;
  if (!done && gp < ptr_cols) ptr[(int64_t)r * ptr_stride + gp] = r;
}

// Row i of a group's n rows (row stride ``stride``, ``cols`` columns) becomes old row par[i]; column ``at`` of row i
// takes put[i] instead (at < 0: none).  Thread tid moves columns tid, tid + blockDim.x, ...: it reads a column of all
// n old rows before it writes that column of the new ones, so the reorder is in place.  The old column is picked by
// selects (a register array indexed by a run-time value would live in scratch memory).
__device__ __forceinline__ void move_columns(int32_t* rows, int64_t stride, int64_t cols, int n, const int* par,
                                             int64_t at, const int64_t* put) {
  int pr[kBeamMax];
#pragma unroll
  for (int i = 0; i < kBeamMax; ++i) pr[i] = i < n ? par[i] : 0;
  for (int64_t col = threadIdx.x; col < cols; col += blockDim.x) {
    int32_t old[kBeamMax];
#pragma unroll
    for (int i = 0; i < kBeamMax; ++i) old[i] = i < n ? rows[i * stride + col] : 0;
#pragma unroll
    for (int i = 0; i < kBeamMax; ++i) {
      if (i >= n) break;
      int32_t v = old[0];
#pragma unroll
      for (int j = 1; j < kBeamMax; ++j) v = pr[i] == j ? old[j] : v;
      rows[i * stride + col] = col == at ? (int32_t)put[i] : v;
    }
  }
}

// Score values are moved, never computed: ScoreBits is the score's width (fp32 or fp64) as an integer.
template <typename ScoreBits>
__global__ __launch_bounds__(256) void beam_take_over_kernel(int beams, int64_t vocab, const ScoreBits* best,
                                                             const int64_t* flat, int32_t* ptr, int64_t ptr_stride,
                                                             int64_t ptr_cols, int32_t* hist, int64_t hist_stride,
                                                             int64_t hist_cols, uint8_t* ended, ScoreBits* score,
                                                             int64_t* count, int64_t* tok, int64_t* k_step,
                                                             uint8_t* gdone, const int64_t* ctx, int64_t limit,
                                                             int32_t eos, int32_t pad) {
  __shared__ int par[kBeamMax];       // parent of row i, as a row of the group
  __shared__ int64_t chosen[kBeamMax];
  __shared__ int new_ended[kBeamMax];
  const int g = blockIdx.x, tid = threadIdx.x, n = beams;
  const int64_t r0 = (int64_t)g * n;
  const bool live = gdone[g] == 0;
  const int64_t k = k_step[g];  // the step's position in the rows' histories (before the counter moves)
  ScoreBits new_score = 0;
  int64_t new_count = 0;
  if (tid < n) {
    const int64_t fl = flat[r0 + tid];
    // topk's index into the group's N x V offers (clamped into the group: an index past it reads no other group)
    const int64_t fp = fl / vocab;
    const int p = live ? (int)(fp < 0 ? 0 : fp >= n ? n - 1 : fp) : tid;
    int64_t ch = live ? fl % vocab : tok[r0 + tid];
    const bool was_ended = ended[r0 + p] != 0;
    if (was_ended) ch = eos;
    const bool extends = live && !was_ended;
    new_score = extends ? best[r0 + tid] : score[r0 + p];
    new_count = count[r0 + p] + ((extends && ch != pad && ch != eos) ? 1 : 0);
    new_ended[tid] = live ? (ch == eos) : was_ended;
    par[tid] = p;
    chosen[tid] = ch;
  }
  __syncthreads();  // every old value of the group's rows has been read
  if (tid < n) {
    ended[r0 + tid] = (uint8_t)new_ended[tid];
    score[r0 + tid] = new_score;
    count[r0 + tid] = new_count;
    tok[r0 + tid] = chosen[tid];
  }
  // The rows' ptr and hist rows: thread tid moves columns tid, tid + 256, ... of all of them.  The old column is
  // picked by selects (a register array indexed by a run-time value would live in scratch memory).
  move_columns(ptr + r0 * ptr_stride, ptr_stride, ptr_cols, n, par, -1, chosen);  // no column replaced
  move_columns(hist + r0 * hist_stride, hist_stride, hist_cols, n, par, live ? k : -1, chosen);
  if (tid == 0) {
    const int64_t k_new = k + (live ? 1 : 0);
    k_step[g] = k_new;
    bool all_ended = true;
    for (int i = 0; i < n; ++i) all_ended &= new_ended[i] != 0;
    gdone[g] = (uint8_t)(!live || all_ended || ctx[g] + k_new - 2 >= limit);
  }
}

}  // namespace omni

extern "C" int omni_beam_prepare(int32_t groups, int32_t beams, const int64_t* ctx, const int64_t* k_step,
                                 const uint8_t* group_done, int32_t* ptr, int64_t ptr_stride, int64_t ptr_cols,
                                 int64_t* pos, int64_t* gen_pos, int64_t* ctx_len, int64_t* gen_len, void* stream) {
  if (groups < 0 || beams < 1 || beams > omni::kBeamMax || ptr_cols < 0 || ptr_stride < ptr_cols)
    return OMNI_ERR_INVALID;
  if (groups == 0) return OMNI_OK;
  if (!ctx || !k_step || !group_done || !ptr || !pos || !gen_pos || !ctx_len || !gen_len) return OMNI_ERR_INVALID;
  const int rows = groups * beams;
  omni::beam_prepare_kernel<<<(rows + 255) / 256, 256, 0, (hipStream_t)stream>>>(
      groups, beams, ctx, k_step, group_done, ptr, ptr_stride, ptr_cols, pos, gen_pos, ctx_len, gen_len);
  return omni_launch_status();
}

extern "C" int omni_beam_take_over(int32_t groups, int32_t beams, int64_t vocab, const void* best,
                                   const int64_t* flat, int32_t* ptr, int64_t ptr_stride, int64_t ptr_cols,
                                   int32_t* hist, int64_t hist_stride, int64_t hist_cols, uint8_t* ended,
                                   void* score, int32_t score_bytes, int64_t* count, int64_t* tok, int64_t* k_step,
                                   uint8_t* group_done, const int64_t* ctx, int64_t limit, int32_t eos, int32_t pad,
                                   void* stream) {
  if (groups < 0 || beams < 1 || beams > omni::kBeamMax || vocab < 1 || ptr_cols < 0 || ptr_stride < ptr_cols ||
      hist_cols < 0 || hist_stride < hist_cols)
    return OMNI_ERR_INVALID;
  if (score_bytes != 4 && score_bytes != 8) return OMNI_ERR_DTYPE;
  if (groups == 0) return OMNI_OK;
  if (!best || !flat || !ptr || !hist || !ended || !score || !count || !tok || !k_step || !group_done || !ctx)
    return OMNI_ERR_INVALID;
  hipStream_t s = (hipStream_t)stream;
  if (score_bytes == 4)
    omni::beam_take_over_kernel<uint32_t><<<groups, 256, 0, s>>>(
        beams, vocab, (const uint32_t*)best, flat, ptr, ptr_stride, ptr_cols, hist, hist_stride, hist_cols, ended,
        (uint32_t*)score, count, tok, k_step, group_done, ctx, limit, eos, pad);
  else
    omni::beam_take_over_kernel<uint64_t><<<groups, 256, 0, s>>>(
        beams, vocab, (const uint64_t*)best, flat, ptr, ptr_stride, ptr_cols, hist, hist_stride, hist_cols, ended,
        (uint64_t*)score, count, tok, k_step, group_done, ctx, limit, eos, pad);
  return omni_launch_status();
}
