// The decode loop's per-step bookkeeping on the device.
//
// One step of the reference's one-forward tree loop (src/pe/serve.py:289-343)
// ends with host work: the accepted path's K/V kept (gather_cache), its fused
// features appended (torch.cat), the tokens emitted, the root logit row and
// the pending bonus re-rooted, or on a miss a one-token forward of the pending
// bonus. Here the loop's state lives in device memory so a recorded step
// (a HIP graph) needs no host value:
//
//   state[0] = P, the tokens cached and featurised;  state[1] = the pending
//   bonus (emitted, not yet cached); ids[0 .. P] the context tokens, ids[P]
//   the pending one; feats[0 .. P) their fused feature rows; root the logit
//   row that predicted ids[P].
//
// pe_loop_commit consumes a walk's result [n, bonus, path...]: rows P + i of
// feats and ids take the accepted nodes' features and tokens, root takes the
// last accepted node's logit row, the new bonus becomes pending at ids[P + n]
// and P advances by n. n == 0 leaves the state as it is (the caller runs the
// miss pass: one node, the pending token at position P, whose logits go to
// root), and pe_loop_miss_commit then appends that pass's feature row, takes
// the argmax of its logit row from the lm_head's argmax keys as the new
// pending bonus and advances P by one.
//
// Both write a small record for the host's one read per step: rec[0] = n,
// rec[1] = the bonus, rec[2] |= every status word handed in (cleared after),
// rec[3] = the miss pass's bonus, rec[4 + i] = the accepted tokens.

#include "pe_common.h"

namespace {

__device__ __forceinline__ void copy_row(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, int64_t bytes) {
  if ((((uintptr_t)dst | (uintptr_t)src | (uintptr_t)bytes) & 15) == 0) {
    for (int64_t c = threadIdx.x; c < bytes / 16; c += blockDim.x) ((uint4*)dst)[c] = ((const uint4*)src)[c];
  } else {
    for (int64_t c = threadIdx.x; c < bytes; c += blockDim.x) dst[c] = src[c];
  }
}

// blocks 0 .. T-1: accepted row i (if any) to feats / ids row P + i; block T:
// the last accepted node's logit row to root
__global__ __launch_bounds__(256) void loop_commit_rows_kernel(const int32_t* __restrict__ res, int T,
                                                               const int64_t* __restrict__ tokens,
                                                               const uint8_t* __restrict__ fused, int64_t feat_bytes,
                                                               const uint8_t* __restrict__ logits, int64_t row_bytes,
                                                               uint8_t* __restrict__ feats, int64_t* __restrict__ ids,
                                                               uint8_t* __restrict__ root, int64_t cap,
                                                               const int64_t* __restrict__ state) {
  const int n = res[0];
  const int64_t P = state[0];
  if (n <= 0 || n > T || P < 0 || P + n + 1 > cap) return;  // the record kernel reports a bad length
  const int i = blockIdx.x;
  if (i < T) {
    if (i >= n) return;
    const int src = res[2 + i];
    if (src < 0 || src >= T) return;
    copy_row(feats + (P + i) * feat_bytes, fused + (int64_t)src * feat_bytes, feat_bytes);
    if (threadIdx.x == 0) ids[P + i] = tokens[src];
    return;
  }
  const int last = res[2 + n - 1];
  if (last < 0 || last >= T) return;
  copy_row(root, logits + (int64_t)last * row_bytes, row_bytes);
}

__device__ __forceinline__ int32_t take_status(int32_t* s) {
  if (!s) return 0;
  const int32_t v = *s;
  *s = 0;
  return v;
}

__global__ void loop_commit_state_kernel(const int32_t* __restrict__ res, int T, const int64_t* __restrict__ tokens,
                                         int64_t* __restrict__ ids, int64_t cap, int64_t* __restrict__ state,
                                         int32_t* __restrict__ rec, int rec_path, int32_t* s0, int32_t* s1,
                                         int32_t* s2) {
  const int n = res[0];
  const int64_t P = state[0];
  const bool ok = n >= 0 && n <= T && P >= 0 && P + n + 1 <= cap;
  for (int i = threadIdx.x; i < rec_path; i += blockDim.x) {
    int32_t tok = -1;
    if (ok && i < n) {
      const int src = res[2 + i];
      tok = (src >= 0 && src < T) ? (int32_t)tokens[src] : -1;
    }
    rec[4 + i] = tok;
  }
  if (threadIdx.x != 0) return;
  int32_t st = take_status(s0) | take_status(s1) | take_status(s2);
  if (!ok) st |= (n < 0 || n > T) ? PE_ERR_TREE : PE_ERR_CAPACITY;
  rec[0] = ok ? n : 0;
  rec[1] = res[1];
  rec[2] |= st;
  if (ok && n > 0) {
    ids[P + n] = res[1];
    state[0] = P + n;
    state[1] = res[1];
  }
}

__global__ __launch_bounds__(256) void loop_miss_rows_kernel(const uint8_t* __restrict__ fused_row,
                                                             int64_t feat_bytes, uint8_t* __restrict__ feats,
                                                             int64_t cap, const int64_t* __restrict__ state) {
  const int64_t P = state[0];
  if (P < 0 || P + 2 > cap) return;
  copy_row(feats + P * feat_bytes, fused_row, feat_bytes);
}

constexpr int kMissThreads = 256;

// The miss pass's bonus: the argmax of its logit row, from the lm_head's
// argmax keys (the largest key names the row's largest value at its lowest
// column, NaN largest: torch.argmax) or, without keys, from a row argmax the
// caller computed (pe_argmax_rows).
__global__ __launch_bounds__(kMissThreads) void loop_miss_state_kernel(const uint64_t* __restrict__ keys, int groups,
                                                                       const int32_t* __restrict__ amax,
                                                                       int64_t* __restrict__ ids, int64_t cap,
                                                                       int64_t* __restrict__ state,
                                                                       int32_t* __restrict__ rec, int32_t* s0,
                                                                       int32_t* s1, int32_t* s2) {
  uint64_t best = 0;
  if (keys)
    for (int i = threadIdx.x; i < groups; i += kMissThreads) best = keys[i] > best ? keys[i] : best;
  __shared__ uint64_t wk[kMissThreads];
  wk[threadIdx.x] = best;
  __syncthreads();
  for (int o = kMissThreads / 2; o > 0; o >>= 1) {
    if (threadIdx.x < o) wk[threadIdx.x] = wk[threadIdx.x + o] > wk[threadIdx.x] ? wk[threadIdx.x + o] : wk[threadIdx.x];
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
  const int64_t P = state[0];
  int32_t st = take_status(s0) | take_status(s1) | take_status(s2);
  const int32_t bonus = keys ? (wk[0] ? (int32_t)(0xFFFFFFFFu - (uint32_t)wk[0]) : -1) : amax[0];
  const bool ok = P >= 0 && P + 2 <= cap && bonus >= 0;
  if (!ok) st |= bonus < 0 ? PE_ERR_VALUE : PE_ERR_CAPACITY;
  rec[2] |= st;
  rec[3] = bonus;
  if (ok) {
    ids[P + 1] = bonus;
    state[0] = P + 1;
    state[1] = bonus;
  }
}

int esz(int dtype) { return dtype == PE_DTYPE_F32 ? 4 : 2; }

}  // namespace

extern "C" int pe_loop_commit(const int32_t* accept_out, int T, const int64_t* node_tokens, const void* node_fused,
                              int feat_dim, const void* node_logits, int64_t V, int dtype, void* feats, int64_t* ids,
                              void* root, int64_t cap, int64_t* state, int32_t* rec, int rec_path, int32_t* status0,
                              int32_t* status1, int32_t* status2, void* stream) {
  if (!accept_out || !node_tokens || !node_fused || !node_logits || !feats || !ids || !root || !state || !rec ||
      T <= 0 || T > 64 * PE_TREE_MAX_WORDS || feat_dim <= 0 || V <= 0 || cap <= 0 || rec_path < 0)
    return PE_ERR_ARG;
  if (dtype != PE_DTYPE_F32 && dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16) return PE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const int es = esz(dtype);
  loop_commit_rows_kernel<<<T + 1, 256, 0, st>>>(accept_out, T, node_tokens, (const uint8_t*)node_fused,
                                                  (int64_t)feat_dim * es, (const uint8_t*)node_logits, V * es,
                                                  (uint8_t*)feats, ids, (uint8_t*)root, cap, state);
  PE_CHECK_LAUNCH();
  loop_commit_state_kernel<<<1, 64, 0, st>>>(accept_out, T, node_tokens, ids, cap, state, rec, rec_path, status0,
                                             status1, status2);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_loop_miss_commit(const void* fused_row, int feat_dim, const uint64_t* keys, int groups,
                                   const int32_t* row_argmax, int dtype, void* feats, int64_t* ids, int64_t cap,
                                   int64_t* state, int32_t* rec, int32_t* status0, int32_t* status1, int32_t* status2,
                                   void* stream) {
  if (!fused_row || !feats || !ids || !state || !rec || feat_dim <= 0 || cap <= 0) return PE_ERR_ARG;
  if (keys ? (groups <= 0 || row_argmax) : !row_argmax) return PE_ERR_ARG;  // exactly one of the two
  if (dtype != PE_DTYPE_F32 && dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16) return PE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  loop_miss_rows_kernel<<<1, 256, 0, st>>>((const uint8_t*)fused_row, (int64_t)feat_dim * esz(dtype),
                                           (uint8_t*)feats, cap, state);
  PE_CHECK_LAUNCH();
  loop_miss_state_kernel<<<1, kMissThreads, 0, st>>>(keys, groups, row_argmax, ids, cap, state, rec, status0, status1,
                                                     status2);
  PE_CHECK_LAUNCH();
  return PE_OK;
}
