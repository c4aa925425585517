// Tree masks, the greedy acceptance walk and in-place KV compaction.
//
// pe_tree_masks replaces tree_depths / tree_allow_mask / tree_position_ids
// (src/pe/masks.py:118-156) with one small kernel that turns `parents` into a
// per-node ancestor bitmask (bit u of bits[t] set iff u is t or an ancestor of t),
// the node depth and its RoPE position P + depth.
//
// pe_accept_tree is accept_tree_cached (src/pe/decode/verify.py:104-125): the
// argmax of the root logit and of every node row (first index among equal
// maxima, as torch.argmax), then the walk that descends into the first child (in
// node order) whose token equals the current argmax. It runs on the device so
// the host reads back one small result instead of syncing per depth.
//
// pe_kv_compact keeps rows [0, P) and the accepted path: row P + path[i] moves
// to P + i. path[i] >= i and path is increasing, so ascending i never
// overwrites a row still to be read; only |path| rows per layer/head move
// instead of index_select copying the whole cache (src/pe/target.py:194-201).

#include "pe_common.h"

namespace {

__global__ void tree_masks_kernel(const int32_t* __restrict__ parents, int T, int64_t P, uint64_t* __restrict__ bits,
                                  int words, int64_t* __restrict__ positions, int32_t* __restrict__ depths,
                                  int32_t* status) {
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    uint64_t b[PE_TREE_MAX_WORDS] = {0ull, 0ull, 0ull, 0ull};
    int depth = 0;
    bool bad = false;
    int a = t;
    // walk up: each step must go to a strictly smaller index
    for (int steps = 0; steps <= T; ++steps) {
      b[a >> 6] |= 1ull << (a & 63);
      const int p = parents[a];
      if (p == -1) break;
      if (p < -1 || p >= a) { bad = true; break; }
      a = p;
      ++depth;
    }
    if (bad && status) atomicOr(status, PE_ERR_TREE);
    for (int w = 0; w < words; ++w) bits[(int64_t)t * words + w] = bad ? 0ull : b[w];
    if (positions) positions[t] = P + depth;
    if (depths) depths[t] = depth;
  }
}

__global__ void allow_dense_kernel(const uint64_t* __restrict__ bits, int T, int words, int64_t P,
                                   uint8_t* __restrict__ allow) {
  const int64_t n = P + T;
  const int64_t total = n * n;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    const int64_t i = idx / n, j = idx % n;
    uint8_t v;
    if (i < P) {
      v = j <= i;
    } else if (j < P) {
      v = 1;
    } else {
      const int t = (int)(i - P), u = (int)(j - P);
      v = (bits[(int64_t)t * words + (u >> 6)] >> (u & 63)) & 1ull;
    }
    allow[idx] = v;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void bias_to_bits_kernel(const typename Elem<DT>::T* __restrict__ bias, int64_t ld,
                                                           int T, int64_t P, float masked_below,
                                                           uint64_t* __restrict__ bits, int words, int32_t* status) {
  const int t = blockIdx.x;
  __shared__ unsigned long long w[PE_TREE_MAX_WORDS];
  if (threadIdx.x < PE_TREE_MAX_WORDS) w[threadIdx.x] = 0ull;
  __syncthreads();
  const int64_t S = P + T;
  int err = 0;
  for (int64_t j = threadIdx.x; j < S; j += blockDim.x) {
    const float v = Elem<DT>::load(bias, (int64_t)t * ld + j);
    const bool allowed = v == 0.f;
    const bool masked = v <= masked_below;
    if (!allowed && !masked) err = 1;
    if (j < P) {
      if (!allowed) err = 1;
    } else if (allowed) {
      const int u = (int)(j - P);
      atomicOr(&w[u >> 6], 1ull << (u & 63));
    }
  }
  if (err && status) atomicOr(status, PE_ERR_MASK);
  __syncthreads();
  if (threadIdx.x < words) bits[(int64_t)t * words + threadIdx.x] = w[threadIdx.x];
}

// Row argmax with torch.argmax's semantics: the largest value, a NaN beats
// every number, and among equal maxima (or NaNs) the lowest index wins.
struct ArgBest {
  float v;
  int idx;  // -1: none yet
  int nan;
};

__device__ __forceinline__ bool arg_better(const ArgBest& b, const ArgBest& a) {  // b beats a
  if (b.idx < 0) return false;
  if (a.idx < 0) return true;
  if (a.nan && b.nan) return b.idx < a.idx;
  if (a.nan) return false;
  if (b.nan) return true;
  return (b.v > a.v) || (b.v == a.v && b.idx < a.idx);
}

__device__ __forceinline__ void arg_take(ArgBest& a, float v, int i) {
  ArgBest b = {v, i, v != v};
  if (arg_better(b, a)) a = b;
}

constexpr int kArgThreads = 1024;

// One block of kArgThreads per row. Thread t scans 8-element vectors
// t, t + kArgThreads, ... in increasing index order (all loads issued first),
// then the block reduces with the same rule.
template <int DT>
__device__ void row_argmax(const typename Elem<DT>::T* __restrict__ x, int64_t V, int32_t* out) {
  typedef typename Elem<DT>::T T;
  constexpr int kPer = 16 / sizeof(T);  // elements per 16-byte vector
  constexpr int kVec = 8;               // vectors per thread held in flight
  ArgBest best = {0.f, -1, 0};
  const bool aligned = (((uintptr_t)x) & 15) == 0;
  const int64_t nvec = aligned ? V / kPer : 0;
  for (int64_t v0 = 0; v0 < nvec; v0 += (int64_t)kVec * kArgThreads) {
    u32x4_t buf[kVec];
#pragma unroll
    for (int k = 0; k < kVec; ++k) {
      const int64_t vi = v0 + (int64_t)k * kArgThreads + threadIdx.x;
      if (vi < nvec) buf[k] = *(const u32x4_t*)(x + vi * kPer);
    }
#pragma unroll
    for (int k = 0; k < kVec; ++k) {
      const int64_t vi = v0 + (int64_t)k * kArgThreads + threadIdx.x;
      if (vi < nvec) {
        const T* e = (const T*)&buf[k];
#pragma unroll
        for (int j = 0; j < kPer; ++j) arg_take(best, Elem<DT>::load(e, j), (int)(vi * kPer + j));
      }
    }
  }
  for (int64_t i = nvec * kPer + threadIdx.x; i < V; i += kArgThreads) arg_take(best, Elem<DT>::load(x, i), (int)i);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    ArgBest b;
    b.v = __shfl_xor(best.v, o, 64);
    b.idx = __shfl_xor(best.idx, o, 64);
    b.nan = __shfl_xor(best.nan, o, 64);
    if (arg_better(b, best)) best = b;
  }
  __shared__ ArgBest wbest[kArgThreads / 64];
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgBest a = wbest[0];
    for (int w = 1; w < kArgThreads / 64; ++w)
      if (arg_better(wbest[w], a)) a = wbest[w];
    *out = a.idx;
  }
}

template <int DT>
__global__ __launch_bounds__(kArgThreads) void argmax_rows_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                                  int64_t ld, int64_t V, int32_t* __restrict__ out) {
  row_argmax<DT>(x + (int64_t)blockIdx.x * ld, V, out + blockIdx.x);
}

// row 0 = root logit, rows 1..T = node logits
template <int DT>
__global__ __launch_bounds__(kArgThreads) void accept_argmax_kernel(const typename Elem<DT>::T* __restrict__ root,
                                                                    const typename Elem<DT>::T* __restrict__ nodes,
                                                                    int64_t ld, int64_t V,
                                                                    int32_t* __restrict__ amax) {
  const int r = blockIdx.x;
  const typename Elem<DT>::T* x = (r == 0) ? root : nodes + (int64_t)(r - 1) * ld;
  row_argmax<DT>(x, V, amax + r);
}

__global__ void accept_walk_kernel(const int32_t* __restrict__ amax, int T, const int64_t* __restrict__ tokens,
                                   const int32_t* __restrict__ parents, int32_t* __restrict__ out) {
  if (threadIdx.x != 0) return;
  int cur = -1, len = 0;
  int truth = amax[0];
  for (;;) {
    int nxt = -1;
    for (int t = 0; t < T; ++t) {
      if (parents[t] == cur && tokens[t] == (int64_t)truth) { nxt = t; break; }
    }
    if (nxt < 0 || len >= T) break;
    out[2 + len] = nxt;
    ++len;
    cur = nxt;
    truth = amax[1 + nxt];
  }
  out[0] = len;
  out[1] = truth;
}

// grid: (L * nkv, 2 for K/V); threads over 16-byte chunks of a row
__global__ void kv_compact_kernel(uint8_t* __restrict__ kc, uint8_t* __restrict__ vc, int64_t cap, int64_t row_bytes,
                                  int64_t P, const int32_t* __restrict__ res) {
  const int len = res[0];
  uint8_t* base = (blockIdx.y == 0 ? kc : vc) + (int64_t)blockIdx.x * cap * row_bytes;
  const int64_t nchunk = row_bytes / 16;
  for (int i = 0; i < len; ++i) {
    const int src = res[2 + i];
    if (src == i || src < 0 || P + src >= cap || P + i >= cap) continue;
    const uint4* s = (const uint4*)(base + (P + src) * row_bytes);
    uint4* d = (uint4*)(base + (P + i) * row_bytes);
    for (int64_t c = threadIdx.x; c < nchunk; c += blockDim.x) d[c] = s[c];
    __syncthreads();
  }
}

// validate keep (strictly increasing, < cap) and find the first i with keep[i] != i
__global__ void kv_keep_check_kernel(const int64_t* __restrict__ keep, int64_t n, int64_t cap,
                                     int64_t* __restrict__ first, int32_t* status) {
  __shared__ unsigned long long fmin;
  if (threadIdx.x == 0) fmin = (unsigned long long)n;
  __syncthreads();
  int err = 0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const int64_t k = keep[i];
    if (k < 0 || k >= cap || (i > 0 && keep[i - 1] >= k)) err = 1;
    if (k != i) atomicMin(&fmin, (unsigned long long)i);
  }
  if (err && status) atomicOr(status, PE_ERR_INDEX);
  __syncthreads();
  if (threadIdx.x == 0) *first = err ? n : (int64_t)fmin;
}

__global__ void kv_gather_kernel(uint8_t* __restrict__ kc, uint8_t* __restrict__ vc, int64_t cap, int64_t row_bytes,
                                 const int64_t* __restrict__ keep, int64_t n, const int64_t* __restrict__ first) {
  const int64_t f = *first;
  uint8_t* base = (blockIdx.y == 0 ? kc : vc) + (int64_t)blockIdx.x * cap * row_bytes;
  const int64_t nchunk = row_bytes / 16;
  for (int64_t i = f; i < n; ++i) {
    const int64_t src = keep[i];
    if (src == i) continue;
    const uint4* s = (const uint4*)(base + src * row_bytes);
    uint4* d = (uint4*)(base + i * row_bytes);
    for (int64_t c = threadIdx.x; c < nchunk; c += blockDim.x) d[c] = s[c];
    __syncthreads();
  }
}

int esize(int dtype) { return dtype == PE_DTYPE_F32 ? 4 : 2; }

}  // namespace

extern "C" int pe_tree_masks(const int32_t* parents, int T, int64_t P, uint64_t* bits, int words, int64_t* positions,
                             int32_t* depths, int32_t* status, void* stream) {
  if (!parents || !bits || T <= 0 || P < 0 || words <= 0 || words > PE_TREE_MAX_WORDS) return PE_ERR_ARG;
  if (T > 64 * words) return PE_ERR_TREE;
  tree_masks_kernel<<<1, 256, 0, (hipStream_t)stream>>>(parents, T, P, bits, words, positions, depths, status);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_tree_allow_dense(const uint64_t* bits, int T, int words, int64_t P, uint8_t* allow, void* stream) {
  if (!bits || !allow || T <= 0 || P < 0 || words <= 0 || words > PE_TREE_MAX_WORDS || T > 64 * words)
    return PE_ERR_ARG;
  const int64_t n = P + T;
  int64_t g = (n * n + 255) / 256;
  if (g > 65536) g = 65536;
  allow_dense_kernel<<<(int)g, 256, 0, (hipStream_t)stream>>>(bits, T, words, P, allow);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_bias_to_bits(const void* bias, int64_t ld_bias, int dtype, int T, int64_t P, uint64_t* bits,
                               int words, int32_t* status, void* stream) {
  if (!bias || !bits || T <= 0 || P < 0 || words <= 0 || words > PE_TREE_MAX_WORDS) return PE_ERR_ARG;
  if (T > 64 * words) return PE_ERR_TREE;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case PE_DTYPE_F32:
      bias_to_bits_kernel<PE_DTYPE_F32><<<T, 256, 0, st>>>((const float*)bias, ld_bias, T, P, -1.7014117e38f, bits,
                                                           words, status);
      break;
    case PE_DTYPE_BF16:
      bias_to_bits_kernel<PE_DTYPE_BF16><<<T, 256, 0, st>>>((const uint16_t*)bias, ld_bias, T, P, -1.69e38f, bits,
                                                            words, status);
      break;
    case PE_DTYPE_F16:
      bias_to_bits_kernel<PE_DTYPE_F16><<<T, 256, 0, st>>>((const uint16_t*)bias, ld_bias, T, P, -32752.f, bits,
                                                           words, status);
      break;
    default:
      return PE_ERR_ARG;
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_argmax_rows(const void* x, int64_t ld, int rows, int64_t V, int dtype, int32_t* out_idx,
                              void* stream) {
  if (!x || !out_idx || rows <= 0 || V <= 0) return PE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case PE_DTYPE_F32: argmax_rows_kernel<PE_DTYPE_F32><<<rows, kArgThreads, 0, st>>>((const float*)x, ld, V, out_idx); break;
    case PE_DTYPE_BF16: argmax_rows_kernel<PE_DTYPE_BF16><<<rows, kArgThreads, 0, st>>>((const uint16_t*)x, ld, V, out_idx); break;
    case PE_DTYPE_F16: argmax_rows_kernel<PE_DTYPE_F16><<<rows, kArgThreads, 0, st>>>((const uint16_t*)x, ld, V, out_idx); break;
    default: return PE_ERR_ARG;
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_accept_tree(const void* root_logit, const void* node_logits, int64_t ld, int T, int64_t V, int dtype,
                              const int64_t* node_tokens, const int32_t* parents, int32_t* out, int32_t* scratch,
                              void* stream) {
  if (!root_logit || !out || !scratch || T < 0 || V <= 0) return PE_ERR_ARG;
  if (T > 0 && (!node_logits || !node_tokens || !parents)) return PE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case PE_DTYPE_F32:
      accept_argmax_kernel<PE_DTYPE_F32><<<T + 1, kArgThreads, 0, st>>>((const float*)root_logit, (const float*)node_logits,
                                                                ld, V, scratch);
      break;
    case PE_DTYPE_BF16:
      accept_argmax_kernel<PE_DTYPE_BF16><<<T + 1, kArgThreads, 0, st>>>((const uint16_t*)root_logit,
                                                                 (const uint16_t*)node_logits, ld, V, scratch);
      break;
    case PE_DTYPE_F16:
      accept_argmax_kernel<PE_DTYPE_F16><<<T + 1, kArgThreads, 0, st>>>((const uint16_t*)root_logit,
                                                                (const uint16_t*)node_logits, ld, V, scratch);
      break;
    default:
      return PE_ERR_ARG;
  }
  PE_CHECK_LAUNCH();
  accept_walk_kernel<<<1, 64, 0, st>>>(scratch, T, node_tokens, parents, out);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_kv_compact(void* k_cache, void* v_cache, int L, int nkv, int64_t cap, int hd, int dtype, int64_t P,
                             const int32_t* accept_out, void* stream) {
  if (!k_cache || !v_cache || !accept_out || L <= 0 || nkv <= 0 || hd <= 0 || P < 0) return PE_ERR_ARG;
  const int64_t row_bytes = (int64_t)hd * esize(dtype);
  if (row_bytes % 16) return PE_ERR_ARG;
  dim3 grid(L * nkv, 2);
  kv_compact_kernel<<<grid, 64, 0, (hipStream_t)stream>>>((uint8_t*)k_cache, (uint8_t*)v_cache, cap, row_bytes, P,
                                                         accept_out);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_kv_gather(void* k_cache, void* v_cache, int L, int nkv, int64_t cap, int hd, int dtype,
                            const int64_t* keep, int64_t n_keep, int32_t* status, void* stream) {
  if (!k_cache || !v_cache || !keep || !status || L <= 0 || nkv <= 0 || hd <= 0 || n_keep < 0 || n_keep > cap)
    return PE_ERR_ARG;
  if (n_keep == 0) return PE_OK;
  const int64_t row_bytes = (int64_t)hd * esize(dtype);
  if (row_bytes % 16) return PE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  // `first` lives in the status word's neighbour: callers pass status as int32[4] (8-byte aligned at +8)
  int64_t* first = (int64_t*)(status + 2);
  kv_keep_check_kernel<<<1, 256, 0, st>>>(keep, n_keep, cap, first, status);
  PE_CHECK_LAUNCH();
  dim3 grid(L * nkv, 2);
  kv_gather_kernel<<<grid, 64, 0, st>>>((uint8_t*)k_cache, (uint8_t*)v_cache, cap, row_bytes, keep, n_keep, first);
  PE_CHECK_LAUNCH();
  return PE_OK;
}
