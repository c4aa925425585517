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

#include <mutex>

namespace {

// Depth, position P + depth and ancestor bits of the T nodes of one tree
// (parents in the tree's own numbering), by the threads of one block.
__device__ void tree_masks_rows(const int32_t* __restrict__ parents, int T, int64_t P, uint64_t* __restrict__ bits,
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

__global__ void tree_masks_kernel(const int32_t* __restrict__ parents, int T, int64_t P, uint64_t* __restrict__ bits,
                                  int words, int64_t* __restrict__ positions, int32_t* __restrict__ depths,
                                  int32_t* status) {
  tree_masks_rows(parents, T, P, bits, words, positions, depths, status);
}

// Batched trees: block b handles sequence b's rows [seq_row0[b], seq_row0[b+1]).
__global__ void tree_masks_batch_kernel(const int32_t* __restrict__ parents, const int32_t* __restrict__ seq_row0,
                                        const int64_t* __restrict__ seq_prefix, int max_rows,
                                        uint64_t* __restrict__ bits, int words, int64_t* __restrict__ positions,
                                        int32_t* __restrict__ depths, int32_t* status) {
  const int b = blockIdx.x;
  const int r0 = seq_row0[b], T = seq_row0[b + 1] - r0;
  if (T < 0 || T > max_rows || r0 < 0) {
    if (threadIdx.x == 0 && status) atomicOr(status, PE_ERR_TREE);
    return;
  }
  tree_masks_rows(parents + r0, T, seq_prefix[b], bits + (int64_t)r0 * words, words,
                  positions ? positions + r0 : nullptr, depths ? depths + r0 : nullptr, status);
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
constexpr int kArgThreads = 1024;

// One block of kArgThreads per row. Thread t scans 16-byte vectors t,
// t + kArgThreads, ... in increasing index order (all loads issued first)
// keeping the first element of the largest key; the block then reduces with
// (key descending, index ascending).
template <int DT>
__device__ int row_argmax(const typename Elem<DT>::T* __restrict__ x, int64_t V, int32_t* out) {
  typedef typename Elem<DT>::T T;
  constexpr int kPer = 16 / sizeof(T);  // elements per 16-byte vector
  constexpr int kVec = 8;               // vectors per thread held in flight
  uint32_t bk = 0;                      // below every real key
  int bi = -1;
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
        for (int j = 0; j < kPer; ++j) {
          const uint32_t key = arg_key(Elem<DT>::load(e, j));
          if (key > bk) {
            bk = key;
            bi = (int)(vi * kPer + j);
          }
        }
      }
    }
  }
  for (int64_t i = nvec * kPer + threadIdx.x; i < V; i += kArgThreads) {
    const uint32_t key = arg_key(Elem<DT>::load(x, i));
    if (key > bk) {
      bk = key;
      bi = (int)i;
    }
  }
  auto better = [](uint32_t k2, int i2, uint32_t k1, int i1) {  // (k2, i2) beats (k1, i1)
    if (i2 < 0) return false;
    if (i1 < 0) return true;
    return k2 > k1 || (k2 == k1 && i2 < i1);
  };
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t k2 = __shfl_xor(bk, o, 64);
    const int i2 = __shfl_xor(bi, o, 64);
    if (better(k2, i2, bk, bi)) {
      bk = k2;
      bi = i2;
    }
  }
  __shared__ uint32_t wk[kArgThreads / 64];
  __shared__ int wi[kArgThreads / 64];
  if ((threadIdx.x & 63) == 0) {
    wk[threadIdx.x >> 6] = bk;
    wi[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  int i1 = -1;
  if (threadIdx.x == 0) {
    uint32_t k1 = wk[0];
    i1 = wi[0];
    for (int w = 1; w < kArgThreads / 64; ++w)
      if (better(wk[w], wi[w], k1, i1)) {
        k1 = wk[w];
        i1 = wi[w];
      }
    if (out) *out = i1;
  }
  return i1;
}

// Row argmax from per-column-group keys (arg_key64, written by the lm_head
// GEMM's argmax epilogue): the largest key and its column; the result is
// valid in thread 0.
__device__ int row_argmax_keys(const uint64_t* __restrict__ keys, int groups) {
  uint64_t best = 0;  // below every real key
  for (int i = threadIdx.x; i < groups; i += kArgThreads) {
    const uint64_t k = keys[i];
    best = k > best ? k : best;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t k = shfl_xor_u64(best, o);
    best = k > best ? k : best;
  }
  __shared__ uint64_t wk[kArgThreads / 64];
  if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = best;
  __syncthreads();
  int idx = -1;
  if (threadIdx.x == 0) {
    uint64_t b = wk[0];
    for (int w = 1; w < kArgThreads / 64; ++w) b = wk[w] > b ? wk[w] : b;
    idx = b ? (int)(0xFFFFFFFFu - (uint32_t)b) : -1;
  }
  return idx;
}

template <int DT>
__global__ __launch_bounds__(kArgThreads) void argmax_rows_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                                  int64_t ld, int64_t V, int32_t* __restrict__ out) {
  row_argmax<DT>(x + (int64_t)blockIdx.x * ld, V, out + blockIdx.x);
}

// One launch does the whole acceptance. Block r finds the argmax of row r
// (row 0 = root logit, rows 1..T = node logits) and publishes it in
// work[1 + r]; the last block to count itself on work[0] (every row's argmax
// is then visible) resets that counter and walks the tree. The counter sits
// at index 0 whatever T is, so one scratch buffer serves calls of any size. The walk stages every
// node's argmax, parent and token in LDS; one wave then follows the greedy
// path, each step a ballot over the nodes for the first child of the current
// node whose token equals the current truth (at most kWalkMax nodes).
constexpr int kWalkMax = 64 * PE_TREE_MAX_WORDS;

// Batched trees (seq_row0 non-null): blockIdx.y = sequence b, whose root row
// is root + b * ld_root, node rows start at row seq_row0[b], scratch at
// work + b * (T + 2) and result at out + b * (T + 2), T being the largest
// tree; blocks past the sequence's own node count leave at once.
template <int DT>
__global__ __launch_bounds__(kArgThreads) void accept_kernel(const typename Elem<DT>::T* __restrict__ root,
                                                             int64_t ld_root,
                                                             const typename Elem<DT>::T* __restrict__ nodes,
                                                             int64_t ld, int64_t V, int32_t* __restrict__ work,
                                                             int T, const int32_t* __restrict__ seq_row0,
                                                             const int64_t* __restrict__ tokens,
                                                             const int32_t* __restrict__ parents,
                                                             int32_t* __restrict__ out,
                                                             const uint64_t* __restrict__ node_keys, int groups) {
  if (seq_row0) {
    const int b = blockIdx.y, r0 = seq_row0[b];
    root += b * ld_root;
    nodes += (int64_t)r0 * ld;
    work += (int64_t)b * (T + 2);
    out += (int64_t)b * (T + 2);
    tokens += r0;
    parents += r0;
    T = min(max(seq_row0[b + 1] - r0, 0), T);
    if ((int)blockIdx.x > T) return;
  }
  int32_t* const counter = work;
  int32_t* const amax = work + 1;
  const int r = blockIdx.x;
  const typename Elem<DT>::T* x = (r == 0) ? root : nodes + (int64_t)(r - 1) * ld;
  // node rows from the lm_head's argmax keys when the caller has them
  const int best = (node_keys && r > 0) ? row_argmax_keys(node_keys + (int64_t)(r - 1) * groups, groups)
                                        : row_argmax<DT>(x, V, nullptr);
  __shared__ int s_last;
  if (threadIdx.x == 0) {
    // The row's argmax is stored at agent scope (past this die's L2) and
    // acknowledged before the block counts itself, and the last block reads
    // every argmax at agent scope, so it sees all of them. (An acquire-release
    // count would write back and invalidate the whole L2 in every block.)
    __hip_atomic_store(amax + r, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == T;
    if (old == T) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  __shared__ int32_t s_amax[kWalkMax + 1], s_par[kWalkMax];
  __shared__ int64_t s_tok[kWalkMax];
  const int n = min(T, kWalkMax);
  for (int t = threadIdx.x; t <= n; t += kArgThreads)
    s_amax[t] = __hip_atomic_load(amax + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int t = threadIdx.x; t < n; t += kArgThreads) {
    s_par[t] = parents[t];
    s_tok[t] = tokens[t];
  }
  __syncthreads();
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  int cur = -1, len = 0;
  int truth = s_amax[0];
  for (;;) {
    int nxt = -1;
    for (int base = 0; base < n; base += 64) {
      const int t = base + lane;
      const bool hit = t < n && s_par[t] == cur && s_tok[t] == (int64_t)truth;
      const uint64_t b = __ballot(hit);
      if (b) {
        nxt = base + (int)__builtin_ctzll(b);
        break;
      }
    }
    if (nxt < 0 || len >= n) break;
    if (lane == 0) out[2 + len] = nxt;
    ++len;
    cur = nxt;
    truth = s_amax[1 + nxt];
  }
  if (lane == 0) {
    out[0] = len;
    out[1] = truth;
  }
}

// grid: (L * nkv, 2 for K/V, batch); threads over 16-byte chunks of a row.
// Batched (seq_prefix non-null): sequence b = blockIdx.z has its cache at
// seq_bytes * b, its prefix seq_prefix[b] and its result at res + b * res_stride.
__global__ void kv_compact_kernel(uint8_t* __restrict__ kc, uint8_t* __restrict__ vc, int64_t cap, int64_t row_bytes,
                                  int64_t P, const int32_t* __restrict__ res, const int64_t* __restrict__ seq_prefix,
                                  int64_t seq_bytes, int res_stride) {
  if (seq_prefix) {
    const int b = blockIdx.z;
    P = seq_prefix[b];
    res += (int64_t)b * res_stride;
    kc += b * seq_bytes;
    vc += b * seq_bytes;
  }
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

// Beam tree proposal (propose_tree, src/pe/decode/tree.py:34-55) in two
// launches. draft_topk_kernel: one block per depth row computes the row's
// log-sum-exp in fp32 and selects the row's top c_d tokens one at a time, each
// round the best element after the previous one in (value descending, index
// ascending) order; the winners' log-probabilities (x - max) - log(sum) go to
// scratch. beam_kernel: one block walks the depths; candidate (parent p, rank
// j in the row) scores cum[p] + lp[j] in float64, and its position in the
// stable descending order of the candidate list (parent-major, as the
// reference builds it) is counted directly: j for its own parent, plus, for
// every other parent, the candidates that score higher (or equal, for parents
// before it), found by binary search since each parent's scores do not
// increase with j.
constexpr int kBeamThreads = 256;

struct BeamShape {
  int k;
  int width[PE_PROPOSE_MAX_DEPTH];  // nodes kept at depth d
  int cand[PE_PROPOSE_MAX_DEPTH];   // candidates per parent: min(top_k, width[d])
};

// (k2, i2) before (k1, i1) in the order key descending, index ascending; i < 0 is "none"
__device__ __forceinline__ bool key_before(uint32_t k2, int i2, uint32_t k1, int i1) {
  if (i2 < 0) return false;
  if (i1 < 0) return true;
  return k2 > k1 || (k2 == k1 && i2 < i1);
}

// block-wide (key, index) reduction over kArgThreads threads; every thread gets the result
__device__ void block_best(uint32_t& bk, int& bi, uint32_t* wk, int* wi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t k2 = __shfl_xor(bk, o, 64);
    const int i2 = __shfl_xor(bi, o, 64);
    if (key_before(k2, i2, bk, bi)) {
      bk = k2;
      bi = i2;
    }
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    wk[threadIdx.x >> 6] = bk;
    wi[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  bk = wk[0];
  bi = wi[0];
  for (int w = 1; w < kArgThreads / 64; ++w)
    if (key_before(wk[w], wi[w], bk, bi)) {
      bk = wk[w];
      bi = wi[w];
    }
}

__device__ float block_sum(float v, float* ws) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
  for (int w = 0; w < kArgThreads / 64; ++w) s += ws[w];
  return s;
}

template <int DT>
__global__ __launch_bounds__(kArgThreads) void draft_topk_kernel(const typename Elem<DT>::T* __restrict__ logits,
                                                                 int64_t ld, int64_t V, BeamShape bs,
                                                                 float* __restrict__ lp_out,
                                                                 int32_t* __restrict__ tok_out, int32_t* status) {
  const int d = blockIdx.x;
  const typename Elem<DT>::T* x = logits + (int64_t)d * ld;
  __shared__ uint32_t wk[kArgThreads / 64];
  __shared__ int wi[kArgThreads / 64];
  __shared__ float ws[kArgThreads / 64];
  // the row maximum (the first selection round) and NaN detection
  uint32_t bk = 0;
  int bi = -1;
  int nan = 0;
  for (int64_t i = threadIdx.x; i < V; i += kArgThreads) {
    const float v = Elem<DT>::load(x, i);
    nan |= v != v;
    const uint32_t key = arg_key(v);
    if (key_before(key, (int)i, bk, bi)) {
      bk = key;
      bi = (int)i;
    }
  }
  nan = __syncthreads_or(nan);
  block_best(bk, bi, wk, wi);
  const float mx = Elem<DT>::load(x, bi);
  if (nan || !(mx > -INFINITY) || mx == INFINITY) {
    if (threadIdx.x == 0 && status) atomicOr(status, PE_ERR_VALUE);
    return;
  }
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < V; i += kArgThreads) s += expf(Elem<DT>::load(x, i) - mx);
  const float logsum = logf(block_sum(s, ws));
  const int c = bs.cand[d];
  for (int j = 0;; ++j) {
    if (threadIdx.x == 0) {
      lp_out[d * PE_PROPOSE_MAX_WIDTH + j] = (Elem<DT>::load(x, bi) - mx) - logsum;
      tok_out[d * PE_PROPOSE_MAX_WIDTH + j] = bi;
    }
    if (j + 1 >= c) break;
    // next round: the best element after (bk, bi) in the order
    const uint32_t pk = bk;
    const int pi = bi;
    bk = 0;
    bi = -1;
    for (int64_t i = threadIdx.x; i < V; i += kArgThreads) {
      const uint32_t key = arg_key(Elem<DT>::load(x, i));
      if (key_before(pk, pi, key, (int)i) && key_before(key, (int)i, bk, bi)) {
        bk = key;
        bi = (int)i;
      }
    }
    block_best(bk, bi, wk, wi);
  }
}

__global__ __launch_bounds__(kBeamThreads) void beam_kernel(BeamShape bs, const float* __restrict__ lp,
                                                            const int32_t* __restrict__ tok,
                                                            int64_t* __restrict__ node_tokens,
                                                            int32_t* __restrict__ parents, const int32_t* status) {
  if (status && *status & PE_ERR_VALUE) return;
  __shared__ double cum[PE_PROPOSE_MAX_WIDTH], ncum[PE_PROPOSE_MAX_WIDTH], row[PE_PROPOSE_MAX_WIDTH];
  __shared__ int node[PE_PROPOSE_MAX_WIDTH];
  int nb = 1, base = 0;
  if (threadIdx.x == 0) {
    cum[0] = 0.0;
    node[0] = -1;
  }
  for (int d = 0; d < bs.k; ++d) {
    const int c = bs.cand[d];
    const int n = nb * c;
    const int kept = min(bs.width[d], n);
    if (threadIdx.x < c) row[threadIdx.x] = (double)lp[d * PE_PROPOSE_MAX_WIDTH + threadIdx.x];
    __syncthreads();
    for (int q = threadIdx.x; q < n; q += kBeamThreads) {
      const int p = q / c, j = q - p * c;
      const double sc = cum[p] + row[j];
      int r = j;
      for (int p2 = 0; p2 < nb && r < kept; ++p2) {
        if (p2 == p) continue;
        // count j2 with cum[p2] + row[j2] > sc (>= sc for parents listed before p)
        int lo = 0, hi = c;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          const double s2 = cum[p2] + row[mid];
          if (p2 < p ? s2 >= sc : s2 > sc)
            lo = mid + 1;
          else
            hi = mid;
        }
        r += lo;
      }
      if (r < kept) {
        ncum[r] = sc;
        node_tokens[base + r] = tok[d * PE_PROPOSE_MAX_WIDTH + j];
        parents[base + r] = node[p];
      }
    }
    __syncthreads();
    if (threadIdx.x < kept) {
      cum[threadIdx.x] = ncum[threadIdx.x];
      node[threadIdx.x] = base + threadIdx.x;
    }
    __syncthreads();
    base += kept;
    nb = kept;
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

extern "C" int pe_tree_masks_batch(const int32_t* parents, const int32_t* seq_row0, const int64_t* seq_prefix, int batch,
                                   int max_seq_rows, uint64_t* bits, int words, int64_t* positions, int32_t* depths,
                                   int32_t* status, void* stream) {
  if (!parents || !seq_row0 || !seq_prefix || !bits || batch <= 0 || max_seq_rows <= 0 || words <= 0 ||
      words > PE_TREE_MAX_WORDS)
    return PE_ERR_ARG;
  if (max_seq_rows > 64 * words) return PE_ERR_TREE;
  tree_masks_batch_kernel<<<batch, 256, 0, (hipStream_t)stream>>>(parents, seq_row0, seq_prefix, max_seq_rows, bits,
                                                                   words, positions, depths, status);
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

namespace {

// batch == 0: one tree of T nodes; batch >= 1: seq_row0 [batch + 1] splits the
// node rows into trees of at most T nodes each.
int launch_accept(const void* root_logit, int64_t ld_root, const void* node_logits, int64_t ld, int T, int64_t V,
                  int dtype, const int32_t* seq_row0, int batch, const int64_t* node_tokens, const int32_t* parents,
                  int32_t* out, int32_t* work, hipStream_t st, const uint64_t* node_keys = nullptr,
                  int groups = 0) {
  const dim3 grid(T + 1, batch > 0 ? batch : 1);
  switch (dtype) {
    case PE_DTYPE_F32:
      accept_kernel<PE_DTYPE_F32><<<grid, kArgThreads, 0, st>>>((const float*)root_logit, ld_root,
                                                                (const float*)node_logits, ld, V, work, T, seq_row0,
                                                                node_tokens, parents, out, node_keys, groups);
      break;
    case PE_DTYPE_BF16:
      accept_kernel<PE_DTYPE_BF16><<<grid, kArgThreads, 0, st>>>((const uint16_t*)root_logit, ld_root,
                                                                 (const uint16_t*)node_logits, ld, V, work, T,
                                                                 seq_row0, node_tokens, parents, out, node_keys,
                                                                 groups);
      break;
    case PE_DTYPE_F16:
      accept_kernel<PE_DTYPE_F16><<<grid, kArgThreads, 0, st>>>((const uint16_t*)root_logit, ld_root,
                                                                (const uint16_t*)node_logits, ld, V, work, T,
                                                                seq_row0, node_tokens, parents, out, node_keys,
                                                                groups);
      break;
    default:
      return PE_ERR_ARG;
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}

int check_accept_args(const void* root_logit, const void* node_logits, int T, int64_t V, int dtype,
                      const int64_t* node_tokens, const int32_t* parents, const int32_t* out) {
  if (!root_logit || !out || T < 0 || V <= 0) return PE_ERR_ARG;
  if (dtype != PE_DTYPE_F32 && dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16) return PE_ERR_ARG;
  if (T > 0 && (!node_logits || !node_tokens || !parents)) return PE_ERR_ARG;
  if (T > kWalkMax) return PE_ERR_TREE;
  return PE_OK;
}

// The acceptance scratch of pe_accept_tree_noalloc: an arrival counter and
// the row argmaxes of a tree of up to kWalkMax nodes. One copy per GPU, kept
// for the life of the process; calls on one GPU share it.
static __device__ __align__(256) int32_t scratch[kWalkMax + 2];

// Device address of `scratch` per device (the array's name is a host-side
// stand-in in host code), looked up once per device with that device current.
int32_t* scratch_ptr() {
  static std::mutex mu;
  static int32_t* ptrs[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    ptrs[dev] = (int32_t*)p;
  }
  return ptrs[dev];
}

__global__ void zero_counter_kernel(int32_t* counter) { *counter = 0; }

}  // namespace

extern "C" int pe_accept_tree(const void* root_logit, const void* node_logits, int64_t ld, int T, int64_t V, int dtype,
                              const int64_t* node_tokens, const int32_t* parents, int32_t* out, int32_t* work,
                              void* stream) {
  int rc = check_accept_args(root_logit, node_logits, T, V, dtype, node_tokens, parents, out);
  if (rc != PE_OK) return rc;
  if (!work) return PE_ERR_ARG;
  return launch_accept(root_logit, 0, node_logits, ld, T, V, dtype, nullptr, 0, node_tokens, parents, out, work,
                       (hipStream_t)stream);
}

extern "C" int pe_accept_tree_keys(const void* root_logit, int64_t V, int dtype, const uint64_t* node_keys,
                                   int groups, int T, const int64_t* node_tokens, const int32_t* parents, int32_t* out,
                                   int32_t* scratch, void* stream) {
  if (!root_logit || !out || !scratch || T < 0 || V <= 0) return PE_ERR_ARG;
  if (dtype != PE_DTYPE_F32 && dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16) return PE_ERR_ARG;
  if (T > 0 && (!node_keys || groups <= 0 || !node_tokens || !parents)) return PE_ERR_ARG;
  if (T > kWalkMax) return PE_ERR_TREE;
  return launch_accept(root_logit, 0, nullptr, 0, T, V, dtype, nullptr, 0, node_tokens, parents, out, scratch,
                       (hipStream_t)stream, node_keys, groups);
}

extern "C" int pe_accept_tree_batch(const void* root_logits, int64_t ld_root, const void* node_logits, int64_t ld,
                                    int64_t V, int dtype, const int32_t* seq_row0, int batch, int max_seq_rows,
                                    const int64_t* node_tokens, const int32_t* parents, int32_t* out, int32_t* scratch,
                                    void* stream) {
  if (!root_logits || !node_logits || !seq_row0 || !node_tokens || !parents || !out || !scratch || batch <= 0 ||
      max_seq_rows <= 0 || V <= 0 || ld_root < V || ld < V)
    return PE_ERR_ARG;
  if (dtype != PE_DTYPE_F32 && dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16) return PE_ERR_ARG;
  if (max_seq_rows > kWalkMax) return PE_ERR_TREE;
  return launch_accept(root_logits, ld_root, node_logits, ld, max_seq_rows, V, dtype, seq_row0, batch, node_tokens,
                       parents, out, scratch, (hipStream_t)stream);
}

extern "C" int pe_accept_tree_noalloc(const void* root_logit, const void* node_logits, int64_t ld, int T, int64_t V,
                                      int dtype, const int64_t* node_tokens, const int32_t* parents, int32_t* out,
                                      void* stream) {
  int rc = check_accept_args(root_logit, node_logits, T, V, dtype, node_tokens, parents, out);
  if (rc != PE_OK) return rc;  // T > PE_ACCEPT_NOALLOC_MAX_NODES: PE_ERR_TREE
  int32_t* work = scratch_ptr();
  if (!work) return PE_ERR_LAUNCH;
  hipStream_t st = (hipStream_t)stream;
  // the counter starts at zero: cleared by a kernel (no memset node if the
  // caller captures this call in a graph)
  zero_counter_kernel<<<1, 1, 0, st>>>(work);
  PE_CHECK_LAUNCH();
  return launch_accept(root_logit, 0, node_logits, ld, T, V, dtype, nullptr, 0, node_tokens, parents, out, work, st);
}

extern "C" int pe_propose_tree(const void* logits, int64_t ld, int k, int64_t V, int dtype, const int32_t* widths,
                               int top_k, int64_t* node_tokens, int32_t* parents, int32_t* n_nodes, void* scratch,
                               int32_t* status, void* stream) {
  if (!logits || !widths || !node_tokens || !parents || !n_nodes || !scratch || k < 1 || k > PE_PROPOSE_MAX_DEPTH ||
      V < 1 || V > INT32_MAX || ld < V || top_k < 1)
    return PE_ERR_ARG;
  BeamShape bs{};
  bs.k = k;
  int nb = 1, total = 0;
  for (int d = 0; d < k; ++d) {
    const int w = widths[d];
    if (w < 1 || w > PE_PROPOSE_MAX_WIDTH) return PE_ERR_ARG;
    bs.width[d] = w;
    bs.cand[d] = min(top_k, w);
    if (bs.cand[d] > V) return PE_ERR_ARG;
    nb = min(w, nb * bs.cand[d]);
    total += nb;
  }
  *n_nodes = total;
  float* lp = (float*)scratch;
  int32_t* tok = (int32_t*)((char*)scratch + (size_t)k * PE_PROPOSE_MAX_WIDTH * sizeof(float));
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case PE_DTYPE_F32:
      draft_topk_kernel<PE_DTYPE_F32><<<k, kArgThreads, 0, st>>>((const float*)logits, ld, V, bs, lp, tok, status);
      break;
    case PE_DTYPE_BF16:
      draft_topk_kernel<PE_DTYPE_BF16><<<k, kArgThreads, 0, st>>>((const uint16_t*)logits, ld, V, bs, lp, tok, status);
      break;
    case PE_DTYPE_F16:
      draft_topk_kernel<PE_DTYPE_F16><<<k, kArgThreads, 0, st>>>((const uint16_t*)logits, ld, V, bs, lp, tok, status);
      break;
    default:
      return PE_ERR_ARG;
  }
  PE_CHECK_LAUNCH();
  beam_kernel<<<1, kBeamThreads, 0, st>>>(bs, lp, tok, node_tokens, parents, status);
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
                                                         accept_out, nullptr, 0, 0);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_kv_compact_batch(void* k_cache, void* v_cache, int batch, int64_t cache_seq_stride, int L, int nkv,
                                   int64_t cap, int hd, int dtype, const int64_t* seq_prefix, const int32_t* accept_out,
                                   int max_seq_rows, void* stream) {
  if (!k_cache || !v_cache || !accept_out || !seq_prefix || batch <= 0 || L <= 0 || nkv <= 0 || hd <= 0 ||
      max_seq_rows <= 0)
    return PE_ERR_ARG;
  const int64_t row_bytes = (int64_t)hd * esize(dtype);
  if (row_bytes % 16 || cache_seq_stride < (int64_t)L * nkv * cap * hd) return PE_ERR_ARG;
  dim3 grid(L * nkv, 2, batch);
  kv_compact_kernel<<<grid, 64, 0, (hipStream_t)stream>>>((uint8_t*)k_cache, (uint8_t*)v_cache, cap, row_bytes, 0,
                                                         accept_out, seq_prefix, cache_seq_stride * esize(dtype),
                                                         2 + max_seq_rows);
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
