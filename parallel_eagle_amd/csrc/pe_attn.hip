// Tree-masked GQA attention over the KV cache (split-KV flash decoding).
//
// Query rows are the T tree nodes (x G query heads per KV head); keys are the
// P cached prefix rows followed by the T node rows appended by pe_rope_qkv.
// A node attends to the whole prefix and to the node rows of its ancestor set,
// read from a per-node bitmask (bit u of bits[t] <=> node u is t or an
// ancestor of t), which is the (T, P+T) additive bias of the reference
// (src/pe/masks.py:127-147 + to_additive_bias :29-33) without materialising it.
//
// 16-bit path (hd = 128): one wave per (KV head, key split, 32-row tile).
//   S^T = K Q^T with v_mfma_f32_32x32x16 (A = 32 keys x 16 dims of K straight
//   from the cache, B = Q^T held in registers), so every lane owns one query
//   row (column) and 16 of the 32 keys: the online-softmax max/sum of a row is
//   a 16-value in-lane reduction plus one exchange with lane^32.
//   O^T += V^T P^T (A = V^T from a wave-private LDS transpose of the 32-key V
//   block, B = P^T taken directly from the S^T accumulator registers rounded to
//   the compute dtype), so the per-row rescale is a per-lane scalar.
//   Partial (O, max, sum) per split are merged by attn_combine_kernel.
// Softmax is fp32; exp(s - m) is summed in fp32 and rounded to the compute
// dtype for the PV product, as torch's CPU flash attention does for reduced
// precision inputs.
//
// fp32 path: one block per (row, query head), scores in LDS, VALU arithmetic.

#include "pe_common.h"
#include "pe_internal.h"

namespace {

constexpr float kMaskedScore = -3.0e38f;
constexpr float kInitMax = -2.0e38f;

__device__ __forceinline__ bool key_allowed(int64_t key, int64_t P, int t, int mask_mode, const uint64_t* nb) {
  if (mask_mode == PE_MASK_CAUSAL) return key <= P + t;
  if (key < P) return true;
  const int u = (int)(key - P);
  return (nb[u >> 6] >> (u & 63)) & 1ull;
}

// One workgroup = 4 waves = one (KV head, key split, 32-row tile). Each wave
// takes a contiguous run of the split's 32-key blocks; the next block's K and
// V fragments are loaded as soon as the current ones are consumed (K after the
// S MFMAs, V after its LDS transpose), so the loads overlap softmax and PV.
// Loads are clamped to the wave's last valid key (those scores are masked and
// their probabilities are exactly zero), so no uninitialised cache row is read.
// At the end the 4 waves' (m, l, O) are merged in LDS in wave order and one
// partial per workgroup is written for attn_combine_kernel.
constexpr int kAttnWaves = 4;

template <int DT>
__global__ __launch_bounds__(64 * kAttnWaves) void attn_wg_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t cap,
    int nh, int nkv, int T, int64_t P, int mask_mode, const uint64_t* __restrict__ bits, int words, float scale,
    int keys_per_split, int splits, int rows_pad, float* __restrict__ opart, float* __restrict__ mlpart) {
  constexpr int HD = 128;
  constexpr int kVtBytes = HD * (32 + 8) * 2;
  constexpr int kCmbBytes = (kAttnWaves - 1) * 32 * (HD + 2) * 4;
  constexpr int kSmem = (kAttnWaves * kVtBytes > kCmbBytes) ? kAttnWaves * kVtBytes : kCmbBytes;
  __shared__ __align__(16) uint8_t smem[kSmem];
  const int kvh = blockIdx.x, split = blockIdx.y, rt = blockIdx.z;
  const int G = nh / nkv, rows = T * G;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ln = lane & 31, g = lane >> 5;
  const int64_t S = P + T;
  const int64_t ks0 = (int64_t)split * keys_per_split;
  const int64_t ks1 = min(S, ks0 + keys_per_split);
  const int nb = (int)((ks1 - ks0 + 31) / 32);
  const int b0 = (nb * wave) / kAttnWaves, b1 = (nb * (wave + 1)) / kAttnWaves;
  const int64_t j1 = min(ks1, ks0 + 32 * (int64_t)b1);  // end of this wave's keys
  uint16_t(*vt)[32 + 8] = (uint16_t(*)[32 + 8])(smem + wave * kVtBytes);

  const int r = rt * 32 + ln;
  const bool rvalid = r < rows;
  const int t = rvalid ? r / G : 0;
  const int hq = kvh * G + (rvalid ? r % G : 0);

  uint64_t nbits[PE_TREE_MAX_WORDS];
#pragma unroll
  for (int w = 0; w < PE_TREE_MAX_WORDS; ++w)
    nbits[w] = (mask_mode == PE_MASK_TREE && w < words && rvalid) ? bits[(int64_t)t * words + w] : 0ull;

  const u32x4_t zero4 = {0u, 0u, 0u, 0u};
  u32x4_t qf[8];
  const uint16_t* qp = q + ((int64_t)t * nh + hq) * HD;
#pragma unroll
  for (int j = 0; j < 8; ++j) qf[j] = rvalid ? *(const u32x4_t*)(qp + 16 * j + 8 * g) : zero4;

  f32x16_t o[4];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[h][i] = 0.f;
  float m = kInitMax, l = 0.f;

  const uint16_t* kbase = kc + (int64_t)kvh * cap * HD;
  const uint16_t* vbase = vc + (int64_t)kvh * cap * HD;
  const int64_t jlast = j1 - 1;
  u32x4_t kf[8], vf[8];
  auto load_k = [&](int64_t jb) {
    const uint16_t* kp = kbase + min(jb + ln, jlast) * HD + 8 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) kf[j] = *(const u32x4_t*)(kp + 16 * j);
  };
  auto load_v = [&](int64_t jb) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int chunk = c * 64 + lane;  // 32 keys x 16 chunks of 8 dims
      const int koff = chunk >> 4, dc = chunk & 15;
      vf[c] = *(const u32x4_t*)(vbase + min(jb + koff, jlast) * HD + dc * 8);
    }
  };
  if (b0 < b1) {
    load_k(ks0 + 32 * (int64_t)b0);
    load_v(ks0 + 32 * (int64_t)b0);
  }
  for (int b = b0; b < b1; ++b) {
    const int64_t jb = ks0 + 32 * (int64_t)b;
    const int64_t jnext = ks0 + 32 * (int64_t)min(b + 1, b1 - 1);
    // ---- S^T = K Q^T over hd
    f32x16_t sc;
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (DT == PE_DTYPE_F16)
        sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, kf[j]),
                                                    __builtin_bit_cast(f16x8_t, qf[j]), sc, 0, 0, 0);
      else
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[j]),
                                                     __builtin_bit_cast(bf16x8_t, qf[j]), sc, 0, 0, 0);
    }
    load_k(jnext);
    // ---- scale + mask, block max (sc[i] holds key jb + 8*(i/4) + 4*g + (i%4) of row ln)
    float bmax = kInitMax;
    if (jb + 32 <= min(P, j1) && (mask_mode == PE_MASK_TREE || jb + 32 <= P + 1)) {
      // a whole block of prefix keys: every key is visible to every node
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        sc[i] = rvalid ? sc[i] * scale : kMaskedScore;
        bmax = fmaxf(bmax, sc[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t kj = jb + 8 * (i >> 2) + 4 * g + (i & 3);
        const bool ok = rvalid && kj < j1 && key_allowed(kj, P, t, mask_mode, nbits);
        sc[i] = ok ? sc[i] * scale : kMaskedScore;
        bmax = fmaxf(bmax, sc[i]);
      }
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float mnew = fmaxf(m, bmax);
    const float alpha = expf(m - mnew);
    float psum = 0.f;
    uint32_t pb[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = expf(sc[i] - mnew), p1 = expf(sc[i + 1] - mnew);
      psum += p0 + p1;
      pb[i >> 1] = (DT == PE_DTYPE_F16) ? ((uint32_t)f32_to_f16_bits(p0) | ((uint32_t)f32_to_f16_bits(p1) << 16))
                                        : ((uint32_t)f32_to_bf16_bits(p0) | ((uint32_t)f32_to_bf16_bits(p1) << 16));
    }
    psum += __shfl_xor(psum, 32, 64);
    l = l * alpha + psum;
    // rescale O only if some row's running max moved (alpha == 1 leaves O as is)
    const bool rescale = __builtin_amdgcn_ballot_w64(mnew != m) != 0ull;
    m = mnew;
    if (rescale) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[h][i] *= alpha;
    }

    // ---- V^T into LDS, then the next block's V
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int chunk = c * 64 + lane;
      const int koff = chunk >> 4, dc = chunk & 15;
      const uint16_t* ve = (const uint16_t*)&vf[c];
#pragma unroll
      for (int e = 0; e < 8; ++e) vt[dc * 8 + e][koff] = ve[e];
    }
    load_v(jnext);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- O^T += V^T P^T: two 16-key halves c; lane group g holds keys 16c+4g+{0..3}, 16c+8+4g+{0..3}
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      u32x4_t bp;
      bp[0] = pb[4 * c + 0];
      bp[1] = pb[4 * c + 1];
      bp[2] = pb[4 * c + 2];
      bp[3] = pb[4 * c + 3];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int d = h * 32 + ln;
        const uint2 lo = *(const uint2*)&vt[d][16 * c + 4 * g];
        const uint2 hi = *(const uint2*)&vt[d][16 * c + 8 + 4 * g];
        u32x4_t a;
        a[0] = lo.x;
        a[1] = lo.y;
        a[2] = hi.x;
        a[3] = hi.y;
        if constexpr (DT == PE_DTYPE_F16)
          o[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                        __builtin_bit_cast(f16x8_t, bp), o[h], 0, 0, 0);
        else
          o[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                         __builtin_bit_cast(bf16x8_t, bp), o[h], 0, 0, 0);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- merge the waves: (m, l, O) of waves 1..3 through LDS, wave 0 sums in wave order
  __syncthreads();
  float* cmb = (float*)smem;
  if (wave > 0) {
    float* cw = cmb + (int64_t)(wave - 1) * 32 * (HD + 2);
    if (g == 0) {
      cw[ln * (HD + 2) + HD] = m;
      cw[ln * (HD + 2) + HD + 1] = l;
    }
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int i = 0; i < 16; ++i) cw[ln * (HD + 2) + h * 32 + 8 * (i >> 2) + 4 * g + (i & 3)] = o[h][i];
  }
  __syncthreads();
  if (wave != 0 || !rvalid) return;
  float mw[kAttnWaves], wt[kAttnWaves];
  mw[0] = m;
  float M = m;
#pragma unroll
  for (int w = 1; w < kAttnWaves; ++w) {
    mw[w] = cmb[(int64_t)(w - 1) * 32 * (HD + 2) + ln * (HD + 2) + HD];
    M = fmaxf(M, mw[w]);
  }
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) {
    wt[w] = expf(mw[w] - M);
    const float lw = (w == 0) ? l : cmb[(int64_t)(w - 1) * 32 * (HD + 2) + ln * (HD + 2) + HD + 1];
    L += wt[w] * lw;
  }
  const int64_t pidx = ((int64_t)kvh * splits + split) * rows_pad + r;
  float* op = opart + pidx * HD;
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = h * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
      float v = wt[0] * o[h][i];
#pragma unroll
      for (int w = 1; w < kAttnWaves; ++w) v += wt[w] * cmb[(int64_t)(w - 1) * 32 * (HD + 2) + ln * (HD + 2) + d];
      op[d] = v;
    }
  if (g == 0) {
    mlpart[pidx * 2 + 0] = M;
    mlpart[pidx * 2 + 1] = L;
  }
}

// out[t][hq*hd + d] = sum_s e^{m_s - M} O_s[d] / sum_s e^{m_s - M} l_s
template <int DT>
__global__ __launch_bounds__(128) void attn_combine_kernel(const float* __restrict__ opart,
                                                           const float* __restrict__ mlpart, int nh, int nkv, int T,
                                                           int hd, int splits, int rows_pad,
                                                           typename Elem<DT>::T* __restrict__ out, int64_t ld_out,
                                                           int out_units) {
  const int r = blockIdx.x, kvh = blockIdx.y;
  const int G = nh / nkv;
  const int t = r / G, hq = kvh * G + r % G;
  float M = kInitMax;
  for (int s = 0; s < splits; ++s) M = fmaxf(M, mlpart[(((int64_t)kvh * splits + s) * rows_pad + r) * 2]);
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float num = 0.f, den = 0.f;
    for (int s = 0; s < splits; ++s) {
      const int64_t pidx = ((int64_t)kvh * splits + s) * rows_pad + r;
      const float w = expf(mlpart[pidx * 2] - M);
      den += w * mlpart[pidx * 2 + 1];
      num += w * opart[pidx * hd + d];
    }
    const int col = hq * hd + d;
    Elem<DT>::store(out, out_units ? xtile_index(t, col, out_units) : (int64_t)t * ld_out + col, num / den);
  }
}

// Generic path (fp32, any hd <= 256): one block per (row t, query head), all keys.
template <int DT>
__global__ __launch_bounds__(128) void attn_generic_kernel(
    const typename Elem<DT>::T* __restrict__ q, const typename Elem<DT>::T* __restrict__ kc,
    const typename Elem<DT>::T* __restrict__ vc, int64_t cap, int nh, int nkv, int hd, int T, int64_t P,
    int mask_mode, const uint64_t* __restrict__ bits, int words, float scale, typename Elem<DT>::T* __restrict__ out,
    int64_t ld_out, float* __restrict__ scores /* [T*nh][P+T] */) {
  typedef Elem<DT> E;
  const int t = blockIdx.x, hq = blockIdx.y;
  const int G = nh / nkv, kvh = hq / G;
  const int64_t S = P + T;
  uint64_t nb[PE_TREE_MAX_WORDS];
  for (int w = 0; w < PE_TREE_MAX_WORDS; ++w)
    nb[w] = (mask_mode == PE_MASK_TREE && w < words) ? bits[(int64_t)t * words + w] : 0ull;
  const typename E::T* qr = q + ((int64_t)t * nh + hq) * hd;
  float* sc = scores + ((int64_t)t * nh + hq) * S;
  __shared__ float red[2];
  float lmax = kInitMax;
  for (int64_t j = threadIdx.x; j < S; j += blockDim.x) {
    float v = kMaskedScore;
    if (key_allowed(j, P, t, mask_mode, nb)) {
      const typename E::T* kr = kc + ((int64_t)kvh * cap + j) * hd;
      float acc = 0.f;
      for (int d = 0; d < hd; ++d) acc = fmaf(E::load(qr, d), E::load(kr, d), acc);
      v = acc * scale;
    }
    sc[j] = v;
    lmax = fmaxf(lmax, v);
  }
  lmax = wave_max(lmax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = lmax;
  __syncthreads();
  const float M = fmaxf(red[0], red[1]);
  __syncthreads();
  float lsum = 0.f;
  for (int64_t j = threadIdx.x; j < S; j += blockDim.x) {
    const float p = expf(sc[j] - M);
    sc[j] = p;
    lsum += p;
  }
  lsum = wave_sum(lsum);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = lsum;
  __syncthreads();
  const float L = red[0] + red[1];
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.f;
    for (int64_t j = 0; j < S; ++j) {
      const float p = sc[j];
      if (p != 0.f) acc = fmaf(E::round(p), E::load(vc + ((int64_t)kvh * cap + j) * hd, d), acc);
    }
    E::store(out, (int64_t)t * ld_out + (int64_t)hq * hd + d, acc / L);
  }
}

struct AttnPlan {
  int splits, keys_per_split, row_tiles, rows_pad;
  int64_t opart_bytes, ml_bytes;
};

AttnPlan attn_plan(int T, int nh, int nkv, int64_t S) {
  AttnPlan p;
  const int rows = T * (nh / nkv);
  p.row_tiles = (rows + 31) / 32;
  p.rows_pad = p.row_tiles * 32;
  // about one workgroup per CU, each with at least two 32-key blocks per wave
  int64_t want = (256 + (int64_t)nkv * p.row_tiles - 1) / ((int64_t)nkv * p.row_tiles);
  int64_t maxsplit = (S + 32 * 2 * kAttnWaves - 1) / (32 * 2 * kAttnWaves);
  if (want > maxsplit) want = maxsplit;
  if (want < 1) want = 1;
  int64_t kps = (S + want - 1) / want;
  kps = ((kps + 31) / 32) * 32;
  p.keys_per_split = (int)kps;
  p.splits = (int)((S + kps - 1) / kps);
  p.opart_bytes = (int64_t)nkv * p.splits * p.rows_pad * 128 * 4;
  p.ml_bytes = (int64_t)nkv * p.splits * p.rows_pad * 2 * 4;
  return p;
}

}  // namespace

extern "C" int64_t pe_attention_workspace_bytes(int T, int nh, int nkv, int hd, int64_t kv_len, int dtype) {
  if (T <= 0 || nh <= 0 || nkv <= 0 || kv_len <= 0) return 0;
  if (dtype != PE_DTYPE_F32 && hd == 128) {
    AttnPlan p = attn_plan(T, nh, nkv, kv_len);
    return p.opart_bytes + p.ml_bytes;
  }
  return (int64_t)T * nh * kv_len * 4;
}

int pe_internal_tree_attention(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap, int nh,
                               int nkv, int hd, int T, int64_t P, int mask_mode, const uint64_t* bits, int words,
                               float scale, int dtype, void* out, int64_t ld_out, int out_units, void* workspace,
                               int64_t workspace_bytes, hipStream_t st) {
  if (!q || !k_cache || !v_cache || !out || !workspace) return PE_ERR_ARG;
  if (out_units && (dtype == PE_DTYPE_F32 || hd != 128 || T > 64 || out_units * 128 != nh * hd)) return PE_ERR_ARG;
  if (T <= 0 || nh <= 0 || nkv <= 0 || nh % nkv || hd <= 0 || hd > 256 || P < 0) return PE_ERR_ARG;
  if (P + T > cache_cap) return PE_ERR_CAPACITY;
  if (mask_mode != PE_MASK_TREE && mask_mode != PE_MASK_CAUSAL) return PE_ERR_ARG;
  if (mask_mode == PE_MASK_TREE && (!bits || words <= 0 || words > PE_TREE_MAX_WORDS || T > 64 * words))
    return PE_ERR_TREE;
  const int64_t S = P + T;
  if (workspace_bytes < pe_attention_workspace_bytes(T, nh, nkv, hd, S, dtype)) return PE_ERR_WORKSPACE;
  if (dtype != PE_DTYPE_F32 && hd == 128) {
    AttnPlan p = attn_plan(T, nh, nkv, S);
    float* opart = (float*)workspace;
    float* ml = (float*)((char*)workspace + p.opart_bytes);
    dim3 grid(nkv, p.splits, p.row_tiles);
    dim3 cgrid(T * (nh / nkv), nkv);
    if (dtype == PE_DTYPE_BF16) {
      attn_wg_kernel<PE_DTYPE_BF16><<<grid, 64 * kAttnWaves, 0, st>>>((const uint16_t*)q, (const uint16_t*)k_cache,
                                                           (const uint16_t*)v_cache, cache_cap, nh, nkv, T, P,
                                                           mask_mode, bits, words, scale, p.keys_per_split,
                                                           p.splits, p.rows_pad, opart, ml);
      PE_CHECK_LAUNCH();
      attn_combine_kernel<PE_DTYPE_BF16><<<cgrid, 128, 0, st>>>(opart, ml, nh, nkv, T, hd, p.splits, p.rows_pad,
                                                                (uint16_t*)out, ld_out, out_units);
    } else if (dtype == PE_DTYPE_F16) {
      attn_wg_kernel<PE_DTYPE_F16><<<grid, 64 * kAttnWaves, 0, st>>>((const uint16_t*)q, (const uint16_t*)k_cache,
                                                          (const uint16_t*)v_cache, cache_cap, nh, nkv, T, P,
                                                          mask_mode, bits, words, scale, p.keys_per_split, p.splits,
                                                          p.rows_pad, opart, ml);
      PE_CHECK_LAUNCH();
      attn_combine_kernel<PE_DTYPE_F16><<<cgrid, 128, 0, st>>>(opart, ml, nh, nkv, T, hd, p.splits, p.rows_pad,
                                                               (uint16_t*)out, ld_out, out_units);
    } else {
      return PE_ERR_ARG;
    }
    PE_CHECK_LAUNCH();
    return PE_OK;
  }
  dim3 grid(T, nh);
  float* scores = (float*)workspace;
  switch (dtype) {
    case PE_DTYPE_F32:
      attn_generic_kernel<PE_DTYPE_F32><<<grid, 128, 0, st>>>((const float*)q, (const float*)k_cache,
                                                              (const float*)v_cache, cache_cap, nh, nkv, hd, T, P,
                                                              mask_mode, bits, words, scale, (float*)out, ld_out,
                                                              scores);
      break;
    case PE_DTYPE_BF16:
      attn_generic_kernel<PE_DTYPE_BF16><<<grid, 128, 0, st>>>((const uint16_t*)q, (const uint16_t*)k_cache,
                                                               (const uint16_t*)v_cache, cache_cap, nh, nkv, hd, T,
                                                               P, mask_mode, bits, words, scale, (uint16_t*)out,
                                                               ld_out, scores);
      break;
    case PE_DTYPE_F16:
      attn_generic_kernel<PE_DTYPE_F16><<<grid, 128, 0, st>>>((const uint16_t*)q, (const uint16_t*)k_cache,
                                                              (const uint16_t*)v_cache, cache_cap, nh, nkv, hd, T, P,
                                                              mask_mode, bits, words, scale, (uint16_t*)out, ld_out,
                                                              scores);
      break;
    default:
      return PE_ERR_ARG;
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_tree_attention(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap, int nh,
                                 int nkv, int hd, int T, int64_t P, int mask_mode, const uint64_t* bits, int words,
                                 float scale, int dtype, void* out, int64_t ld_out, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  return pe_internal_tree_attention(q, k_cache, v_cache, cache_cap, nh, nkv, hd, T, P, mask_mode, bits, words, scale,
                                    dtype, out, ld_out, 0, workspace, workspace_bytes, (hipStream_t)stream);
}
