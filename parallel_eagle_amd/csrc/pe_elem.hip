// Row-wise ops of the decoder layer: token embedding, RMSNorm, RoPE with the
// in-place KV append, and row copies for the fused features.
//
// Rounding mirrors HF Llama/Qwen2 in the compute dtype: RMSNorm statistics in
// fp32, the normalised row rounded to the dtype before the weight multiply
// (HF modeling_llama.py:62-67); RoPE as round(round(q*cos) + round(rot(q)*sin))
// (modeling_llama.py:130-160). fp32 arithmetic uses __fmul_rn/__fadd_rn so no
// multiply-add is contracted where torch rounds between the two.

#include "pe_common.h"
#include "pe_internal.h"

namespace {

// One block per row; 16-byte pieces, all of a thread's loads issued before its
// stores (rows of the table are random HBM reads).
template <int DT>
__global__ __launch_bounds__(256) void embed_kernel(const int64_t* __restrict__ ids, const typename Elem<DT>::T* __restrict__ table,
                                                    int64_t V, int H, typename Elem<DT>::T* __restrict__ out,
                                                    int64_t ld_out, int32_t* status) {
  typedef typename Elem<DT>::T T;
  const int m = blockIdx.x;
  const int64_t id = ids[m];
  const bool ok = id >= 0 && id < V;
  if (!ok && threadIdx.x == 0 && status) atomicOr(status, PE_ERR_TOKEN);
  const int64_t row_bytes = (int64_t)H * sizeof(T);
  const uint8_t* src = (const uint8_t*)(table + (ok ? id : 0) * H);
  uint8_t* dst = (uint8_t*)(out + (int64_t)m * ld_out);
  if ((row_bytes & 15) == 0 && (((uintptr_t)src | (uintptr_t)dst) & 15) == 0) {
    const int nvec = (int)(row_bytes >> 4);
    constexpr int kU = 4;
    for (int i0 = threadIdx.x; i0 < nvec; i0 += kU * 256) {
      uint4 t[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = i0 + u * 256;
        t[u] = i < nvec ? ((const uint4*)src)[i] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = i0 + u * 256;
        if (i < nvec) ((uint4*)dst)[i] = ok ? t[u] : make_uint4(0, 0, 0, 0);
      }
    }
  } else {
    for (int c = threadIdx.x; c < H; c += blockDim.x)
      out[(int64_t)m * ld_out + c] = ok ? table[id * H + c] : (T)0;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const typename Elem<DT>::T* __restrict__ x, int64_t ldx, int H,
                                                      const typename Elem<DT>::T* __restrict__ w, float eps,
                                                      int mode, typename Elem<DT>::T* __restrict__ out,
                                                      int64_t ld_out) {
  typedef Elem<DT> E;
  const int m = blockIdx.x;
  const typename E::T* xr = x + (int64_t)m * ldx;
  float ss = 0.f;
  for (int c = threadIdx.x; c < H; c += blockDim.x) {
    const float v = E::load(xr, c);
    ss = __fadd_rn(ss, __fmul_rn(v, v));
  }
  __shared__ float part[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const int nw = blockDim.x >> 6;
  float tot = 0.f;
  for (int i = 0; i < nw; ++i) tot += part[i];
  const float var = tot / (float)H;
  const float inv = 1.0f / sqrtf(var + eps);
  typename E::T* orow = out + (int64_t)m * ld_out;
  for (int c = threadIdx.x; c < H; c += blockDim.x) {
    E::store(orow, c, norm_out<E>(mode, E::load(xr, c), inv, E::load(w, c)));
  }
}

// One block per row m; threads over (head, d < hd/2) pairs of q and k, then v copies.
template <int DT>
__global__ __launch_bounds__(256) void rope_qkv_kernel(const typename Elem<DT>::T* __restrict__ qkv, int64_t ld_qkv, int nh,
                                                       int nkv, int hd, const int64_t* __restrict__ pos,
                                                       const typename Elem<DT>::T* __restrict__ cs, int64_t max_pos,
                                                       typename Elem<DT>::T* __restrict__ q_out,
                                                       typename Elem<DT>::T* __restrict__ kc,
                                                       typename Elem<DT>::T* __restrict__ vc, int64_t cap,
                                                       int64_t row0, int32_t* status) {
  typedef Elem<DT> E;
  const int m = blockIdx.x;
  const int64_t p = pos[m];
  const bool ok = p >= 0 && p < max_pos;
  if (!ok) {
    if (threadIdx.x == 0 && status) atomicOr(status, PE_ERR_CAPACITY);
    return;
  }
  const int half = hd >> 1;
  const typename E::T* cosr = cs + p * hd;
  const typename E::T* sinr = cs + (max_pos + p) * hd;
  const typename E::T* row = qkv + (int64_t)m * ld_qkv;
  const int64_t dst_row = row0 + m;
  const int nq = nh * half, nk = nkv * half;
  for (int i = threadIdx.x; i < nq + nk; i += blockDim.x) {
    const bool is_q = i < nq;
    const int ii = is_q ? i : i - nq;
    const int h = ii / half, d = ii % half;
    const typename E::T* src = row + (is_q ? h * hd : nh * hd + h * hd);
    const float x1 = E::load(src, d), x2 = E::load(src, d + half);
    const float c1 = E::load(cosr, d), s1 = E::load(sinr, d);
    const float c2 = E::load(cosr, d + half), s2 = E::load(sinr, d + half);
    const float o1 = __fadd_rn(E::round(__fmul_rn(x1, c1)), E::round(__fmul_rn(-x2, s1)));
    const float o2 = __fadd_rn(E::round(__fmul_rn(x2, c2)), E::round(__fmul_rn(x1, s2)));
    if (is_q) {
      typename E::T* dst = q_out + ((int64_t)m * nh + h) * hd;
      E::store(dst, d, o1);
      E::store(dst, d + half, o2);
    } else {
      typename E::T* dst = kc + ((int64_t)h * cap + dst_row) * hd;
      E::store(dst, d, o1);
      E::store(dst, d + half, o2);
    }
  }
  const typename E::T* vsrc = row + (nh + nkv) * hd;
  for (int i = threadIdx.x; i < nkv * hd; i += blockDim.x) {
    const int h = i / hd, d = i % hd;
    vc[((int64_t)h * cap + dst_row) * hd + d] = vsrc[h * hd + d];
  }
}

// One block per row: the residual add of a split-K projection (partials summed
// in split order, HF modeling_llama.py:317,323) fused with the RMSNorm that
// follows it (modeling_llama.py:62-67) and the hidden-state captures. Each
// thread owns CH chunks of 4 columns. Every load of the row (the residual, the
// norm weight and the S split partials of the thread's chunks) is issued
// before the first use, so the row costs one memory round trip; the partial
// loads past S repeat split S - 1 (SMAX is S rounded up to a multiple of 4)
// and are not summed. With two chunks and more than eight splits the second
// chunk's partials are requested after the first chunk is summed.
constexpr int kNormThreads = 1024;
constexpr int kNormChunks = 2;    // H <= 4 * 1024 * 2
constexpr int kNormMaxSplits = 16;

// four consecutive elements as one raw access (8 bytes for the 16-bit types)
template <int DT> struct Raw4 {
  typedef uint2 R;
  static __device__ __forceinline__ R load(const uint16_t* p) { return *(const uint2*)p; }
  static __device__ __forceinline__ void cvt(R t, float (&v)[4]) {
    v[0] = Vec4Half<DT>::cvt(t.x & 0xffffu);
    v[1] = Vec4Half<DT>::cvt(t.x >> 16);
    v[2] = Vec4Half<DT>::cvt(t.y & 0xffffu);
    v[3] = Vec4Half<DT>::cvt(t.y >> 16);
  }
};
template <> struct Raw4<PE_DTYPE_F32> {
  typedef float4 R;
  static __device__ __forceinline__ R load(const float* p) { return *(const float4*)p; }
  static __device__ __forceinline__ void cvt(R t, float (&v)[4]) {
    v[0] = t.x;
    v[1] = t.y;
    v[2] = t.z;
    v[3] = t.w;
  }
};

// EMB: the row is the embedding of token ids[m] (HF modeling_llama.py:381;
// out-of-range ids flag PE_ERR_TOKEN and read row 0) and is stored to h; the
// first layer's input norm then needs no separate embedding launch.
template <int DT, int CH, int SMAX, bool EMB>
__global__ __launch_bounds__(kNormThreads) void residual_rmsnorm_kernel(
    const float* __restrict__ partial, int S, int M, typename Elem<DT>::T* __restrict__ h, int H,
    const typename Elem<DT>::T* __restrict__ w, float eps, int mode, typename Elem<DT>::T* __restrict__ xn,
    typename Elem<DT>::T* __restrict__ xt, typename Elem<DT>::T* __restrict__ cap_h, int64_t ld_cap_h,
    typename Elem<DT>::T* __restrict__ cap_xn, int64_t ld_cap_xn, const int64_t* __restrict__ ids,
    const typename Elem<DT>::T* __restrict__ table, int64_t vocab, int32_t* __restrict__ status) {
  typedef Elem<DT> E;
  typedef typename E::T T;
  typedef Vec4<DT> V;
  typedef Raw4<DT> RW;
  constexpr int PCH = (CH * SMAX <= 16) ? CH : 1;  // chunks whose partials are in flight together
  const int m = blockIdx.x;
  T* hr = h + (int64_t)m * H;
  const T* src = hr;
  if constexpr (EMB) {
    const int64_t id = ids[m];
    const bool ok = id >= 0 && id < vocab;
    if (!ok && threadIdx.x == 0 && status) atomicOr(status, PE_ERR_TOKEN);
    src = table + (ok ? id : 0) * H;
  }
  const int nchunk = H >> 2;
  const int64_t sstride = (int64_t)M * H;
  // chunk k of this thread (clamped to the last chunk; a clamped chunk is
  // loaded but neither summed nor stored)
  auto chunk = [&](int k) { return min((int)threadIdx.x + k * kNormThreads, nchunk - 1); };
  typename RW::R hraw[CH], wraw[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    hraw[k] = RW::load(src + 4 * chunk(k));
    wraw[k] = RW::load(w + 4 * chunk(k));
  }
  float v[CH][4];
#pragma unroll
  for (int k0 = 0; k0 < CH; k0 += PCH) {
    f32x4_t pt[PCH][SMAX > 0 ? SMAX : 1];
#pragma unroll
    for (int kk = 0; kk < PCH; ++kk)
#pragma unroll
      for (int sp = 0; sp < SMAX; ++sp)
        pt[kk][sp] = *(const f32x4_t*)(partial + (int64_t)m * H + 4 * chunk(k0 + kk) + min(sp, S - 1) * sstride);
    __builtin_amdgcn_sched_barrier(0);  // all of the batch's loads issue before the sums
#pragma unroll
    for (int kk = 0; kk < PCH; ++kk) {
      const int k = k0 + kk;
      RW::cvt(hraw[k], v[k]);
      if (SMAX > 0) {
        float a[4] = {0.f, 0.f, 0.f, 0.f};
        // a select, not an early exit: every partial load stays ahead of the sum
#pragma unroll
        for (int sp = 0; sp < SMAX; ++sp)
#pragma unroll
          for (int e = 0; e < 4; ++e) a[e] = sp < S ? a[e] + pt[kk][sp][e] : a[e];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[k][e] = E::round(__fadd_rn(v[k][e], E::round(a[e])));
      }
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = threadIdx.x + k * kNormThreads;
    if (c >= nchunk) continue;
    if (SMAX > 0 || EMB) V::store(hr + 4 * c, v[k]);
    if (cap_h) V::store(cap_h + (int64_t)m * ld_cap_h + 4 * c, v[k]);
#pragma unroll
    for (int e = 0; e < 4; ++e) ss = __fadd_rn(ss, __fmul_rn(v[k][e], v[k][e]));
  }
  __shared__ float part[kNormThreads / 64];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
  T* orow = xn ? xn + (int64_t)m * H : nullptr;  // null: the A-tiled rows only
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = threadIdx.x + k * kNormThreads;
    if (c >= nchunk) continue;
    float wv[4], o[4];
    RW::cvt(wraw[k], wv);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = norm_out<E>(mode, v[k][e], inv, wv[e]);
    if (orow) V::store(orow + 4 * c, o);
    // four consecutive columns are consecutive in the A-tiled layout too
    if (xt) V::store(xt + xtile_index(m, 4 * c, H >> 7), o);
    if (cap_xn) V::store(cap_xn + (int64_t)m * ld_cap_xn + 4 * c, o);
  }
}

__global__ void copy_rows_kernel(const uint8_t* __restrict__ src, int64_t ld_src, int64_t row_bytes,
                                 uint8_t* __restrict__ dst, int64_t ld_dst) {
  const int m = blockIdx.x;
  const uint8_t* s = src + (int64_t)m * ld_src;
  uint8_t* d = dst + (int64_t)m * ld_dst;
  if ((row_bytes & 3) == 0 && (((uintptr_t)s | (uintptr_t)d) & 3) == 0) {
    for (int64_t i = threadIdx.x; i < row_bytes / 4; i += blockDim.x)
      ((uint32_t*)d)[i] = ((const uint32_t*)s)[i];
  } else {
    for (int64_t i = threadIdx.x; i < row_bytes; i += blockDim.x) d[i] = s[i];
  }
}

}  // namespace

#define PE_DISPATCH_DT(dtype, ...)                               \
  switch (dtype) {                                               \
    case PE_DTYPE_F32: { constexpr int DT = PE_DTYPE_F32; __VA_ARGS__; } break;  \
    case PE_DTYPE_BF16: { constexpr int DT = PE_DTYPE_BF16; __VA_ARGS__; } break; \
    case PE_DTYPE_F16: { constexpr int DT = PE_DTYPE_F16; __VA_ARGS__; } break;   \
    default: return PE_ERR_ARG;                                  \
  }

extern "C" int pe_embed(const int64_t* ids, int M, const void* table, int64_t V, int H, int dtype, void* out,
                        int64_t ld_out, int32_t* status, void* stream) {
  if (!ids || !table || !out || M <= 0 || V <= 0 || H <= 0) return PE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  PE_DISPATCH_DT(dtype, {
    typedef typename Elem<DT>::T T;
    embed_kernel<DT><<<M, 256, 0, st>>>(ids, (const T*)table, V, H, (T*)out, ld_out, status);
  });
  PE_CHECK_LAUNCH();
  return PE_OK;
}

__global__ void kv_offsets_kernel(const int32_t* __restrict__ seq_row0, const int64_t* __restrict__ seq_prefix,
                                  int batch, int M, int64_t seq_stride, int64_t cap, int hd, int64_t max_prefix,
                                  int max_rows, int64_t* __restrict__ off, int32_t* status) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= M) return;
  int b = 0;
  while (b + 1 < batch && seq_row0[b + 1] <= r) ++b;
  const int64_t pre = seq_prefix[b];
  const int rows = seq_row0[b + 1] - seq_row0[b];
  const int64_t slot = pre + (r - seq_row0[b]);
  // the launches were sized for prefixes up to max_prefix and max_rows rows
  // per sequence: a sequence beyond either is not appended (and attention
  // skips it)
  const bool fits = pre >= 0 && pre <= max_prefix && rows <= max_rows;
  const bool ok = fits && r >= seq_row0[b] && r < seq_row0[b + 1] && slot < cap;
  if (!ok && status) atomicOr(status, rows > max_rows ? PE_ERR_TREE : PE_ERR_CAPACITY);
  off[r] = ok ? b * seq_stride + slot * hd : -1;
}

// One thread per 8 consecutive columns of a row: 16 bytes that are 16
// contiguous bytes in the A-tiled layout as well.
__global__ void to_xtile_kernel(const uint16_t* __restrict__ x, int64_t ld, int M, int K, int rows_pad,
                                uint16_t* __restrict__ out, int vec) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int chunks = K >> 3;
  if (i >= (int64_t)rows_pad * chunks) return;
  const int r = (int)(i / chunks), c = (int)(i % chunks) * 8;
  uint16_t* d = out + xtile_index(r, c, K >> 7);
  if (r >= M) {  // the last tile's padding rows: zeros
    *(uint4*)d = uint4{0u, 0u, 0u, 0u};
    return;
  }
  const uint16_t* sp = x + (int64_t)r * ld + c;
  if (vec) {
    *(uint4*)d = *(const uint4*)sp;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = sp[e];
  }
}

int pe_internal_to_xtile(const void* x, int64_t ld, int M, int K, void* out, hipStream_t st) {
  if (!x || !out || M <= 0 || K <= 0 || K % 128 || ld < K) return PE_ERR_ARG;
  const int rows_pad = (M + 31) / 32 * 32;
  const int64_t n = (int64_t)rows_pad * (K / 8);
  const int vec = ((((uintptr_t)x) | (uintptr_t)(ld * 2)) & 15) == 0;
  to_xtile_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>((const uint16_t*)x, ld, M, K, rows_pad,
                                                                (uint16_t*)out, vec);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

// The sequence table of a batch of one: rows [0, M) over a prefix of P rows.
__global__ void one_sequence_kernel(int32_t* seq_row0, int64_t* seq_prefix, int M, int64_t P) {
  seq_row0[0] = 0;
  seq_row0[1] = M;
  seq_prefix[0] = P;
}

int pe_internal_one_sequence(int32_t* seq_row0, int64_t* seq_prefix, int M, int64_t P, hipStream_t st) {
  if (!seq_row0 || !seq_prefix || M <= 0 || P < 0) return PE_ERR_ARG;
  one_sequence_kernel<<<1, 1, 0, st>>>(seq_row0, seq_prefix, M, P);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

int pe_internal_kv_offsets(const int32_t* seq_row0, const int64_t* seq_prefix, int batch, int M, int64_t seq_stride,
                           int64_t cap, int hd, int64_t max_prefix, int max_rows, int64_t* off, int32_t* status,
                           hipStream_t st) {
  if (!seq_row0 || !seq_prefix || !off || batch <= 0 || M <= 0) return PE_ERR_ARG;
  kv_offsets_kernel<<<(M + 255) / 256, 256, 0, st>>>(seq_row0, seq_prefix, batch, M, seq_stride, cap, hd, max_prefix,
                                                     max_rows, off, status);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_rmsnorm_ex(const void* x, int64_t ldx, int M, int H, const void* w, float eps, int dtype, int mode,
                             void* out, int64_t ld_out, void* stream) {
  if (!x || !w || !out || M <= 0 || H <= 0) return PE_ERR_ARG;
  if (mode != PE_NORM_HF && mode != PE_NORM_FP32_WEIGHT) return PE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  PE_DISPATCH_DT(dtype, {
    typedef typename Elem<DT>::T T;
    rmsnorm_kernel<DT><<<M, 256, 0, st>>>((const T*)x, ldx, H, (const T*)w, eps, mode, (T*)out, ld_out);
  });
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_rmsnorm(const void* x, int64_t ldx, int M, int H, const void* w, float eps, int dtype,
                          void* out, int64_t ld_out, void* stream) {
  return pe_rmsnorm_ex(x, ldx, M, H, w, eps, dtype, PE_NORM_HF, out, ld_out, stream);
}

extern "C" int pe_rope_qkv(const void* qkv, int64_t ld_qkv, int M, int nh, int nkv, int hd,
                           const int64_t* positions, const void* cos_sin, int64_t max_pos, int dtype,
                           void* q_out, void* k_cache, void* v_cache, int64_t cache_cap, int64_t row0,
                           int32_t* status, void* stream) {
  if (!qkv || !positions || !cos_sin || !q_out || !k_cache || !v_cache) return PE_ERR_ARG;
  if (M <= 0 || nh <= 0 || nkv <= 0 || nh % nkv || hd <= 0 || hd % 2 || row0 < 0) return PE_ERR_ARG;
  if (row0 + M > cache_cap) return PE_ERR_CAPACITY;
  hipStream_t st = (hipStream_t)stream;
  PE_DISPATCH_DT(dtype, {
    typedef typename Elem<DT>::T T;
    rope_qkv_kernel<DT><<<M, 256, 0, st>>>((const T*)qkv, ld_qkv, nh, nkv, hd, positions, (const T*)cos_sin,
                                           max_pos, (T*)q_out, (T*)k_cache, (T*)v_cache, cache_cap, row0,
                                           status);
  });
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_copy_rows(const void* src, int64_t ld_src, int M, int64_t row_bytes, void* dst, int64_t ld_dst,
                            void* stream) {
  if (!src || !dst || M < 0 || row_bytes < 0) return PE_ERR_ARG;
  if (M == 0 || row_bytes == 0) return PE_OK;
  copy_rows_kernel<<<M, 256, 0, (hipStream_t)stream>>>((const uint8_t*)src, ld_src, row_bytes, (uint8_t*)dst,
                                                       ld_dst);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

template <typename T> struct NormArgs {
  const float* partial;
  int S, M;
  T* h;
  int H;
  const T* w;
  float eps;
  int mode;
  T *xn, *xt, *cap_h;
  int64_t ld_cap_h;
  T* cap_xn;
  int64_t ld_cap_xn;
  const int64_t* ids;
  const T* table;
  int64_t vocab;
  int32_t* status;
};

template <int DT, int CH, int SM>
void launch_norm_sm(const NormArgs<typename Elem<DT>::T>& a, hipStream_t st) {
  if constexpr (SM == 0) {
    if (a.table) {
      residual_rmsnorm_kernel<DT, CH, 0, true><<<a.M, kNormThreads, 0, st>>>(
          a.partial, a.S, a.M, a.h, a.H, a.w, a.eps, a.mode, a.xn, a.xt, a.cap_h, a.ld_cap_h, a.cap_xn, a.ld_cap_xn, a.ids,
          a.table, a.vocab, a.status);
      return;
    }
  }
  residual_rmsnorm_kernel<DT, CH, SM, false><<<a.M, kNormThreads, 0, st>>>(
      a.partial, a.S, a.M, a.h, a.H, a.w, a.eps, a.mode, a.xn, a.xt, a.cap_h, a.ld_cap_h, a.cap_xn, a.ld_cap_xn, nullptr,
      nullptr, 0, nullptr);
}

template <int DT, int CH>
void launch_norm(int smax, const NormArgs<typename Elem<DT>::T>& a, hipStream_t st) {
  switch (smax) {
    case 0: launch_norm_sm<DT, CH, 0>(a, st); break;
    case 4: launch_norm_sm<DT, CH, 4>(a, st); break;
    case 8: launch_norm_sm<DT, CH, 8>(a, st); break;
    case 12: launch_norm_sm<DT, CH, 12>(a, st); break;
    default: launch_norm_sm<DT, CH, 16>(a, st); break;
  }
}

int pe_internal_residual_rmsnorm(const float* partial, int S, int M, void* h, int H, const void* w, float eps,
                                 int mode, int dtype, void* xn, void* xn_tiled, void* cap_h, int64_t ld_cap_h, void* cap_xn,
                                 int64_t ld_cap_xn, hipStream_t st) {
  if (!h || !w || !(xn || xn_tiled) || M <= 0 || H <= 0 || S < 0 || (S > 0 && !partial)) return PE_ERR_ARG;
  if (H % 4 || H > 4 * kNormThreads * kNormChunks || S > kNormMaxSplits) return PE_ERR_ARG;
  if (xn_tiled && (H % 128 || dtype == PE_DTYPE_F32)) return PE_ERR_ARG;
  const int ch = (H >> 2) > kNormThreads ? 2 : 1;
  const int smax = S == 0 ? 0 : (S + 3) / 4 * 4;
  PE_DISPATCH_DT(dtype, {
    typedef typename Elem<DT>::T T;
    const NormArgs<T> na{partial, S, M, (T*)h, H, (const T*)w, eps, mode, (T*)xn, (T*)xn_tiled, (T*)cap_h, ld_cap_h,
                         (T*)cap_xn, ld_cap_xn, nullptr, nullptr, 0, nullptr};
    if (ch == 1)
      launch_norm<DT, 1>(smax, na, st);
    else
      launch_norm<DT, 2>(smax, na, st);
  });
  PE_CHECK_LAUNCH();
  return PE_OK;
}

int pe_internal_embed_rmsnorm(const int64_t* ids, int M, const void* table, int64_t V, void* h, int H, const void* w,
                              float eps, int mode, int dtype, void* xn, void* xn_tiled, void* cap_h, int64_t ld_cap_h,
                              void* cap_xn, int64_t ld_cap_xn, int32_t* status, hipStream_t st) {
  if (!ids || !table || !h || !w || !(xn || xn_tiled) || M <= 0 || H <= 0 || V <= 0) return PE_ERR_ARG;
  if (H % 4 || H > 4 * kNormThreads * kNormChunks) return PE_ERR_ARG;
  if (xn_tiled && (H % 128 || dtype == PE_DTYPE_F32)) return PE_ERR_ARG;
  const int ch = (H >> 2) > kNormThreads ? 2 : 1;
  PE_DISPATCH_DT(dtype, {
    typedef typename Elem<DT>::T T;
    const NormArgs<T> na{nullptr, 0, M, (T*)h, H, (const T*)w, eps, mode, (T*)xn, (T*)xn_tiled, (T*)cap_h, ld_cap_h,
                         (T*)cap_xn, ld_cap_xn, ids, (const T*)table, V, status};
    if (ch == 1)
      launch_norm_sm<DT, 1, 0>(na, st);
    else
      launch_norm_sm<DT, 2, 0>(na, st);
  });
  PE_CHECK_LAUNCH();
  return PE_OK;
}
