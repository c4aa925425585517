// Linear layers of the verification pass: Y[M][N] = X[M][K] . W^T, fp32 accumulate.
//
// The tree block is small (M = T = 26 rows at the 7B shape) and the weights are
// large, so every linear is bound by streaming W from HBM once. The MFMA kernels
// therefore:
//   * stream W in the tiled layouts of pe_format.hip: each wave load instruction
//     reads 1 KiB contiguous,
//   * use v_mfma_f32_32x32x16_{bf16,f16} with X as the A operand (32 rows per
//     M tile) and the dequantised weights as the B operand (32 columns),
//   * dequantise NF4 in registers through a per-lane 16-entry bf16 table in LDS
//     that holds bf16_rne(NF4[c] * absmax) for the lane's current block, so the
//     MFMA consumes exactly the bf16 weights bitsandbytes' dequantize_4bit feeds
//     to its GEMM,
//   * split K across the 4 waves of a workgroup (reduced in LDS) and, when the
//     output has too few column tiles to fill 256 CUs, across workgroups: the
//     last workgroup of a column group (atomic counter) sums the split partials
//     in split order, so results are deterministic and independent of M.

#include "pe_common.h"

namespace {

constexpr int kWaves = 4;
constexpr int64_t kCounterBytes = 32768;  // one u32 per column group, zero between calls

struct EpiArgs {
  int op;
  int M;
  int N;  // GEMM columns
  const void* bias;
  const void* resid;
  int64_t ld_resid;
  void* out;
  int64_t ld_out;
};

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

template <int DT>
__device__ __forceinline__ void epi_value(const EpiArgs& e, int row, int col, float v) {
  typedef Elem<DT> E;
  typename E::T* out = (typename E::T*)e.out;
  if (e.op == PE_EPI_RESIDUAL) {
    const typename E::T* r = (const typename E::T*)e.resid;
    float h = E::round(v);
    E::store(out, (int64_t)row * e.ld_out + col, __fadd_rn(E::load(r, (int64_t)row * e.ld_resid + col), h));
  } else {
    if (e.bias) v = __fadd_rn(v, E::load((const typename E::T*)e.bias, col));
    E::store(out, (int64_t)row * e.ld_out + col, v);
  }
}

template <int DT>
__device__ __forceinline__ void epi_swiglu(const EpiArgs& e, int row, int col, float gv, float uv) {
  typedef Elem<DT> E;
  float gr = E::round(gv), ur = E::round(uv);
  float s = E::round(silu_f(gr));
  E::store((typename E::T*)e.out, (int64_t)row * e.ld_out + col, __fmul_rn(s, ur));
}

__device__ __forceinline__ bf16x8_t nf4_dequant8(uint32_t q, const uint16_t* t) {
  // t points at tab[c = 0][lane]; entries of code c sit 64 elements apart.
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t lo = t[((q >> (8 * p)) & 15u) * 64];
    uint32_t hi = t[((q >> (8 * p + 4)) & 15u) * 64];
    w[p] = lo | (hi << 16);
  }
  return __builtin_bit_cast(bf16x8_t, w);
}

template <int FMT>
__device__ __forceinline__ f32x16_t mfma16(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (FMT == PE_DTYPE_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                   __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                    __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// FMT: PE_WFMT_NF4 (bf16 compute) is encoded as -1; PE_DTYPE_BF16 / PE_DTYPE_F16 dense.
constexpr int kFmtNF4 = -1;

template <int FMT, int MT, int NT>
__global__ __launch_bounds__(256) void mfma_gemm_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, int K, const uint8_t* __restrict__ W,
    const uint16_t* __restrict__ Wabs, int S, int steps_per_split, float* __restrict__ partial,
    uint32_t* __restrict__ counters, EpiArgs e) {
  constexpr int ADT = (FMT == PE_DTYPE_F16) ? PE_DTYPE_F16 : PE_DTYPE_BF16;
  const int group = blockIdx.x, split = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 5, ln = lane & 31;
  const int NS = K >> 7;
  const int s_begin = split * steps_per_split;
  const int s_end = min(NS, s_begin + steps_per_split);
  const int n_steps = max(0, s_end - s_begin);
  const int w0 = s_begin + (n_steps * wave) / kWaves;
  const int w1 = s_begin + (n_steps * (wave + 1)) / kWaves;

  __shared__ uint16_t tab[(FMT == kFmtNF4) ? kWaves * NT * 16 * 64 : 1];
  __shared__ float red[kWaves - 1][16][64];

  f32x16_t acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nt][mt][r] = 0.f;

  // Rows at or beyond M read as zero, so X needs exactly M rows.
  const uint16_t* xrow[MT];
  bool xok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    xok[mt] = (mt * 32 + ln) < e.M;
    xrow[mt] = X + (int64_t)(xok[mt] ? (mt * 32 + ln) : 0) * ldx;
  }
  const u32x4_t zero4 = {0u, 0u, 0u, 0u};

  if constexpr (FMT == kFmtNF4) {
    uint16_t* mytab = tab + (wave * NT) * 16 * 64 + lane;
    u32x4_t qn[NT][2];
    uint16_t an[NT];
    auto load_step = [&](int s) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int64_t ts = (int64_t)(group * NT + nt) * NS + s;
        const uint8_t* wp = W + ts * 2048 + lane * 16;
        qn[nt][0] = *(const u32x4_t*)(wp);
        qn[nt][1] = *(const u32x4_t*)(wp + 1024);
        an[nt] = Wabs[ts * 64 + lane];
      }
    };
    if (w0 < w1) load_step(w0);
    for (int s = w0; s < w1; ++s) {
      u32x4_t qc[NT][2];
      uint16_t ac[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) { qc[nt][0] = qn[nt][0]; qc[nt][1] = qn[nt][1]; ac[nt] = an[nt]; }
      if (s + 1 < w1) load_step(s + 1);
      // per-lane dequant tables for this step's block of each column tile
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float sc = f16_bits_to_f32(ac[nt]);
        uint16_t* t = mytab + nt * 16 * 64;
#pragma unroll
        for (int c = 0; c < 16; ++c) t[c * 64] = f32_to_bf16_bits(kNF4[c] * sc);
      }
      const int kb = 128 * s + 64 * g;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        u32x4_t a[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) a[mt] = xok[mt] ? *(const u32x4_t*)(xrow[mt] + kb + 8 * j) : zero4;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const uint32_t q = qc[nt][j >> 2][j & 3];
          bf16x8_t bv = nf4_dequant8(q, mytab + nt * 16 * 64);
          u32x4_t b = __builtin_bit_cast(u32x4_t, bv);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16<PE_DTYPE_BF16>(a[mt], b, acc[nt][mt]);
        }
      }
    }
  } else {
    const int KS = K >> 4;
    const uint16_t* Wd = (const uint16_t*)W;
    for (int s = w0; s < w1; ++s) {
      u32x4_t b[NT][8];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          b[nt][j] = *(const u32x4_t*)(Wd + (((int64_t)(group * NT + nt) * KS + 8 * s + j) * 64 + lane) * 8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = 16 * (8 * s + j) + 8 * g;
        u32x4_t a[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) a[mt] = xok[mt] ? *(const u32x4_t*)(xrow[mt] + k) : zero4;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16<FMT>(a[mt], b[nt][j], acc[nt][mt]);
      }
    }
  }

  // ---- reduce the 4 waves' K slices: ((w0 + w1) + w2) + w3
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave - 1][r][lane] = acc[nt][mt][r];
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int w = 0; w < kWaves - 1; ++w)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[nt][mt][r] += red[w][r][lane];
      }
      __syncthreads();
    }
  }
  if (wave != 0) return;

  if (S > 1) {
    constexpr int kVals = NT * MT * 16;
    float* mine = partial + ((int64_t)group * S + split) * kVals * 64;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mine[((nt * MT + mt) * 16 + r) * 64 + lane] = acc[nt][mt][r];
    __threadfence();
    uint32_t old = 0;
    if (lane == 0) old = atomicAdd(&counters[group], 1u);
    old = __shfl(old, 0, 64);
    if (old != (uint32_t)(S - 1)) return;
    __threadfence();
    const float* base = partial + (int64_t)group * S * kVals * 64;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = 0.f;
          for (int sp = 0; sp < S; ++sp) v += base[((int64_t)sp * kVals + (nt * MT + mt) * 16 + r) * 64 + lane];
          acc[nt][mt][r] = v;
        }
    if (lane == 0) counters[group] = 0u;
  }

  // ---- epilogue
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = mt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
      if (row >= e.M) continue;
      if (e.op == PE_EPI_SWIGLU) {
        if constexpr (NT == 2) epi_swiglu<ADT>(e, row, group * 32 + ln, acc[0][mt][r], acc[1][mt][r]);
      } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) epi_value<ADT>(e, row, (group * NT + nt) * 32 + ln, acc[nt][mt][r]);
      }
    }
  }
}

// fp32 linear on VALU: thread = output column, 8 rows per block row.
__global__ __launch_bounds__(64) void f32_gemm_kernel(const float* __restrict__ X, int64_t ldx, int M, int K,
                                                      const float* __restrict__ W, int n_out, EpiArgs e) {
  const int col = blockIdx.x * 64 + threadIdx.x;
  const int m0 = blockIdx.y * 8;
  if (col >= n_out) return;
  const bool swiglu = e.op == PE_EPI_SWIGLU;
  const int wrow = swiglu ? (col >> 5) * 64 + (col & 31) : col;
  const float* wg = W + (int64_t)wrow * K;
  const float* wu = W + (int64_t)(wrow + 32) * K;
  float a[8], b[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) { a[r] = 0.f; b[r] = 0.f; }
  const int nrow = min(8, M - m0);
  for (int k = 0; k < K; ++k) {
    const float w1 = wg[k];
    const float w2 = swiglu ? wu[k] : 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (r < nrow) {
        const float x = X[(int64_t)(m0 + r) * ldx + k];
        a[r] = fmaf(x, w1, a[r]);
        if (swiglu) b[r] = fmaf(x, w2, b[r]);
      }
    }
  }
  for (int r = 0; r < nrow; ++r) {
    if (swiglu) epi_swiglu<PE_DTYPE_F32>(e, m0 + r, col, a[r], b[r]);
    else epi_value<PE_DTYPE_F32>(e, m0 + r, col, a[r]);
  }
}

struct Plan {
  int NT, MT, S, steps, groups;
  int64_t partial_bytes;
};

int round_mt(int M) {
  int mt = (M + 31) / 32;
  if (mt <= 1) return 1;
  if (mt <= 2) return 2;
  if (mt <= 4) return 4;
  return 8;
}

Plan make_plan(int M, int N, int K, int epi) {
  Plan p;
  p.NT = (epi == PE_EPI_SWIGLU) ? 2 : 1;
  p.MT = round_mt(M);
  p.groups = N / (32 * p.NT);
  const int NS = K / 128;
  int S = (512 + p.groups - 1) / p.groups;
  int smax = NS / kWaves;
  if (smax < 1) smax = 1;
  if (S > smax) S = smax;
  if (S < 1) S = 1;
  p.steps = (NS + S - 1) / S;
  p.S = (NS + p.steps - 1) / p.steps;
  p.partial_bytes = (p.S > 1) ? (int64_t)p.groups * p.S * p.NT * p.MT * 16 * 64 * 4 : 0;
  return p;
}

template <int FMT, int NT>
int launch_mt(const Plan& p, hipStream_t st, const uint16_t* x, int64_t ldx, int K, const uint8_t* w,
              const uint16_t* a, float* partial, uint32_t* counters, const EpiArgs& e) {
  dim3 grid(p.groups, p.S);
  switch (p.MT) {
    case 1: mfma_gemm_kernel<FMT, 1, NT><<<grid, 256, 0, st>>>(x, ldx, K, w, a, p.S, p.steps, partial, counters, e); break;
    case 2: mfma_gemm_kernel<FMT, 2, NT><<<grid, 256, 0, st>>>(x, ldx, K, w, a, p.S, p.steps, partial, counters, e); break;
    case 4: mfma_gemm_kernel<FMT, 4, NT><<<grid, 256, 0, st>>>(x, ldx, K, w, a, p.S, p.steps, partial, counters, e); break;
    default: mfma_gemm_kernel<FMT, 8, NT><<<grid, 256, 0, st>>>(x, ldx, K, w, a, p.S, p.steps, partial, counters, e); break;
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}

template <int FMT>
int launch_fmt(const Plan& p, hipStream_t st, const uint16_t* x, int64_t ldx, int K, const uint8_t* w,
               const uint16_t* a, float* partial, uint32_t* counters, const EpiArgs& e) {
  if (p.NT == 2) return launch_mt<FMT, 2>(p, st, x, ldx, K, w, a, partial, counters, e);
  return launch_mt<FMT, 1>(p, st, x, ldx, K, w, a, partial, counters, e);
}

int mfma_gemm(int fmt, const void* x, int64_t ldx, int M, int K, const void* w, const uint16_t* wabs, int N,
              int epi, const void* bias, const void* resid, int64_t ld_resid, void* out, int64_t ld_out,
              void* ws, int64_t ws_bytes, hipStream_t st) {
  if (!x || !w || !out || M <= 0 || K <= 0 || N <= 0 || K % 128 || N % 32) return PE_ERR_ARG;
  if (epi == PE_EPI_SWIGLU && N % 64) return PE_ERR_ARG;
  if (epi == PE_EPI_RESIDUAL && !resid) return PE_ERR_ARG;
  if (epi < 0 || epi > PE_EPI_SWIGLU) return PE_ERR_ARG;
  int done = 0;
  while (done < M) {
    const int mc = (M - done > 256) ? 256 : (M - done);
    Plan p = make_plan(mc, N, K, epi);
    if (p.groups * 4 > kCounterBytes) return PE_ERR_ARG;
    if (p.S > 1 && (!ws || ws_bytes < kCounterBytes + p.partial_bytes)) return PE_ERR_WORKSPACE;
    EpiArgs e;
    e.op = epi;
    e.M = mc;
    e.N = N;
    e.bias = bias;
    e.ld_resid = ld_resid;
    e.ld_out = ld_out;
    const size_t esz = 2;
    e.resid = resid ? (const void*)((const char*)resid + (size_t)done * ld_resid * esz) : nullptr;
    e.out = (void*)((char*)out + (size_t)done * ld_out * esz);
    const uint16_t* xc = (const uint16_t*)x + (size_t)done * ldx;
    uint32_t* counters = (uint32_t*)ws;
    float* partial = ws ? (float*)((char*)ws + kCounterBytes) : nullptr;
    int rc;
    if (fmt == kFmtNF4)
      rc = launch_fmt<kFmtNF4>(p, st, xc, ldx, K, (const uint8_t*)w, wabs, partial, counters, e);
    else if (fmt == PE_DTYPE_F16)
      rc = launch_fmt<PE_DTYPE_F16>(p, st, xc, ldx, K, (const uint8_t*)w, nullptr, partial, counters, e);
    else
      rc = launch_fmt<PE_DTYPE_BF16>(p, st, xc, ldx, K, (const uint8_t*)w, nullptr, partial, counters, e);
    if (rc != PE_OK) return rc;
    done += mc;
  }
  return PE_OK;
}

}  // namespace

extern "C" int64_t pe_gemm_workspace_bytes(int M, int N, int K, int wfmt, int dtype, int epilogue) {
  (void)wfmt;
  if (dtype == PE_DTYPE_F32 && wfmt == PE_WFMT_DENSE) return 0;
  if (M <= 0 || N <= 0 || K < 128) return kCounterBytes;
  const int mc = M > 256 ? 256 : M;
  Plan p = make_plan(mc, N, K, epilogue);
  return kCounterBytes + p.partial_bytes;
}

extern "C" int pe_nf4_gemm(const void* x, int64_t ldx, int M, int K, const uint8_t* w_tiled,
                           const uint16_t* absmax_tiled, int N, int epilogue, const void* bias,
                           const void* resid, int64_t ld_resid, void* out, int64_t ld_out, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  if (!absmax_tiled) return PE_ERR_ARG;
  return mfma_gemm(kFmtNF4, x, ldx, M, K, w_tiled, absmax_tiled, N, epilogue, bias, resid, ld_resid, out,
                   ld_out, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int pe_dense_gemm(const void* x, int64_t ldx, int M, int K, const void* w, int dtype, int N,
                             int epilogue, const void* bias, const void* resid, int64_t ld_resid, void* out,
                             int64_t ld_out, void* workspace, int64_t workspace_bytes, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  if (dtype == PE_DTYPE_F32) {
    if (!x || !w || !out || M <= 0 || K <= 0 || N <= 0) return PE_ERR_ARG;
    if (epilogue == PE_EPI_RESIDUAL && !resid) return PE_ERR_ARG;
    if (epilogue < 0 || epilogue > PE_EPI_SWIGLU) return PE_ERR_ARG;
    if (epilogue == PE_EPI_SWIGLU && N % 64) return PE_ERR_ARG;
    EpiArgs e;
    e.op = epilogue;
    e.M = M;
    e.N = N;
    e.bias = bias;
    e.resid = resid;
    e.ld_resid = ld_resid;
    e.out = out;
    e.ld_out = ld_out;
    const int n_out = epilogue == PE_EPI_SWIGLU ? N / 2 : N;
    dim3 grid((n_out + 63) / 64, (M + 7) / 8);
    f32_gemm_kernel<<<grid, 64, 0, st>>>((const float*)x, ldx, M, K, (const float*)w, n_out, e);
    PE_CHECK_LAUNCH();
    return PE_OK;
  }
  if (dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16) return PE_ERR_ARG;
  return mfma_gemm(dtype, x, ldx, M, K, w, nullptr, N, epilogue, bias, resid, ld_resid, out, ld_out, workspace,
                   workspace_bytes, st);
}
