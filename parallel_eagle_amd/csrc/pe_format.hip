// Synthetic weight generation and the weight formats read by the GEMMs.
//
// NF4 logical layout (bitsandbytes): W[N][K] row-major, block of 64 consecutive
// elements along K shares one absmax; byte j of the packed array holds element
// 2j in its high nibble and element 2j+1 in its low nibble.
//
// NF4 tiled layout (what pe_nf4_gemm streams): for column tile nt (32 output
// columns) and super-step s (128 along K), 2 KiB of codes and 128 B of absmax:
//   codes[((nt*NS + s)*2 + h)*1024 + lane*16 + 4*jj + byte]   h = 0,1; jj = 0..3
//   absmax[(nt*NS + s)*64 + lane]
// lane -> column nt*32 + (lane & 31), block b = 2s + (lane >> 5); dword j = 4h + jj
// holds the 8 codes of k = 64b + 8j + e (e = 0..7) with code e at bits [4e, 4e+4).
// One MFMA step j of a super-step consumes dword j of every lane, so each wave
// load instruction is 1 KiB contiguous.
//
// Dense 16-bit tiled layout: tiled[((nt*(K/16) + ks)*64 + lane)*8 + e]
//   = W[nt*32 + (lane & 31)][16ks + 8(lane >> 5) + e].

#include "pe_common.h"

#pragma clang fp contract(off)

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z ^= z >> 30;
  z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27;
  z *= 0x94D049BB133111EBull;
  z ^= z >> 31;
  return z;
}

__device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint64_t sid) {
  return mix64(seed * 0x9E3779B97F4A7C15ull + sid * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull);
}

__device__ __forceinline__ float normal_at(uint64_t key, int64_t i, double sd) {
  uint64_t z = mix64(key + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull);
  uint64_t s = (z & 0xFFFF) + ((z >> 16) & 0xFFFF) + ((z >> 32) & 0xFFFF) + (z >> 48);
  double x = ((double)s + 2.0) / 65536.0 - 2.0;
  double v = x * 1.7320508075688772;
  return (float)(v * sd);
}

template <int DT>
__global__ void fill_normal_kernel(typename Elem<DT>::T* out, int64_t n, uint64_t key, double sd) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    Elem<DT>::store(out, i, normal_at(key, i, sd));
}

__global__ void fill_uniform_int_kernel(int64_t* out, int64_t n, uint64_t key, uint64_t hi) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint64_t z = mix64(key + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull);
    out[i] = (int64_t)(((z >> 32) * hi) >> 32);
  }
}

// One thread per 64-element block.
__global__ void nf4_quantize_kernel(const float* __restrict__ w, int64_t nblocks,
                                    uint8_t* __restrict__ packed, uint16_t* __restrict__ absmax) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblocks; b += stride) {
    const float* x = w + b * 64;
    float amax = 0.f;
    for (int i = 0; i < 64; ++i) amax = fmaxf(amax, fabsf(x[i]));
    uint16_t a16 = f32_to_f16_bits(amax);
    absmax[b] = a16;
    float sc = f16_bits_to_f32(a16);
    uint8_t* dst = packed + b * 32;
    for (int i = 0; i < 64; i += 2) {
      int code[2];
      for (int h = 0; h < 2; ++h) {
        float xn = sc > 0.f ? x[i + h] / sc : 0.f;
        int best = 0;
        float bd = fabsf(xn - kNF4[0]);
        for (int c = 1; c < 16; ++c) {
          float d = fabsf(xn - kNF4[c]);
          if (d < bd) { bd = d; best = c; }
        }
        code[h] = best;
      }
      dst[i >> 1] = (uint8_t)((code[0] << 4) | code[1]);
    }
  }
}

// One thread per (tile, super-step, lane). A: the absmax bits (fp16 or fp32),
// copied as they are.
template <typename A>
__global__ void nf4_repack_kernel(const uint8_t* __restrict__ packed, const A* __restrict__ absmax, int64_t N,
                                  int64_t K, uint8_t* __restrict__ tiled, A* __restrict__ tabs) {
  const int64_t NS = K / 128, total = (N / 32) * NS * 64;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    int lane = (int)(idx & 63);
    int64_t ts = idx >> 6;  // nt * NS + s
    int64_t nt = ts / NS, s = ts % NS;
    int64_t n = nt * 32 + (lane & 31);
    int64_t b = 2 * s + (lane >> 5);
    const uint8_t* src = packed + n * (K / 2) + b * 32;  // 64 codes of block b
    uint32_t dw[8];
    for (int j = 0; j < 8; ++j) {
      uint32_t v = 0;
      for (int e = 0; e < 8; ++e) {
        int el = 8 * j + e;
        uint8_t byte = src[el >> 1];
        uint32_t code = (el & 1) ? (byte & 15u) : (byte >> 4);
        v |= code << (4 * e);
      }
      dw[j] = v;
    }
    uint32_t* d0 = (uint32_t*)(tiled + (ts * 2 + 0) * 1024 + lane * 16);
    uint32_t* d1 = (uint32_t*)(tiled + (ts * 2 + 1) * 1024 + lane * 16);
    for (int jj = 0; jj < 4; ++jj) { d0[jj] = dw[jj]; d1[jj] = dw[4 + jj]; }
    tabs[ts * 64 + lane] = absmax[n * (K / 64) + b];
  }
}

template <typename A>
__global__ void nf4_dequant_kernel(const uint8_t* __restrict__ tiled, const A* __restrict__ tabs, int64_t N,
                                   int64_t K, uint16_t* __restrict__ out) {
  const int64_t NS = K / 128, total = (N / 32) * NS * 64;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    int lane = (int)(idx & 63);
    int64_t ts = idx >> 6;
    int64_t nt = ts / NS, s = ts % NS;
    int64_t n = nt * 32 + (lane & 31);
    int64_t b = 2 * s + (lane >> 5);
    const float sc = sizeof(A) == 4 ? __uint_as_float((uint32_t)tabs[ts * 64 + lane])
                                    : f16_bits_to_f32((uint16_t)tabs[ts * 64 + lane]);
    for (int j = 0; j < 8; ++j) {
      const uint32_t* src = (const uint32_t*)(tiled + (ts * 2 + (j >> 2)) * 1024 + lane * 16);
      uint32_t q = src[j & 3];
      for (int e = 0; e < 8; ++e) {
        uint32_t c = (q >> (4 * e)) & 15u;
        out[n * K + 64 * b + 8 * j + e] = f32_to_bf16_bits(kNF4[c] * sc);
      }
    }
  }
}

__global__ void dense_repack_kernel(const uint16_t* __restrict__ w, int64_t N, int64_t K,
                                    uint16_t* __restrict__ tiled) {
  const int64_t KS = K / 16, total = (N / 32) * KS * 64;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    int lane = (int)(idx & 63);
    int64_t t = idx >> 6;
    int64_t nt = t / KS, ks = t % KS;
    int64_t n = nt * 32 + (lane & 31);
    const uint16_t* src = w + n * K + 16 * ks + 8 * (lane >> 5);
    uint16_t* dst = tiled + idx * 8;
    for (int e = 0; e < 8; ++e) dst[e] = src[e];
  }
}

__global__ void copy_bytes_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t n) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

int grid_for(int64_t n, int block) {
  int64_t g = (n + block - 1) / block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

// bitsandbytes' blockwise 8-bit dequantisation of the absmax plus its offset:
// one fp32 product, then one fp32 sum (two roundings: contraction into a
// fused multiply-add is switched off here).
__global__ void nf4_absmax_dequant_kernel(const uint8_t* __restrict__ q, int64_t n, const float* __restrict__ code,
                                          const float* __restrict__ nested, int nbs, float offset,
                                          float* __restrict__ out) {
#pragma clang fp contract(off)
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float prod = code[q[i]] * nested[i / nbs];  // rounded to fp32
    out[i] = prod + offset;                            // rounded again
  }
}

}  // namespace

extern "C" int pe_fill_normal(void* out, int64_t n, int dtype, uint64_t seed, uint64_t stream_id,
                              double std_, void* stream) {
  if (!out || n < 0) return PE_ERR_ARG;
  if (n == 0) return PE_OK;
  hipStream_t st = (hipStream_t)stream;
  uint64_t key;
  {
    // host copy of stream_key (same integer arithmetic)
    uint64_t z = seed * 0x9E3779B97F4A7C15ull + stream_id * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull;
    z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull; z ^= z >> 27; z *= 0x94D049BB133111EBull; z ^= z >> 31;
    key = z;
  }
  int g = grid_for(n, 256);
  switch (dtype) {
    case PE_DTYPE_F32: fill_normal_kernel<PE_DTYPE_F32><<<g, 256, 0, st>>>((float*)out, n, key, std_); break;
    case PE_DTYPE_BF16: fill_normal_kernel<PE_DTYPE_BF16><<<g, 256, 0, st>>>((uint16_t*)out, n, key, std_); break;
    case PE_DTYPE_F16: fill_normal_kernel<PE_DTYPE_F16><<<g, 256, 0, st>>>((uint16_t*)out, n, key, std_); break;
    default: return PE_ERR_ARG;
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_fill_uniform_int(int64_t* out, int64_t n, int64_t hi, uint64_t seed,
                                   uint64_t stream_id, void* stream) {
  if (!out || n < 0 || hi <= 0 || hi > 0xFFFFFFFFll) return PE_ERR_ARG;
  if (n == 0) return PE_OK;
  uint64_t z = seed * 0x9E3779B97F4A7C15ull + stream_id * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull;
  z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull; z ^= z >> 27; z *= 0x94D049BB133111EBull; z ^= z >> 31;
  fill_uniform_int_kernel<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(out, n, z, (uint64_t)hi);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_nf4_quantize(const float* w, int64_t N, int64_t K, uint8_t* packed, uint16_t* absmax,
                               void* stream) {
  if (!w || !packed || !absmax || N <= 0 || K <= 0 || K % 64) return PE_ERR_ARG;
  int64_t nb = N * K / 64;
  nf4_quantize_kernel<<<grid_for(nb, 256), 256, 0, (hipStream_t)stream>>>(w, nb, packed, absmax);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_nf4_repack(const uint8_t* packed, const uint16_t* absmax, int64_t N, int64_t K,
                             uint8_t* tiled, uint16_t* tiled_absmax, void* stream) {
  if (!packed || !absmax || !tiled || !tiled_absmax || N <= 0 || N % 32 || K <= 0 || K % 128)
    return PE_ERR_ARG;
  int64_t total = (N / 32) * (K / 128) * 64;
  nf4_repack_kernel<uint16_t><<<grid_for(total, 256), 256, 0, (hipStream_t)stream>>>(packed, absmax, N, K, tiled,
                                                                                    tiled_absmax);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_nf4_repack_f32abs(const uint8_t* packed, const float* absmax, int64_t N, int64_t K,
                                    uint8_t* tiled, float* tiled_absmax, void* stream) {
  if (!packed || !absmax || !tiled || !tiled_absmax || N <= 0 || N % 32 || K <= 0 || K % 128)
    return PE_ERR_ARG;
  int64_t total = (N / 32) * (K / 128) * 64;
  nf4_repack_kernel<uint32_t><<<grid_for(total, 256), 256, 0, (hipStream_t)stream>>>(
      packed, (const uint32_t*)absmax, N, K, tiled, (uint32_t*)tiled_absmax);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_nf4_absmax_dequant(const uint8_t* q, int64_t n, const float* code, const float* nested_absmax,
                                     int nested_blocksize, float offset, float* absmax, void* stream) {
  if (!q || !code || !nested_absmax || !absmax || n <= 0 || nested_blocksize <= 0) return PE_ERR_ARG;
  nf4_absmax_dequant_kernel<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(q, n, code, nested_absmax,
                                                                                nested_blocksize, offset, absmax);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_nf4_dequant(const uint8_t* tiled, const uint16_t* tiled_absmax, int64_t N, int64_t K,
                              uint16_t* out, void* stream) {
  if (!tiled || !tiled_absmax || !out || N <= 0 || N % 32 || K <= 0 || K % 128) return PE_ERR_ARG;
  int64_t total = (N / 32) * (K / 128) * 64;
  nf4_dequant_kernel<uint16_t><<<grid_for(total, 256), 256, 0, (hipStream_t)stream>>>(tiled, tiled_absmax, N, K,
                                                                                     out);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_nf4_dequant_f32abs(const uint8_t* tiled, const float* tiled_absmax, int64_t N, int64_t K,
                                     uint16_t* out, void* stream) {
  if (!tiled || !tiled_absmax || !out || N <= 0 || N % 32 || K <= 0 || K % 128) return PE_ERR_ARG;
  int64_t total = (N / 32) * (K / 128) * 64;
  nf4_dequant_kernel<uint32_t><<<grid_for(total, 256), 256, 0, (hipStream_t)stream>>>(
      tiled, (const uint32_t*)tiled_absmax, N, K, out);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int pe_dense_repack(const void* w, int64_t N, int64_t K, int dtype, void* tiled, void* stream) {
  if (!w || !tiled || N <= 0 || K <= 0) return PE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == PE_DTYPE_F32) {
    int64_t nbytes = N * K * 4;
    copy_bytes_kernel<<<grid_for(nbytes, 256), 256, 0, st>>>((const uint8_t*)w, (uint8_t*)tiled, nbytes);
  } else if (dtype == PE_DTYPE_BF16 || dtype == PE_DTYPE_F16) {
    if (N % 32 || K % 16) return PE_ERR_ARG;
    int64_t total = (N / 32) * (K / 16) * 64;
    dense_repack_kernel<<<grid_for(total, 256), 256, 0, st>>>((const uint16_t*)w, N, K, (uint16_t*)tiled);
  } else {
    return PE_ERR_ARG;
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}
