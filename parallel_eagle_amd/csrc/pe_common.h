// Shared device helpers for the verification-pass kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/pe_hip.h"

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
typedef float f32x2_t __attribute__((ext_vector_type(2)));

#define PE_WAVE 64

// ---------------------------------------------------------------------------
// Scalar conversions. Rounding is round-to-nearest-even everywhere, which is
// what torch's float -> bfloat16 / float16 casts do.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Two floats rounded (nearest even) to the 16-bit type DT and packed, lo in
// the low half: one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 instead of two
// conversions and a pack; the same bits as f32_to_bf16_bits / f32_to_f16_bits.
template <int DT>
__device__ __forceinline__ uint32_t pack2_16(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  if constexpr (DT == PE_DTYPE_F16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Element access by storage type: dtype codes follow PE_DTYPE_* in pe_hip.h.
template <int DT> struct Elem;
template <> struct Elem<PE_DTYPE_F32> {
  typedef float T;
  static __device__ __forceinline__ float load(const T* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(T* p, int64_t i, float v) { p[i] = v; }
  static __device__ __forceinline__ float round(float v) { return v; }
};
template <> struct Elem<PE_DTYPE_BF16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const T* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ void store(T* p, int64_t i, float v) { p[i] = f32_to_bf16_bits(v); }
  static __device__ __forceinline__ float round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
};
template <> struct Elem<PE_DTYPE_F16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const T* p, int64_t i) { return f16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ void store(T* p, int64_t i, float v) { p[i] = f32_to_f16_bits(v); }
  static __device__ __forceinline__ float round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
};

// Four consecutive elements as floats through one access: 8 bytes for the
// 16-bit types, 16 bytes for fp32 (the pointer is aligned to that size).
template <int DT> struct Vec4;
template <> struct Vec4<PE_DTYPE_F32> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    const float4 t = *(const float4*)p;
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  }
};
template <int DT> struct Vec4Half {
  static __device__ __forceinline__ float cvt(uint32_t b) {
    return DT == PE_DTYPE_BF16 ? bf16_bits_to_f32((uint16_t)b) : f16_bits_to_f32((uint16_t)b);
  }
  static __device__ __forceinline__ uint32_t bits(float f) {
    return DT == PE_DTYPE_BF16 ? f32_to_bf16_bits(f) : f32_to_f16_bits(f);
  }
  static __device__ __forceinline__ void load(const uint16_t* p, float (&v)[4]) {
    const uint2 t = *(const uint2*)p;
    v[0] = cvt(t.x & 0xffffu); v[1] = cvt(t.x >> 16); v[2] = cvt(t.y & 0xffffu); v[3] = cvt(t.y >> 16);
  }
  static __device__ __forceinline__ void store(uint16_t* p, const float (&v)[4]) {
    *(uint2*)p = make_uint2(bits(v[0]) | (bits(v[1]) << 16), bits(v[2]) | (bits(v[3]) << 16));
  }
};
template <> struct Vec4<PE_DTYPE_BF16> : Vec4Half<PE_DTYPE_BF16> {};
template <> struct Vec4<PE_DTYPE_F16> : Vec4Half<PE_DTYPE_F16> {};

// The published NF4 code book (QLoRA / bitsandbytes), fp32. Code 7 is 0.
__device__ __constant__ static const float kNF4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

// The normalised value of x times the weight w, rounded as PE_NORM_HF (the
// normalised value rounded, then a rounded multiply by w: HF LlamaRMSNorm,
// modeling_llama.py:62-67) or PE_NORM_FP32_WEIGHT (x * inv * w in fp32, one
// rounding: src/pe/nn.py:22-26).
template <typename E>
__device__ __forceinline__ float norm_out(int mode, float x, float inv, float w) {
  const float y = __fmul_rn(x, inv);
  return mode == PE_NORM_FP32_WEIGHT ? E::round(__fmul_rn(y, w)) : E::round(__fmul_rn(w, E::round(y)));
}

// Wave-level reductions (wave64) through DPP-free shuffles.
// Order-preserving key of a value for torch.argmax's semantics: larger value
// -> larger key, every NaN -> the largest key, -0 and +0 -> the same key (they
// compare equal).
__device__ __forceinline__ uint32_t arg_key(float f) {
  if (f != f) return 0xFFFFFFFFu;
  const uint32_t u = f == 0.f ? 0u : __float_as_uint(f);
  return (u >> 31) ? ~u : (u | 0x80000000u);
}
// (value key, column) as one 64-bit key whose maximum is the largest value at
// the lowest column
__device__ __forceinline__ uint64_t arg_key64(float f, int col) {
  return ((uint64_t)arg_key(f) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)col);
}
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_xor((uint32_t)v, o, 64), hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// A-tiled activations: the order in which the NF4 GEMM reads X as its MFMA A
// operand, so that every X load instruction of a wave reads 1 KiB contiguous.
// Element (row, col) of an [M][K] activation (K % 128 == 0, `units` = K / 128)
// sits in 128-column unit p = col / 128, k-step s = (col % 64) / 8 and lane
// row % 32 + 32 * ((col % 128) / 64) of M tile row / 32; a lane holds 8
// consecutive columns. Rows past M inside the last M tile are never written:
// they only feed MFMA rows whose results are discarded.
__host__ __device__ __forceinline__ int64_t xtile_index(int row, int col, int units) {
  const int mt = row >> 5, ln = row & 31;
  const int p = col >> 7, c = col & 127;
  return ((((int64_t)mt * units + p) * 8 + ((c & 63) >> 3)) * 64 + ln + 32 * (c >> 6)) * 8 + (c & 7);
}
// Bytes of an A-tiled [M][K] 16-bit activation.
__host__ __device__ __forceinline__ int64_t xtile_bytes(int M, int K) { return (int64_t)((M + 31) / 32) * K * 64; }

// Data handed between workgroups of one launch (split partials read by the
// last workgroup to arrive): 16-byte accesses with cache policy sc1, i.e.
// agent-coherent, written through to / read from the level all XCDs share,
// and still coalesced across the wave (unlike one atomic per lane). Through a
// buffer resource over [base, base + bytes); the compiler tracks the waits.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t agent_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}
constexpr int kCpolSC1 = 16;
typedef unsigned int pe_u4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store_agent_x4(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(pe_u4_t, v), r, off, 0, kCpolSC1);
}
__device__ __forceinline__ f32x4_t load_agent_x4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolSC1));
}

// 16 bytes per lane from global memory straight into LDS at lds_base + 16 *
// lane (lds_base wave-uniform, through M0), for rings of LDS buffers.
//
// A pointer that is the same in every lane, held in scalar registers.
__device__ __forceinline__ const uint16_t* uniform_ptr(const uint16_t* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint16_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// The source is a wave-uniform base (SGPRs) plus a per-lane 32-bit byte
// offset (callers keep every source within 4 GiB of the base). Issued as
// inline assembly so that the compiler, which cannot tell these LDS writes
// from the LDS being read, adds no wait for them in front of every LDS read;
// callers order them with an explicit vmcnt wait and a workgroup barrier.
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds_base)
               : "memory", "m0");
}

#define PE_CHECK_LAUNCH()                                   \
  do {                                                      \
    hipError_t _e = hipGetLastError();                      \
    if (_e != hipSuccess) return PE_ERR_LAUNCH;             \
  } while (0)

static inline int pe_cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
