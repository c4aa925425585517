// Library-internal entry points shared between the kernel files and the
// pass driver (pe_model.cpp); not part of the C ABI in include/pe_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define PE_INTERNAL __attribute__((visibility("hidden")))

// pe_gemm.hip
PE_INTERNAL int pe_internal_gemm_partials(int wfmt, int dtype, const void* x, int64_t ldx, int M, int K,
                                          const void* w, const uint16_t* wabs, int N, float* partial,
                                          int64_t partial_bytes, int* S_out, hipStream_t st);
PE_INTERNAL int pe_internal_gemm_epilogue(int wfmt, int dtype, const void* x, int64_t ldx, int M, int K,
                                          const void* w, const uint16_t* wabs, int N, int epi, const void* bias,
                                          const void* resid, int64_t ld_resid, void* out, int64_t ld_out,
                                          hipStream_t st);
PE_INTERNAL int pe_internal_gemm_rope_kv(int wfmt, int dtype, const void* x, int64_t ldx, int M, int K,
                                         const void* w, const uint16_t* wabs, int nh, int nkv, int hd,
                                         const void* bias, const int64_t* positions, const void* cos_sin,
                                         int64_t max_pos, void* q_out, void* k_cache, void* v_cache, int64_t cap,
                                         int64_t row0, int32_t* status, hipStream_t st);
PE_INTERNAL int64_t pe_internal_gemm_partial_bytes(int M, int N, int K, int wfmt);

// pe_elem.hip: h = round(h + round(sum_s partial[s])) (S == 0: h unchanged),
// xn = w * round(h * rsqrt(mean(h^2) + eps)); optional copies of the new h
// (cap_h) and of xn (cap_xn) into the fused-feature rows.
PE_INTERNAL int pe_internal_residual_rmsnorm(const float* partial, int S, int M, void* h, int H, const void* w,
                                             float eps, int dtype, void* xn, void* cap_h, int64_t ld_cap_h,
                                             void* cap_xn, int64_t ld_cap_xn, hipStream_t st);
