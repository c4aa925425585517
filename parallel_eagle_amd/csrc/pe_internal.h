// Library-internal entry points shared between the kernel files and the
// pass driver (pe_model.cpp); not part of the C ABI in include/pe_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define PE_INTERNAL __attribute__((visibility("hidden")))

#include "pe_hip.h"

// NF4 weight formats (absmax fp16 or fp32); wabs points at the tiled absmax
// of that type
inline bool pe_wfmt_nf4(int wfmt) { return wfmt == PE_WFMT_NF4 || wfmt == PE_WFMT_NF4_F32ABS; }

// pe_gemm.hip: the q/k/v projection with bias, RoPE and the in-place K/V
// append in its epilogue (one launch over M <= 64 rows); ws as for
// pe_nf4_gemm (zeroed counters, then partials), of pe_internal_gemm_rope_kv_bytes.
PE_INTERNAL int pe_internal_gemm_rope_kv(int wfmt, int dtype, const void* x, int64_t ldx, int M, int K,
                                         const void* w, const void* wabs, int nh, int nkv, int hd,
                                         const void* bias, const int64_t* positions, const void* cos_sin,
                                         int64_t max_pos, void* q_out, void* k_cache, void* v_cache, int64_t cap,
                                         int64_t row0, int32_t* status, void* ws, int64_t ws_bytes, bool x_tiled,
                                         hipStream_t st, const int64_t* kv_off = nullptr);
PE_INTERNAL int64_t pe_internal_gemm_rope_kv_bytes(int M, int N, int K, int wfmt);
// pe_nf4_gemm / pe_dense_gemm with A-tiled X (x_tiled, M <= 64, K % 128 == 0)
// and/or an A-tiled output (out_units = N_out / 128, not with the residual
// epilogue).
PE_INTERNAL int pe_internal_linear(int wfmt, int dtype, const void* x, int64_t ldx, bool x_tiled, int M, int K,
                                   const void* w, const void* wabs, int N, int epi, const void* bias,
                                   const void* resid, int64_t ld_resid, void* out, int64_t ld_out, int out_units,
                                   void* ws, int64_t ws_bytes, hipStream_t st);

// pe_gemm.hip: Y = X . W^T as split partials partial[S][M][N] fp32 (plain
// stores, summed by the consumer in split order); *splits receives S. M <= 64.
PE_INTERNAL int pe_internal_linear_partials(int wfmt, int dtype, const void* x, int64_t ldx, bool x_tiled, int M,
                                            int K, const void* w, const void* wabs, int N, float* partial,
                                            int64_t partial_bytes, int* splits, hipStream_t st);
PE_INTERNAL int64_t pe_internal_linear_partials_bytes(int M, int N, int K, int wfmt);

// pe_gemm.hip: the dense 16-bit lm_head over A-tiled rows (M <= 64), logits in
// the dtype and, with keys, each row's per-column-group argmax keys.
PE_INTERNAL int pe_internal_dense_gemm_tiled(const void* x_tiled, int M, int K, const void* w, int dtype, int N,
                                             void* out, int64_t ld_out, uint64_t* keys, void* ws, int64_t ws_bytes,
                                             hipStream_t st);

// pe_gemm.hip: the q/k/v epilogue (bias, RoPE, q out, K/V appended at cache rows
// row0 + row) and the SwiGLU epilogue (N / 2 outputs, A-tiled when out_units)
// applied to the S split partials of their projections (the head-paired /
// gate-up interleaved column orders of the fused path).
PE_INTERNAL int pe_internal_rope_kv_partials(const float* partial, int S, int M, int nh, int nkv, int hd,
                                             const void* bias, const int64_t* positions, const void* cos_sin,
                                             int64_t max_pos, void* q_out, void* k_cache, void* v_cache, int64_t cap,
                                             int64_t row0, int32_t* status, int dtype, hipStream_t st,
                                             const int64_t* kv_off = nullptr);
// pe_gemm.hip: the NF4 GEMM for many rows (A-tiled X, 64 < M <= 256,
// N % 128 == 0, fp16 absmax): each weight dequantised once for all rows;
// fp32 split partials [S][M][N] (*splits receives S).
// Dense 16-bit Y[M][N] = X . W^T for many rows (X A-tiled, W in the
// MFMA-tiled layout, K % 128 == 0, N % 128 == 0), one workgroup per 128
// columns and block of 256 rows, each weight read once per row block; Y
// row-major (leading dimension ld_out) in the dtype, or the fp32 sums as they
// are (f32_out: split partials [S][M][ld_out] for the prefill's epilogue
// kernels; with `splits` given the launch may take S = 2 K splits and reports
// S there, else S = 1).
PE_INTERNAL int pe_internal_dense_bigm(const void* x_tiled, int M, int K, const void* w, int dtype, int N, void* out,
                                       int64_t ld_out, hipStream_t st, bool f32_out = false,
                                       int* splits = nullptr);
// The prefill's NF4 linear over all M rows (A-tiled X, blocks of 256 rows, one
// K split): fp32 sums y[M][N], or with out_units > 0 (the interleaved gate/up
// weight, N = 2 * 128 * out_units) the SwiGLU activation stored A-tiled.
PE_INTERNAL int pe_internal_nf4_prefill(const void* x_tiled, int M, int K, const void* w, const void* wabs, int N,
                                        float* y, void* act, int out_units, hipStream_t st);
// Row-major 16-bit [M][K] (leading dimension ld) -> the A-tiled layout
// (K % 128 == 0; rows past M of the last 32-row tile are written as zeros).
PE_INTERNAL int pe_internal_to_xtile(const void* x, int64_t ld, int M, int K, void* out, hipStream_t st);
PE_INTERNAL int64_t pe_internal_nf4_bigm_partials_bytes(int M, int N, int K);
PE_INTERNAL int pe_internal_nf4_bigm_partials(const void* x_tiled, int M, int K, const void* w, const void* wabs,
                                              int N, float* partial, int64_t partial_bytes, int* splits,
                                              hipStream_t st);
// The gate/up linear of the many-row pass with its SwiGLU: when the plan has
// one split (and bf16 compute) the GEMM stores the A-tiled activation itself
// and *splits = 0; otherwise it writes split partials (*splits = S) for
// pe_internal_swiglu_partials.
PE_INTERNAL int pe_internal_nf4_bigm_swiglu(const void* x_tiled, int M, int K, const void* w, const void* wabs, int N,
                                            void* out, int out_units, int dtype, float* partial, int64_t partial_bytes,
                                            int* splits, hipStream_t st);
PE_INTERNAL int pe_internal_swiglu_partials(const float* partial, int S, int M, int N, void* out, int64_t ld_out,
                                            int out_units, int dtype, hipStream_t st);

// pe_elem.hip: h = round(h + round(sum_s partial[s])) (S == 0: h unchanged),
// xn = the RMSNorm of h rounded as `mode` (PE_NORM_*), also A-tiled into xn_tiled when
// given (xn may then be null: the tiled rows only); optional copies of the new
// h (cap_h) and of xn (cap_xn) into the fused-feature rows.
PE_INTERNAL int pe_internal_residual_rmsnorm(const float* partial, int S, int M, void* h, int H, const void* w,
                                             float eps, int mode, int dtype, void* xn, void* xn_tiled, void* cap_h,
                                             int64_t ld_cap_h, void* cap_xn, int64_t ld_cap_xn, hipStream_t st);
// pe_elem.hip: the first layer's input norm fused with the embedding gather:
// h[m] = embed[ids[m]] (out-of-range ids flag PE_ERR_TOKEN in *status and read
// row 0), then xn / xn_tiled / captures as pe_internal_residual_rmsnorm.
PE_INTERNAL int pe_internal_embed_rmsnorm(const int64_t* ids, int M, const void* table, int64_t V, void* h, int H,
                                          const void* w, float eps, int mode, int dtype, void* xn, void* xn_tiled, void* cap_h,
                                          int64_t ld_cap_h, void* cap_xn, int64_t ld_cap_xn, int32_t* status,
                                          hipStream_t st);

// The pass workspace's first 32 KiB hold arrival counters: GEMM column
// groups use ints [0, kGemmCounterInts) and return them to zero; attention
// (head, row tile) pairs use the 1024 ints from kPassAttnCounterInt on, which
// the last workgroup of each pair also returns to zero.
constexpr int kGemmCounterInts = 7168;
constexpr int kPassAttnCounterInt = 7168;

// pe_attn.hip: pe_tree_attention whose output is A-tiled when out_units > 0
// (hd == 128 16-bit path only), in softmax mode attn_mode (PE_ATTN_*). counters: the launch's arrival counters
// (nullptr: the head of the workspace).
PE_INTERNAL int pe_internal_tree_attention(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap,
                                           int nh, int nkv, int hd, int T, int64_t P, int mask_mode,
                                           const uint64_t* bits, int words, float scale, int dtype, void* out,
                                           int64_t ld_out, int out_units, void* workspace, int64_t workspace_bytes,
                                           int* counters, hipStream_t st, int attn_mode = PE_ATTN_SDPA);
// Workspace of pe_internal_tree_attention in the given PE_ATTN_* mode.
PE_INTERNAL int64_t attention_workspace_bytes(int T, int nh, int nkv, int hd, int64_t kv_len, int dtype,
                                              int attn_mode);

// pe_attn.hip: tree attention of `batch` sequences in one launch (16-bit,
// hd == 128): sequence b's query rows are [seq_row0[b], seq_row0[b+1]) of q,
// bits and out (row-major), its cache kc / vc + b * seq_stride elements with
// seq_prefix[b] cached rows; max_prefix and max_rows size the launch (a
// sequence whose device prefix or row count exceeds them is skipped: no key is
// read past them, and pe_internal_kv_offsets reports it); with out_units > 0
// out is A-tiled over all rows (K = 128 * out_units). dyn_split: each
// sequence's key splits cover its own prefix + rows (round32(ceil(S / splits))
// keys each, the split count fixed by the launch), so a launch sized for a
// longer prefix than the device holds keeps its splits balanced, and a
// single sequence gets the key ranges pe_internal_tree_attention gives it.
PE_INTERNAL int64_t pe_internal_attention_batch_bytes(int max_rows, int nh, int nkv, int64_t max_kv_len, int batch);
PE_INTERNAL int pe_internal_tree_attention_batch(const void* q, const void* k_cache, const void* v_cache,
                                                 int64_t cache_cap, int64_t seq_stride, int nh, int nkv, int max_rows,
                                                 int64_t max_prefix, int batch, const int32_t* seq_row0,
                                                 const int64_t* seq_prefix, const uint64_t* bits, int words,
                                                 float scale, int dtype, void* out, int64_t ld_out, int out_units,
                                                 void* workspace, int64_t workspace_bytes, int* counters,
                                                 hipStream_t st, int dyn_split = 0);
// pe_elem.hip: per-row K/V slot offsets of a batched pass (see EpiArgs::kv_off):
// off[r] = b * seq_stride + (seq_prefix[b] + r - seq_row0[b]) * hd for row r of
// sequence b, or -1 (and PE_ERR_CAPACITY in *status) past the sequence's cache
// or when seq_prefix[b] exceeds max_prefix (the bound the launches were sized
// for); a sequence of more than max_rows rows sets PE_ERR_TREE and drops its
// rows' K/V.
// pe_elem.hip: the device sequence table of a batch of one (seq_row0 = {0, M},
// seq_prefix = {P}), written by a kernel so that a recorded pass can hold it.
PE_INTERNAL int pe_internal_one_sequence(int32_t* seq_row0, int64_t* seq_prefix, int M, int64_t P, hipStream_t st);
PE_INTERNAL int pe_internal_kv_offsets(const int32_t* seq_row0, const int64_t* seq_prefix, int batch, int M,
                                       int64_t seq_stride, int64_t cap, int hd, int64_t max_prefix, int max_rows,
                                       int64_t* off, int32_t* status, hipStream_t st);

