/*
 * pe_hip.h: C ABI of the MI355X tree-verification pass (libpe_hip.so).
 *
 * Every entry point takes plain device pointers and sizes, launches on the
 * HIP stream it is given (`stream`, a hipStream_t passed as void*), never
 * allocates device memory, and returns a PE_* status (PE_OK == 0). Errors
 * that depend on device data (a non-topological tree, a token id out of the
 * vocabulary, a dense bias that is not a tree mask) are written to a
 * caller-provided device int32 `status` word with atomicOr of the PE_ERR_*
 * bit; the host reads it after the stream synchronises.
 *
 * Scratch buffers (`workspace`) are caller-owned; their counters region must
 * be zero when first used. GEMM calls leave their counters zero; attention
 * calls leave theirs multiples of 16.
 *
 * The reference implements this pass in Python over transformers/torch/
 * bitsandbytes; each entry point below names the reference function it
 * replaces (file:line in puneethgv/parallel_eagle, "HF:" = transformers 5.x).
 */
#ifndef PE_HIP_H
#define PE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes (bit flags so device-side errors can be OR-ed) */
#define PE_OK 0
#define PE_ERR_ARG 1       /* invalid argument: null pointer, shape, unsupported size */
#define PE_ERR_LAUNCH 2    /* a kernel launch failed */
#define PE_ERR_TREE 4      /* parents not topological / out of range, tree too large */
#define PE_ERR_CAPACITY 8  /* KV cache capacity exceeded / position out of table */
#define PE_ERR_MASK 16     /* dense bias is not a prefix+ancestor tree mask */
#define PE_ERR_TOKEN 32    /* token id outside the vocabulary */
#define PE_ERR_INDEX 64    /* keep index not strictly increasing / out of range */
#define PE_ERR_WORKSPACE 128 /* workspace too small */
#define PE_ERR_VALUE 256   /* NaN in a logit row, or a row with no finite value */

/* element types */
#define PE_DTYPE_F32 0
#define PE_DTYPE_BF16 1
#define PE_DTYPE_F16 2

/* linear-weight storage formats */
#define PE_WFMT_DENSE 0 /* dtype weights, MFMA-tiled (16-bit) or row-major (fp32) */
#define PE_WFMT_NF4 1   /* NF4 codes + fp16 absmax per 64 along K, MFMA-tiled */
#define PE_WFMT_NF4_F32ABS 2 /* NF4 codes + fp32 absmax (bitsandbytes' own), MFMA-tiled */

/* GEMM epilogues */
#define PE_EPI_STORE 0    /* out = round(acc + bias) */
#define PE_EPI_RESIDUAL 1 /* out = round(resid + round(acc)); out may alias resid */
#define PE_EPI_SWIGLU 2   /* columns interleaved by 32 (gate tile, up tile):
                             out = round(round(silu(round(g))) * round(u)) */

/* row order of the fused q/k/v weight */
#define PE_QKV_PLAIN 0       /* q heads, k heads, v heads; head dims in order */
#define PE_QKV_ROPE_PAIRED 1 /* same heads, dims of each head in 32-row tiles ordered
                                [0,32) [hd/2, hd/2+32) [32,64) [hd/2+32, hd/2+64) ...:
                                the two halves a RoPE pair needs share a GEMM column
                                group; bias stays in plain order (16-bit, hd == 128) */

/* attention masks */
#define PE_MASK_TREE 0   /* rows are tree nodes: whole prefix + ancestor bits */
#define PE_MASK_CAUSAL 1 /* rows are consecutive tokens: key j allowed iff j <= P + row */

/* RMSNorm rounding (fp32 statistics either way) */
#define PE_NORM_HF 0          /* w * round(x * rsqrt(mean(x^2) + eps)): HF LlamaRMSNorm
                                 (modeling_llama.py:62-67), the target's norms */
#define PE_NORM_FP32_WEIGHT 1 /* round(x * rsqrt(mean(x^2) + eps) * float(w)): one rounding,
                                 the drafter's RMSNorm (src/pe/nn.py:22-26) */

/* attention softmax arithmetic */
#define PE_ATTN_SDPA 0  /* fp32 softmax, unnormalised probabilities rounded to the dtype for PV, one
                           division at the end: torch's scaled_dot_product_attention as HF calls it
                           (integrations/sdpa_attention.py:79-154), the target's */
#define PE_ATTN_EAGER 1 /* scores rounded to the dtype (dot product, then / sqrt(hd)), fp32 softmax,
                           normalised probabilities rounded to the dtype before PV: the drafter's
                           attention (src/pe/nn.py:84-87) */

#define PE_TREE_MAX_WORDS 4 /* ancestor bitmask words per node: T <= 256 */

const char* pe_status_string(int status);
int pe_version(void);

/* ---------------------------------------------------------------- synthetic data */
/* Counter-based normal(0, std) fill (splitmix64 hash -> 4x16-bit Irwin-Hall sum),
 * bit-identical to the numpy generator used for fixtures. No reference
 * counterpart: the reference loads hub checkpoints (src/pe/target.py:32-38). */
int pe_fill_normal(void* out, int64_t n, int dtype, uint64_t seed, uint64_t stream_id, double std_,
                   void* stream);
int pe_fill_uniform_int(int64_t* out, int64_t n, int64_t hi, uint64_t seed, uint64_t stream_id,
                        void* stream);

/* ---------------------------------------------------------------- NF4 format */
/* Blockwise NF4 quantisation of fp32 W[N][K] (block 64 along K) into the logical
 * bitsandbytes layout: packed[N*K/2] (element 2j in the high nibble of byte j),
 * absmax[N*K/64] fp16. Nearest code, lowest index on ties. Stands in for the
 * pre-quantized checkpoint the reference loads (src/pe/target.py:32-38). */
int pe_nf4_quantize(const float* w, int64_t N, int64_t K, uint8_t* packed, uint16_t* absmax,
                    void* stream);
/* Logical NF4 -> MFMA-tiled layout read by pe_nf4_gemm. */
int pe_nf4_repack(const uint8_t* packed, const uint16_t* absmax, int64_t N, int64_t K,
                  uint8_t* tiled, uint16_t* tiled_absmax, void* stream);
/* Tiled NF4 -> logical bf16 W[N][K]: bf16_rne(NF4[c] * float(absmax)). Replaces
 * bitsandbytes dequantize_4bit (src/pe/target.py:55-62). */
int pe_nf4_dequant(const uint8_t* tiled, const uint16_t* tiled_absmax, int64_t N, int64_t K,
                   uint16_t* out, void* stream);
/* The same two for fp32 absmax, the type bitsandbytes stores (Params4bit
 * quant_state.absmax; src/pe/target.py:32-38 loads such checkpoints):
 * bf16_rne(NF4[c] * absmax) with the fp32 absmax as is. */
int pe_nf4_repack_f32abs(const uint8_t* packed, const float* absmax, int64_t N, int64_t K, uint8_t* tiled,
                         float* tiled_absmax, void* stream);
int pe_nf4_dequant_f32abs(const uint8_t* tiled, const float* tiled_absmax, int64_t N, int64_t K, uint16_t* out,
                          void* stream);
/* bitsandbytes double quantisation of the absmax (compress_statistics): the
 * fp32 absmax of block i is code[q[i]] * nested_absmax[i / nested_blocksize]
 * + offset, one fp32 product and one fp32 sum, as bitsandbytes'
 * dequantize_blockwise followed by `absmax += offset` in dequantize_4bit.
 * code: the 256-entry nested quant map. */
int pe_nf4_absmax_dequant(const uint8_t* q, int64_t n, const float* code, const float* nested_absmax,
                          int nested_blocksize, float offset, float* absmax, void* stream);
/* Row-major 16-bit W[N][K] -> MFMA-tiled layout read by pe_dense_gemm (copy for fp32). */
int pe_dense_repack(const void* w, int64_t N, int64_t K, int dtype, void* tiled, void* stream);

/* ---------------------------------------------------------------- GEMMs */
/* Bytes of workspace a GEMM of this shape needs (split-K partials + counters). */
int64_t pe_gemm_workspace_bytes(int M, int N, int K, int wfmt, int dtype, int epilogue);
/* Y[M][N] = X[M][K] . deq(W)^T with fp32 accumulation, then the epilogue.
 * Replaces bitsandbytes Linear4bit.forward (dequantize then F.linear) at
 * src/pe/target.py:32-38 / HF modeling_llama.py:175,254-256,280.
 * K % 128 == 0, N % 32 == 0 (N % 64 for PE_EPI_SWIGLU). */
int pe_nf4_gemm(const void* x, int64_t ldx, int M, int K, const uint8_t* w_tiled,
                const uint16_t* absmax_tiled, int N, int epilogue, const void* bias,
                const void* resid, int64_t ld_resid, void* out, int64_t ld_out, void* workspace,
                int64_t workspace_bytes, void* stream);
/* pe_nf4_gemm on fp32-absmax weights (pe_nf4_repack_f32abs). */
int pe_nf4_gemm_f32abs(const void* x, int64_t ldx, int M, int K, const uint8_t* w_tiled, const float* absmax_tiled,
                       int N, int epilogue, const void* bias, const void* resid, int64_t ld_resid, void* out,
                       int64_t ld_out, void* workspace, int64_t workspace_bytes, void* stream);
/* pe_nf4_gemm on the activation layout the fused pass hands between kernels:
 * x is A-tiled (element (m, k) at ((((m/32)*(K/128) + k/128)*8 + (k%64)/8)*64
 * + m%32 + 32*((k%128)/64))*8 + k%8), M <= 64; with out_units > 0 (N/128 for
 * PE_EPI_STORE, N/256 for PE_EPI_SWIGLU) the output is A-tiled too (not with
 * PE_EPI_RESIDUAL). Same kernels and results as pe_nf4_gemm; no counterpart in
 * the reference (a layout variant of its dequantize + F.linear, used by the
 * pass and timed on its own by the benchmark). 64 < M <= 256: PE_EPI_SWIGLU
 * with an A-tiled output (out_units = N/256) only, the batched pass's gate/up
 * linear (the many-row kernel; workspace of pe_gemm_workspace_bytes). */
int pe_nf4_gemm_tiled(const void* x_tiled, int M, int K, const uint8_t* w_tiled, const uint16_t* absmax_tiled,
                      int N, int epilogue, const void* bias, const void* resid, int64_t ld_resid, void* out,
                      int64_t ld_out, int out_units, void* workspace, int64_t workspace_bytes, void* stream);
/* The NF4 linear as fp32 split partials: partials[S][M][N] with
 * sum_s partials[s] = X . deq(W)^T (sum in split order s = 0 .. S-1), written
 * with plain stores and no exchange between workgroups; *splits (host memory)
 * receives S. X row-major (ldx) or A-tiled (x_tiled != 0). M <= 64, K % 128 == 0,
 * N % 32 == 0; or 64 < M <= 256 with A-tiled X and N % 128 == 0 (the many-row
 * kernel: each weight dequantised once for all rows). Layout variant of
 * pe_nf4_gemm with no reference counterpart: the pass's residual + RMSNorm,
 * RoPE and SwiGLU kernels consume it. */
int64_t pe_nf4_gemm_partials_bytes(int M, int N, int K);
int pe_nf4_gemm_partials(const void* x, int64_t ldx, int x_tiled, int M, int K, const uint8_t* w_tiled,
                         const uint16_t* absmax_tiled, int N, float* partials, int64_t partial_bytes, int* splits,
                         void* stream);
/* pe_dense_gemm with PE_EPI_STORE (16-bit dtypes, no bias) that also writes,
 * per output row and column group g, the argmax key of the group's stored
 * values: keys[row * groups + g] = (order-preserving value bits << 32) |
 * (0xFFFFFFFF - column), so the largest key of a row names its largest value
 * at its lowest column (NaN largest), torch.argmax's result. groups =
 * pe_dense_gemm_argmax_groups(M, N, K). The reference's walk takes
 * logits.argmax(-1) of each node row after the lm_head (verify.py:52,120;
 * HF modeling_llama.py:480); this folds that argmax into the lm_head. */
int pe_dense_gemm_argmax_groups(int M, int N, int K);
int pe_dense_gemm_argmax(const void* x, int64_t ldx, int M, int K, const void* w, int dtype, int N, void* out,
                         int64_t ld_out, uint64_t* keys, void* workspace, int64_t workspace_bytes, void* stream);
/* Dense linear in dtype (bf16/fp16 MFMA on tiled weights, fp32 VALU on row-major).
 * Replaces F.linear in HF modeling_llama.py:175,254-256,280,480. */
int pe_dense_gemm(const void* x, int64_t ldx, int M, int K, const void* w, int dtype, int N,
                  int epilogue, const void* bias, const void* resid, int64_t ld_resid, void* out,
                  int64_t ld_out, void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- elementwise */
/* out[m][:] = table[ids[m]][:]. HF modeling_llama.py:381 (embed_tokens). */
int pe_embed(const int64_t* ids, int M, const void* table, int64_t V, int H, int dtype, void* out,
             int64_t ld_out, int32_t* status, void* stream);
/* HF LlamaRMSNorm (modeling_llama.py:62-67): w * round(x * rsqrt(mean(x^2) + eps)). */
int pe_rmsnorm(const void* x, int64_t ldx, int M, int H, const void* w, float eps, int dtype,
               void* out, int64_t ld_out, void* stream);
/* pe_rmsnorm with the rounding chosen by `mode` (PE_NORM_*): PE_NORM_FP32_WEIGHT
 * is the drafter's RMSNorm.forward (src/pe/nn.py:22-26), used for its
 * feat_norm (src/pe/drafter.py:130). */
int pe_rmsnorm_ex(const void* x, int64_t ldx, int M, int H, const void* w, float eps, int dtype, int mode,
                  void* out, int64_t ld_out, void* stream);
/* RoPE at the given positions on q and k of a fused qkv row block, HF
 * apply_rotary_pos_emb (modeling_llama.py:130-160); writes roped q to q_out
 * [M][nh][hd] and appends k, v at cache rows [row0, row0 + M) in place of
 * DynamicLayer.update's torch.cat (HF cache_utils.py:127-146).
 * cos_sin: [max_pos][hd] cos followed by [max_pos][hd] sin, in dtype. */
int pe_rope_qkv(const void* qkv, int64_t ld_qkv, int M, int nh, int nkv, int hd,
                const int64_t* positions, const void* cos_sin, int64_t max_pos, int dtype,
                void* q_out, void* k_cache, void* v_cache, int64_t cache_cap, int64_t row0,
                int32_t* status, void* stream);
/* dst[m][0:H] = src[m][0:H] (feature capture, src/pe/target.py:161-162). */
int pe_copy_rows(const void* src, int64_t ld_src, int M, int64_t row_bytes, void* dst,
                 int64_t ld_dst, void* stream);

/* ---------------------------------------------------------------- tree masks */
/* Per-node ancestor bitmask (bits[t][w], bit u set iff node u is t or an
 * ancestor of t), depth and position P + depth. Replaces tree_depths /
 * tree_allow_mask / tree_position_ids (src/pe/masks.py:118-156). */
int pe_tree_masks(const int32_t* parents, int T, int64_t P, uint64_t* bits, int words,
                  int64_t* positions, int32_t* depths, int32_t* status, void* stream);
/* Dense bool allow matrix (P+T)^2 from the bitmasks (masks.py:127-147). */
int pe_tree_allow_dense(const uint64_t* bits, int T, int words, int64_t P, uint8_t* allow,
                        void* stream);
/* Additive bias (T rows of a (.., T, P+T) mask, to_additive_bias masks.py:29-33)
 * back to bitmasks; PE_ERR_MASK if a prefix column is masked or a value is
 * neither 0 nor <= finfo(dtype).min / 2. */
int pe_bias_to_bits(const void* bias, int64_t ld_bias, int dtype, int T, int64_t P,
                    uint64_t* bits, int words, int32_t* status, void* stream);

/* ---------------------------------------------------------------- attention */
int64_t pe_attention_workspace_bytes(int T, int nh, int nkv, int hd, int64_t kv_len, int dtype);
/* softmax(q k^T * scale + mask) v over cache rows [0, P + T) of one layer,
 * replacing HF sdpa_attention_forward (integrations/sdpa_attention.py:79-154)
 * with the tree bias of masks.py:127-147. q [T][nh][hd], caches [nkv][cap][hd],
 * out [T][ld_out] with head h at columns [h*hd, (h+1)*hd). The workspace's
 * first 4 KiB are arrival counters: zero before the first call; every call
 * leaves them multiples of 16. bf16 / fp16 with hd = 128 (the matrix-core
 * path) requires scale > 0 (1/sqrt(hd) in every model) and cache_cap < 2^24
 * rows, else PE_ERR_ARG. */
int pe_tree_attention(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap,
                      int nh, int nkv, int hd, int T, int64_t P, int mask_mode,
                      const uint64_t* bits, int words, float scale, int dtype, void* out,
                      int64_t ld_out, void* workspace, int64_t workspace_bytes, void* stream);

/* The same attention for B sequences in one launch, each over its own cache
 * (per sequence HF sdpa_attention_forward, integrations/sdpa_attention.py:79-154,
 * with the tree bias of masks.py:127-147, as serve.py:289-297 runs it for one
 * sequence). Sequence b's nodes are rows [seq_row0[b], seq_row0[b + 1]) of q
 * [M][nh][128], bits [M][words] and out [M][ld_out]; its keys are its
 * seq_prefix[b] cached rows (device memory) followed by its node rows, in
 * k_cache / v_cache + b * seq_stride elements ([nkv][cap][128] per sequence).
 * max_rows and max_prefix bound every sequence's node count and prefix and
 * size the launch (a sequence beyond them is skipped). bf16 / fp16, hd = 128.
 * workspace: pe_attention_batch_workspace_bytes bytes, its first 4 KiB arrival
 * counters (zero before the first call; every call leaves them zero). */
int64_t pe_attention_batch_workspace_bytes(int max_rows, int nh, int nkv, int64_t max_kv_len, int batch);
int pe_tree_attention_batch(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap,
                            int64_t seq_stride, int nh, int nkv, int max_rows, int64_t max_prefix, int batch,
                            const int32_t* seq_row0, const int64_t* seq_prefix, const uint64_t* bits, int words,
                            float scale, int dtype, void* out, int64_t ld_out, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- acceptance */
/* Row argmax (first index among equal maxima; NaN counts as the maximum). */
int pe_argmax_rows(const void* x, int64_t ld, int rows, int64_t V, int dtype, int32_t* out_idx,
                   void* stream);
/* Greedy tree walk of accept_tree_cached (src/pe/decode/verify.py:104-125):
 * out[0] = |path|, out[1] = bonus token, out[2 + i] = path node i.
 * One launch: per-row argmax blocks, the last of which walks.
 * scratch: T + 2 int32 (an arrival counter at index 0, then the row
 * argmaxes), zero before the first call; every call leaves the counter at
 * zero again, so one buffer serves calls of any T. Calls that share a
 * scratch buffer must not overlap. T <= 64 * PE_TREE_MAX_WORDS. */
int pe_accept_tree(const void* root_logit, const void* node_logits, int64_t ld, int T, int64_t V,
                   int dtype, const int64_t* node_tokens, const int32_t* parents, int32_t* out,
                   int32_t* scratch, void* stream);
/* accept_tree_cached (src/pe/decode/verify.py:104-125) with each node row's
 * argmax (verify.py:120) taken from the argmax keys that pe_dense_gemm_argmax
 * (or pe_forward with node_keys) wrote with the logits, [T][groups], instead of
 * re-reading the T node rows; the root row is read as in pe_accept_tree.
 * Same outputs, scratch and limits as pe_accept_tree. */
int pe_accept_tree_keys(const void* root_logit, int64_t V, int dtype, const uint64_t* node_keys, int groups,
                        int T, const int64_t* node_tokens, const int32_t* parents, int32_t* out,
                        int32_t* scratch, void* stream);
/* pe_accept_tree without a scratch argument and without any allocation: the
 * scratch is a library-owned device array of PE_ACCEPT_NOALLOC_MAX_NODES + 2
 * int32 per GPU (held until the process ends), its counter cleared by a small
 * kernel before each walk. No counterpart in the reference: for callers that
 * cannot allocate (HIP graph capture, serving loops that forbid hipMalloc).
 * T > PE_ACCEPT_NOALLOC_MAX_NODES returns PE_ERR_TREE. Every call on one GPU
 * shares that array: calls that overlap on one GPU (other streams, other
 * threads) race. */
#define PE_ACCEPT_NOALLOC_MAX_NODES (64 * PE_TREE_MAX_WORDS)
int pe_accept_tree_noalloc(const void* root_logit, const void* node_logits, int64_t ld, int T, int64_t V,
                           int dtype, const int64_t* node_tokens, const int32_t* parents, int32_t* out,
                           void* stream);
/* Move accepted rows P + path[i] -> P + i in every layer's K and V, in place;
 * path read from a pe_accept_tree result on the device. Replaces
 * TargetModel.gather_cache (src/pe/target.py:194-201) for the keep index
 * serve.py:308-309 builds. Caches [L][nkv][cap][hd]. */
int pe_kv_compact(void* k_cache, void* v_cache, int L, int nkv, int64_t cap, int hd, int dtype,
                  int64_t P, const int32_t* accept_out, void* stream);
/* General in-place gather of rows keep[0..n) (strictly increasing) on the
 * sequence axis, gather_cache with an arbitrary keep index. */
int pe_kv_gather(void* k_cache, void* v_cache, int L, int nkv, int64_t cap, int hd, int dtype,
                 const int64_t* keep, int64_t n_keep, int32_t* status, void* stream);

/* ------------------------------------------------------------ batched trees */
/* The batched workload's per-sequence steps (no single reference function: the
 * reference verifies one sequence at a time, src/pe/serve.py:289-314, and this
 * is that step for each of `batch` sequences in one launch). Rows of sequence
 * b are [seq_row0[b], seq_row0[b+1]) (device int32 [batch + 1]); parents are in
 * each sequence's own node numbering. */
/* tree_depths / tree_allow_mask / tree_position_ids (src/pe/masks.py:118-156)
 * per sequence: positions = seq_prefix[b] + depth. */
int pe_tree_masks_batch(const int32_t* parents, const int32_t* seq_row0, const int64_t* seq_prefix, int batch,
                        int max_seq_rows, uint64_t* bits, int words, int64_t* positions, int32_t* depths,
                        int32_t* status, void* stream);
/* accept_tree_cached (src/pe/decode/verify.py:104-125) per sequence: root row
 * root_logits + b * ld_root; out[b * (2 + max_seq_rows) + ...] as
 * pe_accept_tree's out; scratch batch * (max_seq_rows + 2) int32, zero before
 * the first call and left zero. */
int pe_accept_tree_batch(const void* root_logits, int64_t ld_root, const void* node_logits, int64_t ld, int64_t V,
                         int dtype, const int32_t* seq_row0, int batch, int max_seq_rows, const int64_t* node_tokens,
                         const int32_t* parents, int32_t* out, int32_t* scratch, void* stream);
/* gather_cache with the accepted-path keep index (src/pe/target.py:194-201,
 * src/pe/serve.py:308-309) per sequence: in sequence b's cache (k_cache /
 * v_cache + b * cache_seq_stride elements) rows seq_prefix[b] + path[i] move
 * to seq_prefix[b] + i, the path read from pe_accept_tree_batch's out. */
int pe_kv_compact_batch(void* k_cache, void* v_cache, int batch, int64_t cache_seq_stride, int L, int nkv,
                        int64_t cap, int hd, int dtype, const int64_t* seq_prefix, const int32_t* accept_out,
                        int max_seq_rows, void* stream);

/* ------------------------------------------------------------ tree proposal */
#define PE_PROPOSE_MAX_DEPTH 16
#define PE_PROPOSE_MAX_WIDTH 64
/* Beam tree proposal of propose_tree (src/pe/decode/tree.py:34-55) on k rows
 * of draft logits already on the device (row d predicts depth d; a caller
 * with `pending` confirmed depths passes the row after them). For depth d:
 * log_softmax in fp32; the top c_d = min(top_k, widths[d]) tokens (value
 * descending, the lowest index first among equal values); every surviving
 * parent extended by them; the candidates stably ordered by cumulative
 * log-probability (float64 sums, as the reference's Python floats) and the
 * best widths[d] kept (fewer when the parents times c_d are fewer).
 * The reference's rule is widths[d] = max(1, min(top_k, max_nodes / k)).
 * widths: host array of k values in [1, PE_PROPOSE_MAX_WIDTH]; c_d <= V.
 * node_tokens (int64) and parents (int32, -1 = hangs off the prefix) receive
 * the nodes in topological order; *n_nodes (host) their count, known on the
 * host before the kernels run. scratch: k * PE_PROPOSE_SCRATCH_PER_DEPTH
 * bytes of device memory. status: PE_ERR_VALUE when a row holds a NaN or no
 * finite value (the reference's order is undefined there). */
#define PE_PROPOSE_SCRATCH_PER_DEPTH 512
int pe_propose_tree(const void* logits, int64_t ld, int k, int64_t V, int dtype, const int32_t* widths, int top_k,
                    int64_t* node_tokens, int32_t* parents, int32_t* n_nodes, void* scratch, int32_t* status,
                    void* stream);

/* ------------------------------------------------------------ decode loop */
/* The bookkeeping that ends one step of the reference's one-forward tree loop
 * (src/pe/serve.py:305-343: the accepted path's features appended with
 * torch.cat, the tokens emitted, root_logit re-rooted, the pending bonus),
 * kept in device memory so that a recorded step needs no host value:
 * state (int64 [2]) = {P: tokens cached and featurised, the pending bonus};
 * ids (int64 [cap]) the context tokens with the pending one at ids[P]; feats
 * ([cap][feat_dim] in dtype) their fused features; root ([V]) the logit row
 * that predicted ids[P]. With a walk's result [n, bonus, path...]
 * (pe_accept_tree*): feats / ids rows P + i take node path[i]'s fused row and
 * token (i < n), root takes node path[n-1]'s logit row, ids[P + n] = bonus
 * becomes pending and P += n; n == 0 changes nothing (the caller then runs the
 * one-node miss pass of serve.py:315-328 and pe_loop_miss_commit). rec (int32,
 * read by the host once per step): rec[0] = n, rec[1] = bonus, rec[2] |= the
 * status words given (each cleared; NULL entries skipped), rec[4 + i] (i <
 * rec_path) the accepted tokens, -1 past n. */
#define PE_LOOP_REC_HEAD 4
int pe_loop_commit(const int32_t* accept_out, int T, const int64_t* node_tokens, const void* node_fused,
                   int feat_dim, const void* node_logits, int64_t V, int dtype, void* feats, int64_t* ids,
                   void* root, int64_t cap, int64_t* state, int32_t* rec, int rec_path, int32_t* status0,
                   int32_t* status1, int32_t* status2, void* stream);
/* After the miss pass (the pending token at position P, its logit row written
 * to root): feats row P takes its fused row, its argmax (from the lm_head's
 * argmax keys [groups], or from row_argmax[0] as pe_argmax_rows wrote it:
 * exactly one of the two) becomes the pending bonus at ids[P + 1], P += 1;
 * rec[3] = that bonus, rec[2] |= the status words. */
int pe_loop_miss_commit(const void* fused_row, int feat_dim, const uint64_t* keys, int groups,
                        const int32_t* row_argmax, int dtype, void* feats, int64_t* ids, int64_t cap, int64_t* state,
                        int32_t* rec, int32_t* status0, int32_t* status1, int32_t* status2, void* stream);

/* ---------------------------------------------------------------- whole pass */
typedef struct pe_model_desc {
  int32_t num_layers, hidden, num_heads, num_kv_heads, head_dim, intermediate, vocab;
  int32_t intermediate_padded; /* intermediate rounded up to 32 */
  int32_t dtype;               /* activations, norms, embeddings, lm_head, KV */
  int32_t weight_format;       /* PE_WFMT_* of the per-layer linears */
  int32_t qkv_layout;          /* PE_QKV_* row order of w_qkv */
  float rms_eps;
  int32_t norm_mode;        /* PE_NORM_* of the per-layer norms; the final norm is PE_NORM_HF */
  int32_t embed_rows;       /* rows of `embed` (ids must lie below); 0 = vocab */
  int32_t attn_mode;        /* PE_ATTN_* of every layer */
  int32_t _reserved;
  int64_t max_positions;
  const void* embed;        /* [embed_rows or V][H] */
  const void* final_norm;   /* [H] */
  const void* lm_head;      /* dense [V][H], tiled for 16-bit dtypes */
  const void* rope_cos_sin; /* [max_pos][hd] cos, then [max_pos][hd] sin */
  /* arrays of num_layers pointers */
  const void* const* attn_norm;
  const void* const* mlp_norm;
  const void* const* w_qkv; /* N = (nh + 2 nkv) * hd */
  const void* const* a_qkv; /* NF4 absmax (NULL entries for dense) */
  const void* const* b_qkv; /* bias [N] or NULL entries */
  const void* const* w_o;
  const void* const* a_o;
  const void* const* w_gu; /* gate/up interleaved by 32 rows, N = 2 * intermediate_padded */
  const void* const* a_gu;
  const void* const* w_down; /* K = intermediate_padded */
  const void* const* a_down;
} pe_model_desc;

typedef struct pe_pass_args {
  const int64_t* input_ids; /* [M] */
  const int64_t* positions; /* [M] */
  int32_t M;                /* rows of this pass (tree nodes or tokens) */
  int32_t mask_mode;        /* PE_MASK_TREE | PE_MASK_CAUSAL */
  int64_t prefix_len;       /* P: new K/V rows land at [P, P + M) */
  const uint64_t* tree_bits;
  int32_t bits_words;
  int32_t num_features;     /* hidden-state slots to fuse (0..4) */
  int32_t feature_layers[4];/* 0 = embeddings, i < L = after layer i, L = final norm */
  int32_t _pad;
  void* k_cache;
  void* v_cache;
  int64_t cache_capacity;
  void* logits; /* [M][V] or NULL */
  void* fused;  /* [M][num_features * H] or NULL */
  void* workspace;
  int64_t workspace_bytes;
  int32_t* status;
  /* Batched verification (batch >= 1; 0 = the single sequence above): `batch`
   * independent sequences, each a tree over its own cached prefix. Sequence b
   * owns rows [seq_row0[b], seq_row0[b+1]) of the pass (device int32
   * [batch + 1], seq_row0[0] = 0, seq_row0[batch] = M), its cache is k_cache /
   * v_cache + b * cache_seq_stride elements (each [L][nkv][cache_capacity][hd])
   * with seq_prefix[b] rows cached (device int64 [batch]); tree_bits of a row
   * name nodes of its own sequence (pe_tree_masks_batch). prefix_len is the
   * largest seq_prefix and max_seq_rows the largest row count: they size the
   * launches; a sequence whose device prefix or row count exceeds them sets
   * PE_ERR_CAPACITY / PE_ERR_TREE in status and is skipped (no K/V written,
   * no key read past the bounds). A row's K/V land at its sequence's rows
   * [prefix, prefix + rows). 16-bit models with hd 128 and RoPE-paired q/k/v,
   * PE_MASK_TREE. batch == 1 with M <= 64 rows (max_seq_rows == M) runs the
   * single-sequence pass with its prefix read from seq_prefix[0] on the
   * device: one recorded launch sequence (a HIP graph) serves every prefix up
   * to prefix_len, and for seq_prefix[0] == prefix_len the result equals the
   * batch == 0 pass bit for bit. */
  int32_t batch;
  int32_t max_seq_rows;
  const int32_t* seq_row0;
  const int64_t* seq_prefix;
  int64_t cache_seq_stride;
  /* Optional (single-sequence 16-bit passes of at most 64 rows with logits,
   * batch 0 or 1): the lm_head also writes each row's argmax keys,
   * [M][pe_dense_gemm_argmax_groups(M, vocab, hidden)] (see
   * pe_dense_gemm_argmax), for pe_accept_tree_keys. NULL: none. */
  uint64_t* node_keys;
} pe_pass_args;

/* Workspace for pe_forward with up to M rows and kv_len = P + M keys. */
int64_t pe_forward_workspace_bytes(const pe_model_desc* m, int M, int64_t kv_len);
/* Workspace for a batched pe_forward: M rows in all, at most max_seq_rows per
 * sequence, at most max_kv_len = prefix + rows keys per sequence. */
int64_t pe_forward_batch_workspace_bytes(const pe_model_desc* m, int M, int max_seq_rows, int64_t max_kv_len,
                                         int batch);
/* The masked verification forward TargetModel.forward_cached
 * (src/pe/target.py:203-224 -> HF LlamaForCausalLM / Qwen2ForCausalLM forward,
 * modeling_llama.py:347-490): embeddings, L decoder layers with in-place KV
 * append, final norm, lm_head over all M rows, fused features.
 * A causal pass of more than 256 rows of a 16-bit model with 128-dim heads, NF4
 * or dense (a prefill), runs every linear once over all rows in blocks of 256
 * rows on the matrix cores (each NF4 weight dequantised once per block inside
 * the GEMM) and attention once over all rows. Set PE_PREFILL_GEMM=0 to run such
 * passes in 64-row chunks of the fused pass instead.
 * A tree pass (batch 0) of 65 to 64 * PE_TREE_MAX_WORDS nodes on such a model
 * runs as a batch of one sequence (its sequence table written into the
 * workspace, which pe_forward_workspace_bytes covers); node_keys must be NULL. */
int pe_forward(const pe_model_desc* m, const pe_pass_args* a, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PE_HIP_H */
