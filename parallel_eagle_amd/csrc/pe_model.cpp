// Whole verification pass: the decoder forward of TargetModel.forward_cached
// (src/pe/target.py:203-224 -> HF modeling_llama.py:367-480), launched from
// C++ as one sequence of kernels on the caller's stream so a host loop over
// layers never sits between launches (and the sequence can be captured in a
// HIP graph by the caller).
//
// Per layer:
//   rmsnorm -> qkv linear (+bias) -> RoPE + in-place K/V append -> tree attention
//   -> o linear (+residual) -> rmsnorm -> gate/up linear (SwiGLU epilogue)
//   -> down linear (+residual)
// then final rmsnorm and lm_head over all rows. Hidden-state slots for the fused
// features follow HF's output_hidden_states tuple: slot 0 = embeddings, slot
// i in [1, L) = residual stream after layer i, slot L = final-norm output
// (HF utils/output_capturing.py:269-277; src/pe/target.py:161-162).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "../../include/pe_hip.h"
#include "pe_internal.h"

namespace {

constexpr int64_t kAlign = 256;
constexpr int64_t kCounterBytes = 32768;

int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
int esize(int dtype) { return dtype == PE_DTYPE_F32 ? 4 : 2; }

// Offsets into the pass workspace. The GEMM arrival counters sit at the head
// of the GEMM region, at offset 0 whatever M is, so a counter is never memory
// another pass shape used for data; they are zero on first use and every
// launch leaves them zero.
struct Layout {
  int64_t gemm;  // GEMM arrival counters, then split-K partials
  int64_t gemm_bytes;
  int64_t h, xn, qkv, q, attn, act, attn_ws, attn_ws_bytes;
  int64_t xn_t, attn_t, act_t;  // A-tiled GEMM inputs of the fused pass
  int64_t part, part_bytes;      // split partials of the fused NF4 pass's GEMMs
  int64_t kvoff;                 // per-row K/V slots of a pass whose prefix is read on the device
  int64_t total;
};

// The 16-bit pass with fused epilogues (see pe_forward) needs the q/k/v rows
// in RoPE-paired order and hd == 128 attention.
bool fused_path(const pe_model_desc* m, int M) {
  return m->dtype != PE_DTYPE_F32 && m->qkv_layout == PE_QKV_ROPE_PAIRED && m->head_dim == 128 && M <= 64;
}

// A tree pass of more nodes than one fused chunk (65 up to the bitmask limit):
// it runs as a batch of one sequence on the batched pass's kernels (each NF4
// weight dequantised once for all rows), its sequence table written into the
// workspace after the batch layout.
bool wide_tree_path(const pe_model_desc* m, int M) {
  return m->dtype != PE_DTYPE_F32 && m->qkv_layout == PE_QKV_ROPE_PAIRED && m->head_dim == 128 &&
         m->attn_mode == PE_ATTN_SDPA && M > 64 && M <= 64 * PE_TREE_MAX_WORDS;
}
constexpr int64_t kOneSeqBytes = 256;  // seq_row0 {0, M} at +0, seq_prefix {P} at +16

// The fused pass hands the GEMMs their X A-tiled (see xtile_index): NF4 and
// dense 16-bit weights alike (the dense kernel's X loads then read whole
// cache lines), except with eager attention (the drafter's), whose output is
// row-major.
bool tiled_path(const pe_model_desc* m, int M) {
  return fused_path(m, M) && (pe_wfmt_nf4(m->weight_format) || m->weight_format == PE_WFMT_DENSE) &&
         m->attn_mode != PE_ATTN_EAGER && m->hidden % 128 == 0 &&
         (m->num_heads * m->head_dim) % 128 == 0 && m->intermediate_padded % 128 == 0;
}

int64_t xtile_bytes(int M, int K) { return (int64_t)((M + 31) / 32) * K * 64; }

int64_t gemm_ws(const pe_model_desc* m, int M, int N, int K, int epi) {
  const int wf = m->weight_format;
  return pe_gemm_workspace_bytes(M, N, K, wf, m->dtype, epi);
}

Layout make_layout(const pe_model_desc* m, int M, int64_t kv_len) {
  Layout L;
  const int es = esize(m->dtype);
  const int H = m->hidden, qd = m->num_heads * m->head_dim, kvd = m->num_kv_heads * m->head_dim;
  const int nqkv = qd + 2 * kvd, ip = m->intermediate_padded;
  int64_t g = kCounterBytes;
  int64_t cand[6] = {gemm_ws(m, M, nqkv, H, PE_EPI_STORE), gemm_ws(m, M, H, qd, PE_EPI_RESIDUAL),
                     gemm_ws(m, M, 2 * ip, H, PE_EPI_SWIGLU), gemm_ws(m, M, H, ip, PE_EPI_RESIDUAL),
                     pe_gemm_workspace_bytes(M, m->vocab, H, PE_WFMT_DENSE, m->dtype, PE_EPI_STORE), 0};
  if (fused_path(m, M)) cand[5] = pe_internal_gemm_rope_kv_bytes(M, nqkv, H, m->weight_format);
  for (int i = 0; i < 6; ++i)
    if (cand[i] > g) g = cand[i];
  int64_t off = 0;
  L.gemm = off;
  L.gemm_bytes = align_up(g);
  off += L.gemm_bytes;
  L.h = off; off += align_up((int64_t)M * H * es);
  const int xw = H > ip ? H : ip;
  L.xn = off; off += align_up((int64_t)M * (xw > qd ? xw : qd) * es);
  L.qkv = off; off += align_up((int64_t)M * nqkv * es);
  L.q = off; off += align_up((int64_t)M * qd * es);
  L.attn = off; off += align_up((int64_t)M * qd * es);
  L.act = off; off += align_up((int64_t)M * ip * es);
  L.xn_t = L.attn_t = L.act_t = L.part = L.part_bytes = 0;
  if (tiled_path(m, M)) {
    L.xn_t = off; off += align_up(xtile_bytes(M, H));
    L.attn_t = off; off += align_up(xtile_bytes(M, qd));
    L.act_t = off; off += align_up(xtile_bytes(M, ip));
  }
  if (fused_path(m, M)) {  // o and down write split partials (NF4 and dense)
    const int wf = m->weight_format;
    const int64_t pb[2] = {pe_internal_linear_partials_bytes(M, H, qd, wf),
                           pe_internal_linear_partials_bytes(M, H, ip, wf)};
    for (int i = 0; i < 2; ++i)
      if (pb[i] > L.part_bytes) L.part_bytes = pb[i];
    L.part_bytes = align_up(L.part_bytes);
    L.part = off; off += L.part_bytes;
  }
  L.attn_ws = off;
  L.attn_ws_bytes = align_up(attention_workspace_bytes(M, m->num_heads, m->num_kv_heads, m->head_dim, kv_len,
                                                       m->dtype, m->attn_mode));
  off += L.attn_ws_bytes;
  L.kvoff = off;
  off += align_up((int64_t)M * 8);
  L.total = off;
  return L;
}

// Rows of the embedding table the pass gathers from.
int64_t embed_rows(const pe_model_desc* m) { return m->embed_rows > 0 ? m->embed_rows : m->vocab; }

int linear(const pe_model_desc* m, const void* x, int64_t ldx, int M, int K, const void* w, const void* a, int N,
           int epi, const void* bias, const void* resid, int64_t ldr, void* out, int64_t ldo, void* ws, int64_t wsb,
           hipStream_t st) {
  if (m->weight_format == PE_WFMT_NF4)
    return pe_nf4_gemm(x, ldx, M, K, (const uint8_t*)w, (const uint16_t*)a, N, epi, bias, resid, ldr, out, ldo, ws,
                       wsb, st);
  if (m->weight_format == PE_WFMT_NF4_F32ABS)
    return pe_nf4_gemm_f32abs(x, ldx, M, K, (const uint8_t*)w, (const float*)a, N, epi, bias, resid, ldr, out, ldo,
                              ws, wsb, st);
  return pe_dense_gemm(x, ldx, M, K, w, m->dtype, N, epi, bias, resid, ldr, out, ldo, ws, wsb, st);
}

}  // namespace

extern "C" const char* pe_status_string(int status) {
  if (status == PE_OK) return "ok";
  if (status & PE_ERR_ARG) return "invalid argument";
  if (status & PE_ERR_LAUNCH) return "kernel launch failed";
  if (status & PE_ERR_TREE) return "parents are not a topologically ordered tree (or tree too large)";
  if (status & PE_ERR_CAPACITY) return "KV cache capacity or position table exceeded";
  if (status & PE_ERR_MASK) return "attention bias is not a prefix + ancestor tree mask";
  if (status & PE_ERR_TOKEN) return "token id outside the vocabulary";
  if (status & PE_ERR_INDEX) return "keep index not strictly increasing or out of range";
  if (status & PE_ERR_WORKSPACE) return "workspace too small";
  return "unknown error";
}

extern "C" int pe_version(void) { return 1; }

constexpr int kFusedChunk = 64;  // rows per fused pass (causal passes are chunked)

// ---------------------------------------------------------------------------
// Prefill (a causal pass of more than 256 rows of a 16-bit model, NF4 or
// dense, with RoPE-paired q/k/v and 128-dim heads): every linear runs once
// over all M rows in blocks of 256 rows on the matrix cores
// (pe_internal_nf4_prefill: each NF4 weight dequantised once per row block by
// producer waves; pe_internal_dense_bigm: 16-bit tiled weights), with the
// activations A-tiled between kernels. The GEMMs write fp32 sums that the
// fused pass's epilogue kernels treat as one split: RoPE + K/V append for
// q/k/v, SwiGLU for a dense gate/up (the NF4 gate/up stores the activation
// itself), residual + RMSNorm (with the captures) after o and down.
// Attention runs once over all rows, causally. NF4 weights with fp32 absmax
// (checkpoint imports) are dequantised and tiled to 16-bit once per linear
// and prefill. Shorter causal passes run as 64-row chunks of the fused pass.
// ---------------------------------------------------------------------------
constexpr int kPrefillMinRows = 4 * kFusedChunk + 1;
bool prefill_path(const pe_model_desc* m, int M, int mask_mode) {
  static const bool on = [] {
    const char* v = getenv("PE_PREFILL_GEMM");
    return !v || atoi(v) != 0;
  }();
  return on && M >= kPrefillMinRows && mask_mode == PE_MASK_CAUSAL &&
         (pe_wfmt_nf4(m->weight_format) || m->weight_format == PE_WFMT_DENSE) &&
         m->qkv_layout == PE_QKV_ROPE_PAIRED && m->dtype != PE_DTYPE_F32 && m->head_dim == 128 &&
         m->hidden % 128 == 0 && m->intermediate_padded % 128 == 0 && (m->num_heads * m->head_dim) % 128 == 0 &&
         ((m->num_heads + 2 * m->num_kv_heads) * m->head_dim) % 128 == 0 && m->vocab % 128 == 0;
}

struct PrefillLayout {
  int64_t h, xn, xn_t, q, attn, attn_t, act_t, y, wdeq, wtile, attn_ws, attn_ws_bytes, gemm, gemm_bytes, total;
};

PrefillLayout make_prefill_layout(const pe_model_desc* m, int M, int64_t kv_len) {
  PrefillLayout L;
  const int64_t H = m->hidden, qd = (int64_t)m->num_heads * m->head_dim;
  const int64_t nqkv = qd + 2ll * m->num_kv_heads * m->head_dim, ip = m->intermediate_padded;
  // offset 0: the pass's arrival counters, as in the fused layout (the GEMM
  // and attention counter slices rest at zero between passes, whichever path
  // ran last)
  L.gemm = 0;
  L.gemm_bytes = align_up(kCounterBytes);
  int64_t off = L.gemm_bytes;
  auto take = [&](int64_t bytes) {
    const int64_t o = off;
    off += align_up(bytes);
    return o;
  };
  L.h = take(M * H * 2);
  L.xn = take(M * H * 2);
  L.xn_t = take(xtile_bytes(M, (int)H));
  L.q = take(M * qd * 2);
  L.attn = take(M * qd * 2);
  L.attn_t = take(xtile_bytes(M, (int)qd));
  L.act_t = take(xtile_bytes(M, (int)ip));
  int64_t ny = nqkv;
  if (2 * ip > ny) ny = 2 * ip;
  if (H > ny) ny = H;
  L.y = take(M * ny * 4 * 2);  // up to two K splits of fp32 partials
  L.wdeq = L.wtile = 0;
  if (m->weight_format == PE_WFMT_NF4_F32ABS) {  // one linear dequantised, then tiled
    int64_t nw = nqkv * H;
    if (2 * ip * H > nw) nw = 2 * ip * H;
    if (H * ip > nw) nw = H * ip;
    if (H * qd > nw) nw = H * qd;
    L.wdeq = take(nw * 2);
    L.wtile = take(nw * 2);
  }
  L.attn_ws_bytes = align_up(attention_workspace_bytes(M, m->num_heads, m->num_kv_heads, m->head_dim, kv_len,
                                                       m->dtype, m->attn_mode));
  L.attn_ws = take(L.attn_ws_bytes);
  L.total = off;
  return L;
}

// The lm_head over the final normed rows (row-major xn, or A-tiled in the
// tiled fused pass); with a->node_keys (single-sequence 16-bit passes) the
// GEMM also writes each row's argmax keys.
int lm_head(const pe_model_desc* m, const pe_pass_args* a, const void* xn, bool x_tiled, int M, void* ws,
            int64_t wsb, hipStream_t st) {
  const int H = m->hidden;
  if (x_tiled)
    return pe_internal_dense_gemm_tiled(xn, M, H, m->lm_head, m->dtype, m->vocab, a->logits, m->vocab, a->node_keys,
                                        ws, wsb, st);
  if (a->node_keys)
    return pe_dense_gemm_argmax(xn, H, M, H, m->lm_head, m->dtype, m->vocab, a->logits, m->vocab, a->node_keys, ws,
                                wsb, st);
  return pe_dense_gemm(xn, H, M, H, m->lm_head, m->dtype, m->vocab, PE_EPI_STORE, nullptr, nullptr, 0, a->logits,
                       m->vocab, ws, wsb, st);
}

int forward_prefill(const pe_model_desc* m, const pe_pass_args* a, const PrefillLayout& Lp, hipStream_t st) {
  const int M = a->M;
  char* ws = (char*)a->workspace;
  const int es = 2;
  const int H = m->hidden, nh = m->num_heads, nkv = m->num_kv_heads, hd = m->head_dim;
  const int qd = nh * hd, ip = m->intermediate_padded, L = m->num_layers;
  const int nqkv = (nh + 2 * nkv) * hd;
  void* h = ws + Lp.h;
  void* xn = ws + Lp.xn;
  void* xn_t = ws + Lp.xn_t;
  void* q = ws + Lp.q;
  void* attn = ws + Lp.attn;
  void* attn_t = ws + Lp.attn_t;
  void* act_t = ws + Lp.act_t;
  float* y = (float*)(ws + Lp.y);
  const float scale = (float)(1.0 / std::sqrt((double)hd));
  const int64_t layer_stride = (int64_t)nkv * a->cache_capacity * hd * es;
  const int64_t fused_ld = (int64_t)a->num_features * H;
  const bool nf4 = m->weight_format == PE_WFMT_NF4;
  int rc;
#define PE_TRY(expr)            \
  do {                          \
    rc = (expr);                \
    if (rc != PE_OK) return rc; \
  } while (0)
  auto slot_of = [&](int layer) -> int {
    if (!a->fused) return -1;
    for (int f = 0; f < a->num_features; ++f)
      if (a->feature_layers[f] == layer) return f;
    return -1;
  };
  auto slot_ptr = [&](int f) -> void* { return f < 0 ? nullptr : (char*)a->fused + (int64_t)f * H * es; };
  auto copy_repeats = [&](int layer, int first) -> int {
    if (first < 0) return PE_OK;
    for (int f = first + 1; f < a->num_features; ++f) {
      if (a->feature_layers[f] != layer) continue;
      int r = pe_copy_rows(slot_ptr(first), fused_ld * es, M, (int64_t)H * es, slot_ptr(f), fused_ld * es, st);
      if (r != PE_OK) return r;
    }
    return PE_OK;
  };
  // y[ys][M][N] (fp32 split partials) = x (A-tiled) . W^T over all rows
  int ys = 1;
  auto linear = [&](const void* xt, int K, const void* w, const void* ab, int N) -> int {
    ys = 1;
    if (nf4) return pe_internal_nf4_prefill(xt, M, K, w, ab, N, y, nullptr, 0, st);
    const void* wt = w;
    if (m->weight_format == PE_WFMT_NF4_F32ABS) {
      int r = pe_nf4_dequant_f32abs((const uint8_t*)w, (const float*)ab, N, K, (uint16_t*)(ws + Lp.wdeq), st);
      if (r != PE_OK) return r;
      r = pe_dense_repack(ws + Lp.wdeq, N, K, m->dtype, ws + Lp.wtile, st);
      if (r != PE_OK) return r;
      wt = ws + Lp.wtile;
    }
    return pe_internal_dense_bigm(xt, M, K, wt, m->dtype, N, y, N, st, true, &ys);
  };

  {
    const int f0 = slot_of(0);
    PE_TRY(pe_internal_embed_rmsnorm(a->input_ids, M, m->embed, embed_rows(m), h, H, m->attn_norm[0], m->rms_eps,
                                     m->norm_mode, m->dtype, nullptr, xn_t, slot_ptr(f0), fused_ld, nullptr, 0,
                                     a->status, st));
    PE_TRY(copy_repeats(0, f0));
  }
  const bool eager = m->attn_mode == PE_ATTN_EAGER;  // writes row-major output, packed afterwards
  for (int l = 0; l < L; ++l) {
    void* kc = (char*)a->k_cache + l * layer_stride;
    void* vc = (char*)a->v_cache + l * layer_stride;
    PE_TRY(linear(xn_t, H, m->w_qkv[l], m->a_qkv ? m->a_qkv[l] : nullptr, nqkv));
    PE_TRY(pe_internal_rope_kv_partials(y, ys, M, nh, nkv, hd, m->b_qkv ? m->b_qkv[l] : nullptr, a->positions,
                                        m->rope_cos_sin, m->max_positions, q, kc, vc, a->cache_capacity,
                                        a->prefix_len, a->status, m->dtype, st));
    PE_TRY(pe_internal_tree_attention(q, kc, vc, a->cache_capacity, nh, nkv, hd, M, a->prefix_len, PE_MASK_CAUSAL,
                                      nullptr, 0, scale, m->dtype, eager ? attn : attn_t, qd, eager ? 0 : qd / 128,
                                      ws + Lp.attn_ws, Lp.attn_ws_bytes, (int*)(ws + Lp.gemm) + kPassAttnCounterInt,
                                      st, m->attn_mode));
    if (eager) PE_TRY(pe_internal_to_xtile(attn, qd, M, qd, attn_t, st));
    PE_TRY(linear(attn_t, qd, m->w_o[l], m->a_o ? m->a_o[l] : nullptr, H));
    PE_TRY(pe_internal_residual_rmsnorm(y, ys, M, h, H, m->mlp_norm[l], m->rms_eps, m->norm_mode, m->dtype, nullptr, xn_t,
                                        nullptr, 0, nullptr, 0, st));
    if (nf4) {
      PE_TRY(pe_internal_nf4_prefill(xn_t, M, H, m->w_gu[l], m->a_gu[l], 2 * ip, nullptr, act_t, ip / 128, st));
    } else {
      PE_TRY(linear(xn_t, H, m->w_gu[l], m->a_gu ? m->a_gu[l] : nullptr, 2 * ip));
      PE_TRY(pe_internal_swiglu_partials(y, ys, M, 2 * ip, act_t, ip, ip / 128, m->dtype, st));
    }
    PE_TRY(linear(act_t, ip, m->w_down[l], m->a_down ? m->a_down[l] : nullptr, H));
    const bool last = l + 1 == L;
    const int fh = last ? -1 : slot_of(l + 1);
    const int fx = last ? slot_of(L) : -1;
    const void* next_norm = last ? m->final_norm : m->attn_norm[l + 1];
    const int next_mode = last ? PE_NORM_HF : m->norm_mode;
    PE_TRY(pe_internal_residual_rmsnorm(y, ys, M, h, H, next_norm, m->rms_eps, next_mode, m->dtype, nullptr, xn_t,
                                        slot_ptr(fh), fused_ld, slot_ptr(fx), fused_ld, st));
    PE_TRY(copy_repeats(last ? L : l + 1, last ? fx : fh));
  }
  // every lm_head weight read once per 256-row block
  if (a->logits) PE_TRY(pe_internal_dense_bigm(xn_t, M, H, m->lm_head, m->dtype, m->vocab, a->logits, m->vocab, st));
#undef PE_TRY
  return PE_OK;
}

int64_t batch_layout_total(const pe_model_desc* m, int M, int max_rows, int64_t max_kv_len, int batch);

extern "C" int64_t pe_forward_workspace_bytes(const pe_model_desc* m, int M, int64_t kv_len) {
  if (!m || M <= 0 || kv_len <= 0) return 0;
  // a causal pass of more than one chunk may take the prefill path
  const int64_t pre = prefill_path(m, M, PE_MASK_CAUSAL) ? make_prefill_layout(m, M, kv_len).total : 0;
  int64_t fused;
  if (m->qkv_layout == PE_QKV_ROPE_PAIRED && M > kFusedChunk) {
    // 64-row chunks and a shorter last one (its GEMM plans can need more partials)
    fused = make_layout(m, kFusedChunk, kv_len).total;
    if (M % kFusedChunk) {
      const int64_t last = make_layout(m, M % kFusedChunk, kv_len).total;
      if (last > fused) fused = last;
    }
  } else {
    fused = make_layout(m, M, kv_len).total;
  }
  if (wide_tree_path(m, M)) {
    const int64_t wide = batch_layout_total(m, M, M, kv_len, 1) + kOneSeqBytes;
    if (wide > fused) fused = wide;
  }
  return pre > fused ? pre : fused;
}

// The 16-bit pass: per layer
//   q/k/v GEMM with bias + RoPE + in-place K/V append in its epilogue
//   -> tree attention (split-KV) -> combine
//   -> o GEMM (fp32 split partials) -> residual add + post-attention RMSNorm
//   -> gate/up GEMM with SwiGLU epilogue
//   -> down GEMM (fp32 split partials) -> residual add + next RMSNorm
// The RMSNorm after the down projection is the next layer's input norm, or the
// final norm after the last layer; hidden-state captures ride on it.
int forward_fused(const pe_model_desc* m, const pe_pass_args* a, const Layout& Lo, hipStream_t st) {
  const int M = a->M;
  char* ws = (char*)a->workspace;
  void* gws = ws + Lo.gemm;
  const int64_t gwsb = Lo.gemm_bytes;
  const int es = esize(m->dtype);
  const int H = m->hidden, nh = m->num_heads, nkv = m->num_kv_heads, hd = m->head_dim;
  const int qd = nh * hd, ip = m->intermediate_padded, L = m->num_layers, wf = m->weight_format;
  void* h = ws + Lo.h;
  void* xn = ws + Lo.xn;
  void* q = ws + Lo.q;
  void* attn = ws + Lo.attn;
  void* act = ws + Lo.act;
  void* aws = ws + Lo.attn_ws;
  // A-tiled GEMM inputs: x_* is what the GEMMs read, *_units the tiled output widths
  const bool tiled = tiled_path(m, M);
  void* xn_t = tiled ? ws + Lo.xn_t : nullptr;
  void* x_norm = tiled ? xn_t : xn;
  void* xn_rm = tiled ? nullptr : xn;  // row-major norm rows: none when tiled (the lm_head reads A-tiled rows too)
  void* x_attn = tiled ? ws + Lo.attn_t : attn;
  void* x_act = tiled ? ws + Lo.act_t : act;
  const int attn_units = tiled ? qd / 128 : 0, act_units = tiled ? ip / 128 : 0;
  const float scale = (float)(1.0 / std::sqrt((double)hd));
  const int64_t layer_stride = (int64_t)nkv * a->cache_capacity * hd * es;
  const int64_t fused_ld = (int64_t)a->num_features * H;  // elements
  // A batch of one: the sequence's prefix P is read on the device
  // (seq_prefix[0]); a->prefix_len bounds it and sizes the launches. K/V land
  // at per-row slots P + row, and attention takes its keys and splits from the
  // device P (for P == prefix_len the same key splits as a host-P pass).
  const bool devp = a->batch == 1;
  int64_t* kvoff = devp ? (int64_t*)(ws + Lo.kvoff) : nullptr;
  int rc;
#define PE_TRY(expr)            \
  do {                          \
    rc = (expr);                \
    if (rc != PE_OK) return rc; \
  } while (0)
  if (devp)
    PE_TRY(pe_internal_kv_offsets(a->seq_row0, a->seq_prefix, 1, M, a->cache_seq_stride, a->cache_capacity, hd,
                                  a->prefix_len, M, kvoff, a->status, st));
  // first fused-feature slot capturing `layer` (or -1), and extra copies for repeated layers
  auto slot_of = [&](int layer) -> int {
    if (!a->fused) return -1;
    for (int f = 0; f < a->num_features; ++f)
      if (a->feature_layers[f] == layer) return f;
    return -1;
  };
  auto slot_ptr = [&](int f) -> void* { return f < 0 ? nullptr : (char*)a->fused + (int64_t)f * H * es; };
  auto copy_repeats = [&](int layer, int first) -> int {
    if (first < 0) return PE_OK;
    for (int f = first + 1; f < a->num_features; ++f) {
      if (a->feature_layers[f] != layer) continue;
      int r = pe_copy_rows(slot_ptr(first), fused_ld * es, M, (int64_t)H * es, slot_ptr(f), fused_ld * es, st);
      if (r != PE_OK) return r;
    }
    return PE_OK;
  };

  {
    const int f0 = slot_of(0);
    PE_TRY(pe_internal_embed_rmsnorm(a->input_ids, M, m->embed, embed_rows(m), h, H, m->attn_norm[0], m->rms_eps,
                                     m->norm_mode, m->dtype, xn_rm, xn_t, slot_ptr(f0), fused_ld, nullptr, 0, a->status,
                                     st));
    PE_TRY(copy_repeats(0, f0));
  }
  // q/k/v and gate/up run with their RoPE + KV append / SwiGLU epilogues in
  // the GEMM (unsplit in the tiled NF4 pass); o and down write split partials
  // with plain stores that the residual + RMSNorm kernel sums, so no o or down
  // workgroup waits on another of its own launch (NF4 and dense alike: for
  // the dense 14B shapes the partials and one round of workgroups made the
  // pass 7.9% faster than the in-launch exchange).
  float* part = (float*)(ws + Lo.part);
  int S = 0;
  for (int l = 0; l < L; ++l) {
    void* kc = (char*)a->k_cache + l * layer_stride;
    void* vc = (char*)a->v_cache + l * layer_stride;
    const void* a_qkv = m->a_qkv ? m->a_qkv[l] : nullptr;
    const void* b_qkv = m->b_qkv ? m->b_qkv[l] : nullptr;
    PE_TRY(pe_internal_gemm_rope_kv(wf, m->dtype, x_norm, H, M, H, m->w_qkv[l], a_qkv, nh, nkv, hd, b_qkv,
                                    a->positions, m->rope_cos_sin, m->max_positions, q, kc, vc, a->cache_capacity,
                                    a->prefix_len, a->status, gws, gwsb, tiled, st, kvoff));
    if (devp)
      PE_TRY(pe_internal_tree_attention_batch(q, kc, vc, a->cache_capacity, a->cache_seq_stride, nh, nkv, M,
                                              a->prefix_len, 1, a->seq_row0, a->seq_prefix, a->tree_bits,
                                              a->bits_words, scale, m->dtype, x_attn, qd, attn_units, aws,
                                              Lo.attn_ws_bytes, (int*)gws + kPassAttnCounterInt, st, 1));
    else
      PE_TRY(pe_internal_tree_attention(q, kc, vc, a->cache_capacity, nh, nkv, hd, M, a->prefix_len, a->mask_mode,
                                        a->tree_bits, a->bits_words, scale, m->dtype, x_attn, qd, attn_units, aws,
                                        Lo.attn_ws_bytes, (int*)gws + kPassAttnCounterInt, st, m->attn_mode));
    const void* a_o = m->a_o ? m->a_o[l] : nullptr;
    PE_TRY(pe_internal_linear_partials(wf, m->dtype, x_attn, qd, tiled, M, qd, m->w_o[l], a_o, H, part,
                                       Lo.part_bytes, &S, st));
    PE_TRY(pe_internal_residual_rmsnorm(part, S, M, h, H, m->mlp_norm[l], m->rms_eps, m->norm_mode, m->dtype, xn_rm, xn_t,
                                        nullptr, 0, nullptr, 0, st));
    const void* a_gu = m->a_gu ? m->a_gu[l] : nullptr;
    const void* a_down = m->a_down ? m->a_down[l] : nullptr;
    const bool last = l + 1 == L;
    const int fh = last ? -1 : slot_of(l + 1);
    const int fx = last ? slot_of(L) : -1;
    const void* next_norm = last ? m->final_norm : m->attn_norm[l + 1];
    const int next_mode = last ? PE_NORM_HF : m->norm_mode;
    PE_TRY(pe_internal_linear(wf, m->dtype, x_norm, H, tiled, M, H, m->w_gu[l], a_gu, 2 * ip, PE_EPI_SWIGLU, nullptr,
                              nullptr, 0, x_act, ip, act_units, gws, gwsb, st));
    PE_TRY(pe_internal_linear_partials(wf, m->dtype, x_act, ip, tiled, M, ip, m->w_down[l], a_down, H, part,
                                       Lo.part_bytes, &S, st));
    PE_TRY(pe_internal_residual_rmsnorm(part, S, M, h, H, next_norm, m->rms_eps, next_mode, m->dtype, xn_rm, xn_t,
                                        slot_ptr(fh), fused_ld, slot_ptr(fx), fused_ld, st));
    PE_TRY(copy_repeats(last ? L : l + 1, last ? fx : fh));
  }
  if (a->logits) PE_TRY(lm_head(m, a, tiled ? xn_t : xn, tiled, M, gws, gwsb, st));
#undef PE_TRY
  return PE_OK;
}

// ---------------------------------------------------------------------------
// Batched verification: `batch` sequences, each a tree over its own cached
// prefix, all M rows through every linear at once (each weight is streamed
// once per 64-row chunk launch for the whole batch, not once per sequence);
// attention runs over every sequence's own keys in one launch, and the q/k/v
// epilogue appends each row's K/V at its own sequence's rows. Activations are
// row-major (the A-tiled handoff is for single 64-row passes).
// ---------------------------------------------------------------------------
struct BatchLayout {
  int64_t gemm, gemm_bytes, h, xn, q, attn, act, kvoff, attn_ws, attn_ws_bytes;
  bool big;                                   // the many-row NF4 path (A-tiled activations, split partials)
  int64_t xn_t, attn_t, act_t, part, part_bytes;
  int64_t total;
};

// The batched NF4 pass over 65..256 rows dequantises each weight once for all
// rows (pe_internal_nf4_bigm_partials) and hands A-tiled activations between
// the kernels; other batches run each linear in 64-row launches on row-major X.
bool batch_big_path(const pe_model_desc* m, int M) {
  const int H = m->hidden, qd = m->num_heads * m->head_dim, ip = m->intermediate_padded;
  const int nqkv = qd + 2 * m->num_kv_heads * m->head_dim;
  return m->weight_format == PE_WFMT_NF4 && M > kFusedChunk && M <= 256 && H % 128 == 0 && qd % 128 == 0 &&
         ip % 128 == 0 && nqkv % 128 == 0;
}

BatchLayout make_batch_layout(const pe_model_desc* m, int M, int max_rows, int64_t max_kv_len, int batch) {
  BatchLayout L;
  const int es = esize(m->dtype);
  const int H = m->hidden, qd = m->num_heads * m->head_dim, ip = m->intermediate_padded;
  const int nqkv = qd + 2 * m->num_kv_heads * m->head_dim;
  int64_t g = kCounterBytes;
  const int64_t cand[5] = {pe_internal_gemm_rope_kv_bytes(M, nqkv, H, m->weight_format),
                           gemm_ws(m, M, H, qd, PE_EPI_RESIDUAL), gemm_ws(m, M, 2 * ip, H, PE_EPI_SWIGLU),
                           gemm_ws(m, M, H, ip, PE_EPI_RESIDUAL),
                           pe_gemm_workspace_bytes(M, m->vocab, H, PE_WFMT_DENSE, m->dtype, PE_EPI_STORE)};
  for (int i = 0; i < 5; ++i)
    if (cand[i] > g) g = cand[i];
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t o = off;
    off += align_up(bytes);
    return o;
  };
  L.gemm_bytes = align_up(g);
  L.gemm = take(L.gemm_bytes);
  L.h = take((int64_t)M * H * es);
  L.xn = take((int64_t)M * H * es);
  L.q = take((int64_t)M * qd * es);
  L.attn = take((int64_t)M * qd * es);
  L.act = take((int64_t)M * ip * es);
  L.kvoff = take((int64_t)M * 8);
  L.attn_ws_bytes =
      align_up(pe_internal_attention_batch_bytes(max_rows, m->num_heads, m->num_kv_heads, max_kv_len, batch));
  L.attn_ws = take(L.attn_ws_bytes);
  L.big = batch_big_path(m, M);
  L.xn_t = L.attn_t = L.act_t = L.part = L.part_bytes = 0;
  if (L.big) {
    L.xn_t = take(xtile_bytes(M, H));
    L.attn_t = take(xtile_bytes(M, qd));
    L.act_t = take(xtile_bytes(M, ip));
    const int64_t pb[4] = {pe_internal_nf4_bigm_partials_bytes(M, nqkv, H), pe_internal_nf4_bigm_partials_bytes(M, H, qd),
                           pe_internal_nf4_bigm_partials_bytes(M, 2 * ip, H), pe_internal_nf4_bigm_partials_bytes(M, H, ip)};
    for (int i = 0; i < 4; ++i)
      if (pb[i] > L.part_bytes) L.part_bytes = pb[i];
    L.part_bytes = align_up(L.part_bytes);
    L.part = take(L.part_bytes);
  }
  L.total = off;
  return L;
}

int64_t batch_layout_total(const pe_model_desc* m, int M, int max_rows, int64_t max_kv_len, int batch) {
  return make_batch_layout(m, M, max_rows, max_kv_len, batch).total;
}

int forward_batched(const pe_model_desc* m, const pe_pass_args* a, const BatchLayout& Lb, hipStream_t st) {
  const int M = a->M;
  char* ws = (char*)a->workspace;
  void* gws = ws + Lb.gemm;
  const int64_t gwsb = Lb.gemm_bytes;
  const int es = esize(m->dtype);
  const int H = m->hidden, nh = m->num_heads, nkv = m->num_kv_heads, hd = m->head_dim;
  const int qd = nh * hd, ip = m->intermediate_padded, L = m->num_layers, wf = m->weight_format;
  char* h = ws + Lb.h;
  char* xn = ws + Lb.xn;
  char* q = ws + Lb.q;
  char* attn = ws + Lb.attn;
  char* act = ws + Lb.act;
  int64_t* kvoff = (int64_t*)(ws + Lb.kvoff);
  const float scale = (float)(1.0 / std::sqrt((double)hd));
  const int64_t layer_stride = (int64_t)nkv * a->cache_capacity * hd * es;
  const int64_t fused_ld = (int64_t)a->num_features * H;
  int rc;
#define PE_TRY(expr)            \
  do {                          \
    rc = (expr);                \
    if (rc != PE_OK) return rc; \
  } while (0)
  auto slot_of = [&](int layer) -> int {
    if (!a->fused) return -1;
    for (int f = 0; f < a->num_features; ++f)
      if (a->feature_layers[f] == layer) return f;
    return -1;
  };
  auto slot_ptr = [&](int f) -> void* { return f < 0 ? nullptr : (char*)a->fused + (int64_t)f * H * es; };
  auto copy_repeats = [&](int layer, int first) -> int {
    if (first < 0) return PE_OK;
    for (int f = first + 1; f < a->num_features; ++f) {
      if (a->feature_layers[f] != layer) continue;
      int r = pe_copy_rows(slot_ptr(first), fused_ld * es, M, (int64_t)H * es, slot_ptr(f), fused_ld * es, st);
      if (r != PE_OK) return r;
    }
    return PE_OK;
  };
  PE_TRY(pe_internal_kv_offsets(a->seq_row0, a->seq_prefix, a->batch, M, a->cache_seq_stride, a->cache_capacity, hd,
                                a->prefix_len, a->max_seq_rows, kvoff, a->status, st));
  char* xn_t = Lb.big ? ws + Lb.xn_t : nullptr;
  {
    const int f0 = slot_of(0);
    PE_TRY(pe_internal_embed_rmsnorm(a->input_ids, M, m->embed, embed_rows(m), h, H, m->attn_norm[0], m->rms_eps,
                                     m->norm_mode, m->dtype, xn, xn_t, slot_ptr(f0), fused_ld, nullptr, 0,
                                     a->status, st));
    PE_TRY(copy_repeats(0, f0));
  }
  if (Lb.big) {
    // every linear: one launch over all M rows (split partials), consumed by
    // the RoPE + K/V append, SwiGLU and residual + RMSNorm kernels; an
    // unsplit gate/up launch stores the SwiGLU activation itself
    char* attn_t = ws + Lb.attn_t;
    char* act_t = ws + Lb.act_t;
    float* part = (float*)(ws + Lb.part);
    const int nqkv = (nh + 2 * nkv) * hd;
    const bool big_head = m->vocab % 128 == 0 && (m->dtype == PE_DTYPE_BF16 || m->dtype == PE_DTYPE_F16);
    int S = 0;
    for (int l = 0; l < L; ++l) {
      char* kc = (char*)a->k_cache + l * layer_stride;
      char* vc = (char*)a->v_cache + l * layer_stride;
      PE_TRY(pe_internal_nf4_bigm_partials(xn_t, M, H, m->w_qkv[l], m->a_qkv[l], nqkv, part, Lb.part_bytes, &S, st));
      PE_TRY(pe_internal_rope_kv_partials(part, S, M, nh, nkv, hd, m->b_qkv ? m->b_qkv[l] : nullptr, a->positions,
                                          m->rope_cos_sin, m->max_positions, q, kc, vc, a->cache_capacity, 0,
                                          a->status, m->dtype, st, kvoff));
      PE_TRY(pe_internal_tree_attention_batch(q, kc, vc, a->cache_capacity, a->cache_seq_stride, nh, nkv,
                                              a->max_seq_rows, a->prefix_len, a->batch, a->seq_row0, a->seq_prefix,
                                              a->tree_bits, a->bits_words, scale, m->dtype, attn_t, qd, qd / 128,
                                              ws + Lb.attn_ws, Lb.attn_ws_bytes, (int*)gws + kPassAttnCounterInt, st));
      PE_TRY(pe_internal_nf4_bigm_partials(attn_t, M, qd, m->w_o[l], m->a_o[l], H, part, Lb.part_bytes, &S, st));
      PE_TRY(pe_internal_residual_rmsnorm(part, S, M, h, H, m->mlp_norm[l], m->rms_eps, m->norm_mode, m->dtype, xn,
                                          xn_t, nullptr, 0, nullptr, 0, st));
      PE_TRY(pe_internal_nf4_bigm_swiglu(xn_t, M, H, m->w_gu[l], m->a_gu[l], 2 * ip, act_t, ip / 128, m->dtype, part,
                                         Lb.part_bytes, &S, st));
      if (S > 0) PE_TRY(pe_internal_swiglu_partials(part, S, M, 2 * ip, act_t, ip, ip / 128, m->dtype, st));
      PE_TRY(pe_internal_nf4_bigm_partials(act_t, M, ip, m->w_down[l], m->a_down[l], H, part, Lb.part_bytes, &S, st));
      const bool last = l + 1 == L;
      const int fh = last ? -1 : slot_of(l + 1);
      const int fx = last ? slot_of(L) : -1;
      const void* next_norm = last ? m->final_norm : m->attn_norm[l + 1];
      const int next_mode = last ? PE_NORM_HF : m->norm_mode;
      PE_TRY(pe_internal_residual_rmsnorm(part, S, M, h, H, next_norm, m->rms_eps, next_mode, m->dtype, xn,
                                          last && !big_head ? nullptr : xn_t, slot_ptr(fh), fused_ld, slot_ptr(fx),
                                          fused_ld, st));
      PE_TRY(copy_repeats(last ? L : l + 1, last ? fx : fh));
    }
    if (a->logits && big_head)  // every lm_head weight read once for all rows
      PE_TRY(pe_internal_dense_bigm(xn_t, M, H, m->lm_head, m->dtype, m->vocab, a->logits, m->vocab, st));
    else if (a->logits)
      PE_TRY(pe_dense_gemm(xn, H, M, H, m->lm_head, m->dtype, m->vocab, PE_EPI_STORE, nullptr, nullptr, 0, a->logits,
                           m->vocab, gws, gwsb, st));
    return PE_OK;
  }
  for (int l = 0; l < L; ++l) {
    char* kc = (char*)a->k_cache + l * layer_stride;
    char* vc = (char*)a->v_cache + l * layer_stride;
    const void* a_qkv = m->a_qkv ? m->a_qkv[l] : nullptr;
    const void* b_qkv = m->b_qkv ? m->b_qkv[l] : nullptr;
    for (int c0 = 0; c0 < M; c0 += kFusedChunk) {
      const int mc = M - c0 < kFusedChunk ? M - c0 : kFusedChunk;
      PE_TRY(pe_internal_gemm_rope_kv(wf, m->dtype, xn + (int64_t)c0 * H * es, H, mc, H, m->w_qkv[l], a_qkv, nh, nkv,
                                      hd, b_qkv, a->positions + c0, m->rope_cos_sin, m->max_positions,
                                      q + (int64_t)c0 * qd * es, kc, vc, a->cache_capacity, 0, a->status, gws, gwsb,
                                      false, st, kvoff + c0));
    }
    PE_TRY(pe_internal_tree_attention_batch(q, kc, vc, a->cache_capacity, a->cache_seq_stride, nh, nkv,
                                            a->max_seq_rows, a->prefix_len, a->batch, a->seq_row0, a->seq_prefix,
                                            a->tree_bits, a->bits_words, scale, m->dtype, attn, qd, 0, ws + Lb.attn_ws,
                                            Lb.attn_ws_bytes, (int*)gws + kPassAttnCounterInt, st));
    const void* a_o = m->a_o ? m->a_o[l] : nullptr;
    PE_TRY(pe_internal_linear(wf, m->dtype, attn, qd, false, M, qd, m->w_o[l], a_o, H, PE_EPI_RESIDUAL, nullptr, h, H,
                              h, H, 0, gws, gwsb, st));
    PE_TRY(pe_internal_residual_rmsnorm(nullptr, 0, M, h, H, m->mlp_norm[l], m->rms_eps, m->norm_mode, m->dtype, xn,
                                        nullptr, nullptr, 0, nullptr, 0, st));
    const void* a_gu = m->a_gu ? m->a_gu[l] : nullptr;
    const void* a_down = m->a_down ? m->a_down[l] : nullptr;
    PE_TRY(pe_internal_linear(wf, m->dtype, xn, H, false, M, H, m->w_gu[l], a_gu, 2 * ip, PE_EPI_SWIGLU, nullptr,
                              nullptr, 0, act, ip, 0, gws, gwsb, st));
    PE_TRY(pe_internal_linear(wf, m->dtype, act, ip, false, M, ip, m->w_down[l], a_down, H, PE_EPI_RESIDUAL, nullptr,
                              h, H, h, H, 0, gws, gwsb, st));
    const bool last = l + 1 == L;
    const int fh = last ? -1 : slot_of(l + 1);
    const int fx = last ? slot_of(L) : -1;
    const void* next_norm = last ? m->final_norm : m->attn_norm[l + 1];
    const int next_mode = last ? PE_NORM_HF : m->norm_mode;
    PE_TRY(pe_internal_residual_rmsnorm(nullptr, 0, M, h, H, next_norm, m->rms_eps, next_mode, m->dtype, xn, nullptr,
                                        slot_ptr(fh), fused_ld, slot_ptr(fx), fused_ld, st));
    PE_TRY(copy_repeats(last ? L : l + 1, last ? fx : fh));
  }
  if (a->logits)
    PE_TRY(pe_dense_gemm(xn, H, M, H, m->lm_head, m->dtype, m->vocab, PE_EPI_STORE, nullptr, nullptr, 0, a->logits,
                         m->vocab, gws, gwsb, st));
#undef PE_TRY
  return PE_OK;
}

extern "C" int64_t pe_forward_batch_workspace_bytes(const pe_model_desc* m, int M, int max_seq_rows,
                                                    int64_t max_kv_len, int batch) {
  if (!m || M <= 0 || max_seq_rows <= 0 || max_kv_len <= 0 || batch <= 0) return 0;
  const int64_t b = make_batch_layout(m, M, max_seq_rows, max_kv_len, batch).total;
  if (batch == 1 && fused_path(m, M)) {  // the single-sequence pass with a device prefix
    const int64_t f = make_layout(m, M, max_kv_len).total;
    return f > b ? f : b;
  }
  return b;
}

extern "C" int pe_forward(const pe_model_desc* m, const pe_pass_args* a, void* stream) {
  if (!m || !a) return PE_ERR_ARG;
  const int M = a->M;
  if (M <= 0 || !a->input_ids || !a->positions || !a->k_cache || !a->v_cache || !a->workspace) return PE_ERR_ARG;
  // a batched pass appends at most max_seq_rows rows to any one cache (each
  // row's slot is checked again on the device against its own prefix)
  const int64_t appended = a->batch > 0 ? a->max_seq_rows : M;
  if (a->prefix_len < 0 || a->prefix_len + appended > a->cache_capacity) return PE_ERR_CAPACITY;
  if (a->num_features < 0 || a->num_features > 4) return PE_ERR_ARG;
  if (a->mask_mode == PE_MASK_TREE && !a->tree_bits) return PE_ERR_ARG;
  if (m->intermediate_padded % 32 || m->intermediate_padded < m->intermediate) return PE_ERR_ARG;
  if (m->norm_mode != PE_NORM_HF && m->norm_mode != PE_NORM_FP32_WEIGHT) return PE_ERR_ARG;
  if (m->attn_mode != PE_ATTN_SDPA && m->attn_mode != PE_ATTN_EAGER) return PE_ERR_ARG;
  // eager attention writes row-major output: not the A-tiled NF4 pass (dense
  // models with eager attention run the fused pass on row-major activations)
  if (m->attn_mode == PE_ATTN_EAGER && pe_wfmt_nf4(m->weight_format)) return PE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (a->batch < 0) return PE_ERR_ARG;
  // argmax keys: single-sequence 16-bit passes of at most one chunk that write
  // logits (a batch of one included)
  if (a->node_keys && (a->batch > 1 || !a->logits || m->dtype == PE_DTYPE_F32 || M > kFusedChunk))
    return PE_ERR_ARG;
  if (a->batch > 0) {
    if (a->mask_mode != PE_MASK_TREE || !a->tree_bits || !a->seq_row0 || !a->seq_prefix) return PE_ERR_ARG;
    if (m->dtype == PE_DTYPE_F32 || m->head_dim != 128 || m->qkv_layout != PE_QKV_ROPE_PAIRED ||
        m->attn_mode != PE_ATTN_SDPA)
      return PE_ERR_ARG;
    if (a->bits_words <= 0 || a->bits_words > PE_TREE_MAX_WORDS || a->max_seq_rows <= 0 ||
        a->max_seq_rows > 64 * a->bits_words || a->max_seq_rows > M)
      return PE_ERR_TREE;
    const int64_t per_seq = (int64_t)m->num_layers * m->num_kv_heads * a->cache_capacity * m->head_dim;
    if (a->cache_seq_stride < per_seq) return PE_ERR_ARG;
    if (a->batch == 1 && fused_path(m, M)) {
      // one sequence of at most one chunk: the single-sequence pass with its
      // prefix read on the device
      if (a->max_seq_rows != M) return PE_ERR_ARG;
      const Layout Lo = make_layout(m, M, a->prefix_len + M);
      if (a->workspace_bytes < Lo.total) return PE_ERR_WORKSPACE;
      return forward_fused(m, a, Lo, st);
    }
    if (a->node_keys) return PE_ERR_ARG;
    const BatchLayout Lb = make_batch_layout(m, M, a->max_seq_rows, a->prefix_len + a->max_seq_rows, a->batch);
    if (a->workspace_bytes < Lb.total) return PE_ERR_WORKSPACE;
    return forward_batched(m, a, Lb, st);
  }
  const int64_t kv_len = a->prefix_len + M;
  if (a->mask_mode == PE_MASK_TREE && wide_tree_path(m, M)) {
    if (a->bits_words <= 0 || a->bits_words > PE_TREE_MAX_WORDS || M > 64 * a->bits_words) return PE_ERR_TREE;
    const BatchLayout Lb = make_batch_layout(m, M, M, kv_len, 1);
    if (a->workspace_bytes < Lb.total + kOneSeqBytes) return PE_ERR_WORKSPACE;
    int32_t* row0 = (int32_t*)((char*)a->workspace + Lb.total);
    int64_t* prefix = (int64_t*)((char*)row0 + 16);
    pe_pass_args b = *a;
    b.batch = 1;
    b.max_seq_rows = M;
    b.seq_row0 = row0;
    b.seq_prefix = prefix;
    b.cache_seq_stride = (int64_t)m->num_layers * m->num_kv_heads * a->cache_capacity * m->head_dim;
    const int rc = pe_internal_one_sequence(row0, prefix, M, a->prefix_len, st);
    if (rc != PE_OK) return rc;
    return forward_batched(m, &b, Lb, st);
  }
  if (prefill_path(m, M, a->mask_mode)) {
    const PrefillLayout Lp = make_prefill_layout(m, M, kv_len);
    if (a->workspace_bytes < Lp.total) return PE_ERR_WORKSPACE;
    return forward_prefill(m, a, Lp, st);
  }
  const Layout Lo = make_layout(m, M, kv_len);
  if (m->qkv_layout == PE_QKV_ROPE_PAIRED) {
    // 16-bit hd-128 models only; a tree pass must fit one chunk (its nodes see
    // ancestors only, so it cannot be split into causal continuations).
    if (m->dtype == PE_DTYPE_F32 || m->head_dim != 128) return PE_ERR_ARG;
    if (a->mask_mode == PE_MASK_TREE && M > kFusedChunk) return PE_ERR_TREE;
    const int64_t vocab_bytes = (int64_t)m->vocab * esize(m->dtype);
    const int64_t fused_bytes = (int64_t)a->num_features * m->hidden * esize(m->dtype);
    for (int c0 = 0; c0 < M; c0 += kFusedChunk) {
      pe_pass_args b = *a;
      b.M = (M - c0 < kFusedChunk) ? M - c0 : kFusedChunk;
      b.input_ids = a->input_ids + c0;
      b.positions = a->positions + c0;
      b.prefix_len = a->prefix_len + c0;
      b.logits = a->logits ? (char*)a->logits + c0 * vocab_bytes : nullptr;
      b.fused = a->fused ? (char*)a->fused + c0 * fused_bytes : nullptr;
      const Layout Lc = make_layout(m, b.M, b.prefix_len + b.M);
      if (a->workspace_bytes < Lc.total) return PE_ERR_WORKSPACE;
      const int rc = forward_fused(m, &b, Lc, st);
      if (rc != PE_OK) return rc;
    }
    return PE_OK;
  }
  if (a->workspace_bytes < Lo.total) return PE_ERR_WORKSPACE;
  if (m->qkv_layout != PE_QKV_PLAIN) return PE_ERR_ARG;
  char* ws = (char*)a->workspace;
  void* gws = ws + Lo.gemm;
  const int64_t gwsb = Lo.gemm_bytes;
  const int es = esize(m->dtype);
  const int H = m->hidden, nh = m->num_heads, nkv = m->num_kv_heads, hd = m->head_dim;
  const int qd = nh * hd, kvd = nkv * hd, nqkv = qd + 2 * kvd, ip = m->intermediate_padded;
  void* h = ws + Lo.h;
  void* xn = ws + Lo.xn;
  void* qkv = ws + Lo.qkv;
  void* q = ws + Lo.q;
  void* attn = ws + Lo.attn;
  void* act = ws + Lo.act;
  void* aws = ws + Lo.attn_ws;
  const float scale = (float)(1.0 / std::sqrt((double)hd));
  const int64_t layer_stride = (int64_t)nkv * a->cache_capacity * hd * es;
  const int64_t fused_ld = (int64_t)a->num_features * H * es;
  int rc;
#define PE_TRY(expr)            \
  do {                          \
    rc = (expr);                \
    if (rc != PE_OK) return rc; \
  } while (0)

  auto capture = [&](int slot_layer, const void* src) -> int {
    if (!a->fused) return PE_OK;
    for (int f = 0; f < a->num_features; ++f) {
      if (a->feature_layers[f] != slot_layer) continue;
      int r = pe_copy_rows(src, (int64_t)H * es, M, (int64_t)H * es, (char*)a->fused + (int64_t)f * H * es, fused_ld,
                           st);
      if (r != PE_OK) return r;
    }
    return PE_OK;
  };

  PE_TRY(pe_embed(a->input_ids, M, m->embed, embed_rows(m), H, m->dtype, h, H, a->status, st));
  PE_TRY(capture(0, h));
  for (int l = 0; l < m->num_layers; ++l) {
    void* kc = (char*)a->k_cache + l * layer_stride;
    void* vc = (char*)a->v_cache + l * layer_stride;
    PE_TRY(pe_rmsnorm_ex(h, H, M, H, m->attn_norm[l], m->rms_eps, m->dtype, m->norm_mode, xn, H, st));
    PE_TRY(linear(m, xn, H, M, H, m->w_qkv[l], m->a_qkv ? m->a_qkv[l] : nullptr, nqkv, PE_EPI_STORE,
                  m->b_qkv ? m->b_qkv[l] : nullptr, nullptr, 0, qkv, nqkv, gws, gwsb, st));
    PE_TRY(pe_rope_qkv(qkv, nqkv, M, nh, nkv, hd, a->positions, m->rope_cos_sin, m->max_positions, m->dtype, q, kc, vc,
                       a->cache_capacity, a->prefix_len, a->status, st));
    PE_TRY(pe_internal_tree_attention(q, kc, vc, a->cache_capacity, nh, nkv, hd, M, a->prefix_len, a->mask_mode,
                                      a->tree_bits, a->bits_words, scale, m->dtype, attn, qd, 0, aws,
                                      Lo.attn_ws_bytes, (int*)gws + kPassAttnCounterInt, st, m->attn_mode));
    PE_TRY(linear(m, attn, qd, M, qd, m->w_o[l], m->a_o ? m->a_o[l] : nullptr, H, PE_EPI_RESIDUAL, nullptr, h, H, h,
                  H, gws, gwsb, st));
    PE_TRY(pe_rmsnorm_ex(h, H, M, H, m->mlp_norm[l], m->rms_eps, m->dtype, m->norm_mode, xn, H, st));
    PE_TRY(linear(m, xn, H, M, H, m->w_gu[l], m->a_gu ? m->a_gu[l] : nullptr, 2 * ip, PE_EPI_SWIGLU, nullptr,
                  nullptr, 0, act, ip, gws, gwsb, st));
    PE_TRY(linear(m, act, ip, M, ip, m->w_down[l], m->a_down ? m->a_down[l] : nullptr, H, PE_EPI_RESIDUAL, nullptr,
                  h, H, h, H, gws, gwsb, st));
    if (l + 1 < m->num_layers) PE_TRY(capture(l + 1, h));
  }
  PE_TRY(pe_rmsnorm(h, H, M, H, m->final_norm, m->rms_eps, m->dtype, xn, H, st));
  PE_TRY(capture(m->num_layers, xn));
  if (a->logits) PE_TRY(lm_head(m, a, xn, false, M, gws, gwsb, st));
#undef PE_TRY
  return PE_OK;
}
