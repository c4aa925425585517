// Tree-masked GQA attention over the KV cache (split-KV flash decoding).
//
// Query rows are the T tree nodes (x G query heads per KV head); keys are the
// P cached prefix rows followed by the T node rows appended by pe_rope_qkv.
// A node attends to the whole prefix and to the node rows of its ancestor set,
// read from a per-node bitmask (bit u of bits[t] <=> node u is t or an
// ancestor of t), which is the (T, P+T) additive bias of the reference
// (src/pe/masks.py:127-147 + to_additive_bias :29-33) without materialising it.
//
// 16-bit path (hd = 128): one workgroup of 8 waves per (KV head, key split,
// 32-row tile), each wave a run of the split's 32-key blocks.
//   S^T = K Q^T with v_mfma_f32_32x32x16 (A = 32 keys x 16 dims of K straight
//   from the cache, B = Q^T from the tile staged in LDS), so every lane owns one query
//   row (column) and 16 of the 32 keys: the online-softmax max/sum of a row is
//   a 16-value in-lane reduction plus one exchange with lane^32.
//   O^T += V^T P^T (A = V^T from a wave-private LDS transpose of the 32-key V
//   block, B = P^T taken directly from the S^T accumulator registers rounded to
//   the compute dtype), so the per-row rescale is a per-lane scalar.
//   Each workgroup merges its waves and publishes its split's partial
//   (O, max, sum); the last workgroup of a (KV head, row tile) to arrive
//   combines the splits in split order and writes the output.
// Softmax is fp32; exp(s - m) is summed in fp32 and rounded to the compute
// dtype for the PV product, as torch's CPU flash attention does for reduced
// precision inputs. Scores are kept in base 2 (q.k * scale * log2 e), so every
// exponential is one v_exp_f32 (2^x) and the running maxima and split partials
// are in base 2 as well.
//
// The drafter's eager rounding (PE_ATTN_EAGER) at 16 bits: attn_eager_kernel,
// the same tiles in two passes over the keys.
// fp32 path: one block per (row, query head), scores in LDS, VALU arithmetic.

#include "pe_common.h"
#include "pe_internal.h"

#include <type_traits>

namespace {

constexpr float kMaskedScore = -3.0e38f;
constexpr float kInitMax = -2.0e38f;

__device__ __forceinline__ bool key_allowed(int64_t key, int64_t P, int t, int mask_mode, const uint64_t* nb) {
  if (mask_mode == PE_MASK_CAUSAL) return key <= P + t;
  if (key < P) return true;
  const int u = (int)(key - P);
  return (nb[u >> 6] >> (u & 63)) & 1ull;
}

// tree mask of one key, the word chosen by selects (no indexed read of the
// register array)
__device__ __forceinline__ bool tree_key_allowed(int64_t key, int64_t P, const uint64_t* nb) {
  if (key < P) return true;
  const int u = (int)(key - P);
  static_assert(PE_TREE_MAX_WORDS == 4, "one select per word");
  const uint64_t w = u < 64 ? nb[0] : u < 128 ? nb[1] : u < 192 ? nb[2] : nb[3];
  return (w >> (u & 63)) & 1ull;
}

// One workgroup = 8 waves = one (KV head, key split, 32-row tile); each wave
// takes a contiguous run of the split's 32-key blocks. Its first two blocks
// are loaded and processed together as one 64-key block (a run of one block
// processes half of it); a longer run continues one block per round, the
// next block's K (into the other of two K slots) and V (into the one V slot,
// once this block's V is in LDS) in flight during the round: with the O
// accumulators live, a wave holds three block slots, not four, and stays
// within 256 VGPRs without spilling. The row tile's Q, the row's ancestor
// bits and the first pair's K and V are the first loads of the wave, so at
// the 7B shape the whole KV stream is in flight at once. V
// goes to a wave-private LDS transpose before S = K Q^T is formed, the row
// tile's Q is staged once per workgroup in LDS (the B operand of S^T is read
// from there per k-step); the LDS footprint (about 89 KiB) allows one
// workgroup per CU. Loads are clamped to the wave's last valid key (those
// scores are masked and their probabilities are exactly zero), so no
// uninitialised cache row is read. At the end the waves' (m, l, O) are
// merged in LDS in wave order by all threads. With several splits the
// workgroup publishes that partial (rows past the tile's real rows are
// skipped) with agent-coherent 16-byte stores and counts itself on the
// pair's arrival counter; the last to arrive reads every split's partial
// (its own from registers) and combines them in split order: out = sum_s
// e^{m_s - M} O_s / sum_s e^{m_s - M} l_s, accumulated online (running max,
// rescaled sums). Nobody waits for anybody, and the result does not depend
// on the arrival order.
constexpr int kAttnWaves = 8;
constexpr int kQStride = 128 + 8;  // LDS row stride of the staged Q tile (elements)
constexpr int kVRow = 128 + 32;    // LDS row stride of a wave's V tile (elements): 320 B, rows 16 banks apart
constexpr int kCmbRow = 128 + 4;   // LDS row stride of the wave merge (floats; 16-byte aligned rows)
constexpr int kAttnMaxSplits = 16;
// a head's cache rows (256 bytes each at hd 128) are addressed with 32-bit
// byte offsets
constexpr int64_t kAttnMaxCap = int64_t(1) << 24;

// Batched attention (batch >= 1): grid.z runs over (sequence, row tile), the
// sequences in order of decreasing prefix length;
// sequence b's query rows are rows [seq_row0[b], seq_row0[b+1]) of q, bits
// and out, its keys the seq_prefix[b] cached rows plus its own node rows of
// the cache at kc / vc + b * seq_stride. Row tiles past a sequence's rows
// leave at once (all splits of such a tile alike, so no arrival is awaited).
// A sequence whose device prefix or row count exceeds the bounds the launch
// was sized for (max_prefix, max_rows) is skipped by every workgroup alike
// (the K/V offsets kernel reports it), so no key past them is read. With
// dyn_split the key splits of a sequence cover its own P + T keys
// (round32(ceil((P + T) / splits)) each), the split count fixed by the launch.
struct AttnBatch {
  int batch, row_tiles;
  const int32_t* seq_row0;
  const int64_t* seq_prefix;
  int64_t seq_stride;  // elements
  int64_t max_prefix;
  int max_rows;
  int dyn_split;
};

template <int DT>
__global__ __launch_bounds__(64 * kAttnWaves, 1) void attn_wg_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t cap,
    int nh, int nkv, int T, int64_t P, int mask_mode, const uint64_t* __restrict__ bits, int words, float scale,
    int keys_per_split, int splits, int rows_pad, float* __restrict__ opart, float* __restrict__ mlpart,
    int* __restrict__ counters, void* __restrict__ out, int64_t ld_out, int out_units, AttnBatch bt) {
  constexpr int HD = 128;
  constexpr int kQBytes = 32 * kQStride * 2;
  constexpr int kVtBytes = 32 * kVRow * 2;  // one 32-key V block, row-major
  constexpr int kCmbBytes = kAttnWaves * 32 * (kCmbRow + 2) * 4;
  constexpr int kMain = kQBytes + kAttnWaves * kVtBytes;
  constexpr int kSmem = (kMain > kCmbBytes) ? kMain : kCmbBytes;
  __shared__ __align__(16) uint8_t smem[kSmem];
  const int kvh = blockIdx.x, split = blockIdx.y;
  int rt = blockIdx.z, seq = 0;
  int rbase = 0;  // the sequence's first row in q, bits and out
  if (bt.batch > 0) {
    const int pos = blockIdx.z / bt.row_tiles;
    rt = blockIdx.z - pos * bt.row_tiles;
    seq = pos;
    if (bt.batch <= 64) {
      // Workgroups are dispatched in grid order and a launch may hold more of
      // them than there are CUs, so the sequences go longest prefix first
      // (ties by index): those dispatched last, when CUs free up, are the
      // shortest. Lane b ranks sequence b; the lane whose rank is `pos` names
      // the sequence (the ranks are a permutation of 0 .. batch - 1).
      const int lane = threadIdx.x & 63;
      int rank = -1;
      if (lane < bt.batch) {
        const int64_t pl = bt.seq_prefix[lane];
        rank = 0;
        for (int j = 0; j < bt.batch; ++j) {
          const int64_t pj = bt.seq_prefix[j];
          rank += (pj > pl || (pj == pl && j < lane)) ? 1 : 0;
        }
      }
      const uint64_t hit = __builtin_amdgcn_ballot_w64(rank == pos);
      seq = hit ? (int)__builtin_ctzll(hit) : pos;
    }
    rbase = bt.seq_row0[seq];
    T = bt.seq_row0[seq + 1] - rbase;
    P = bt.seq_prefix[seq];
    if (rt * 32 >= T * (nh / nkv) || T <= 0 || T > bt.max_rows || P < 0 || P > bt.max_prefix) return;
    if (bt.dyn_split) keys_per_split = (int)((((P + T) + splits - 1) / splits + 31) / 32 * 32);
    q += (int64_t)rbase * nh * 128;
    bits += (int64_t)rbase * words;
    kc += seq * bt.seq_stride;
    vc += seq * bt.seq_stride;
  }
  const int G = nh / nkv, rows = T * G;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ln = lane & 31, g = lane >> 5;
  const int64_t S = P + T;
  const int64_t ks0 = (int64_t)split * keys_per_split;
  // causal rows of this tile see keys up to P + their last query index
  const int64_t kvis = mask_mode == PE_MASK_CAUSAL ? P + min(T - 1, (rt * 32 + 31) / G) + 1 : S;
  const int64_t ks1 = min(min(S, kvis), ks0 + keys_per_split);
  const int nb = ks1 > ks0 ? (int)((ks1 - ks0 + 31) / 32) : 0;  // trailing splits may be empty
  const int b0 = (nb * wave) / kAttnWaves, b1 = (nb * (wave + 1)) / kAttnWaves;
  const int64_t j1 = min(ks1, ks0 + 32 * (int64_t)b1);  // end of this wave's keys
  const int64_t jlast = j1 - 1;
  uint16_t(*qs)[kQStride] = (uint16_t(*)[kQStride])smem;
  uint16_t(*vs)[kVRow] = (uint16_t(*)[kVRow])(smem + kQBytes + wave * kVtBytes);

  // wave-uniform bases and 32-bit byte offsets (a head's cache rows span
  // cap * 256 bytes < 4 GiB), so each load is base + one offset register
  const char* kbase = (const char*)(kc + (int64_t)kvh * cap * HD);
  const char* vbase = (const char*)(vc + (int64_t)kvh * cap * HD);
  // Rows past the wave's last key (or, for a wave without keys, row 0) are
  // clamped to it. The loads of the rounds after the first pair are
  // unconditional, so each wait there is an exact count of the loads issued
  // after the awaited one.
  const int jcl = (int)max(jlast, (int64_t)0);  // a row index of one head: below cap < 2^24
  u32x4_t kf[2][8], vf[2][8];
  auto load_k = [&](int64_t jb, int slot) {
    const uint32_t ko = (uint32_t)min((int)jb + ln, jcl) * (HD * 2) + 16 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) kf[slot][j] = *(const u32x4_t*)(kbase + ko + 32 * j);
  };
  auto load_v = [&](int64_t jb, int slot) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      // 32 keys x 16 chunks of 8 dims: lane covers key 4c + lane / 16, chunk lane % 16
      const uint32_t vo = (uint32_t)min((int)jb + 4 * c + (lane >> 4), jcl) * (HD * 2) + (lane & 15) * 16;
      vf[slot][c] = *(const u32x4_t*)(vbase + vo);
    }
  };
  // the row's ancestor bits, then Q (rows past `rows` read row rows - 1 and
  // stage zeros), then the first pair's K and V: all requested before
  // anything waits, and staging Q waits for Q alone
  const int r = rt * 32 + ln;
  const int t = r < rows ? r / G : 0;
  constexpr int kQChunks = 512 / (64 * kAttnWaves);  // 32 rows x 16 chunks of 8 dims
  const u32x4_t zero4 = {0u, 0u, 0u, 0u};
  u32x4_t qv[kQChunks];
  bool qok[kQChunks];
#pragma unroll
  for (int c = 0; c < kQChunks; ++c) {
    const int chunk = c * 64 * kAttnWaves + threadIdx.x;
    const int qr = chunk >> 4, dc = chunk & 15;
    const int rr0 = rt * 32 + qr;
    qok[c] = rr0 < rows;
    const int rr = min(rr0, rows - 1);
    qv[c] = *(const u32x4_t*)(q + ((int64_t)(rr / G) * nh + kvh * G + rr % G) * HD + dc * 8);
  }
  uint64_t nbits[PE_TREE_MAX_WORDS];
  if (mask_mode == PE_MASK_TREE) {
    // a visible tree key u < T <= 64 * words only reads words below `words`
#pragma unroll
    for (int w = 0; w < PE_TREE_MAX_WORDS; ++w) nbits[w] = bits[(int64_t)t * words + min(w, words - 1)];
  } else {
#pragma unroll
    for (int w = 0; w < PE_TREE_MAX_WORDS; ++w) nbits[w] = 0ull;
  }
  // the first pair (a wave's last block may be a single one: then only its
  // first block is requested, and staging Q waits for that block too)
  const bool pair2 = b0 + 1 < b1;
  load_k(ks0 + 32 * (int64_t)b0, 0);
  if (pair2) load_k(ks0 + 32 * (int64_t)b0 + 32, 1);
  load_v(ks0 + 32 * (int64_t)b0, 0);
  if (pair2) load_v(ks0 + 32 * (int64_t)b0 + 32, 1);
  __builtin_amdgcn_sched_barrier(0);  // every load issued before staging Q waits for Q
#pragma unroll
  for (int c = 0; c < kQChunks; ++c) {
    const int chunk = c * 64 * kAttnWaves + threadIdx.x;
    *(u32x4_t*)&qs[chunk >> 4][(chunk & 15) * 8] = qok[c] ? qv[c] : zero4;
  }


  // O^T accumulators; the first pair's PV MFMAs start from zero, so O holds
  // no registers while the first pair's K and V are in flight
  f32x16_t o[4];
  float m = kInitMax, l = 0.f;
  __syncthreads();  // Q staged

  const float scale2 = scale * 1.44269504088896341f;  // natural-log scores -> base 2
  // kPair: the block pair in K and V slots 0 and 1, else one block in K slot
  // KS and V slot 0. kNext: requests the block after this one, K into the
  // other K slot (a pair's: into slot 0 once its QK products have read both)
  // and V into V slot 0 once this block's V is in LDS; a pair that
  // prefetches has two blocks.
  auto process = [&](int64_t jb, auto first_c, auto pair_c, auto ks_c, auto next_c) {
    constexpr bool kFirst = decltype(first_c)::value;
    constexpr bool kPair = decltype(pair_c)::value;
    constexpr int KS = decltype(ks_c)::value;
    constexpr bool kNext = decltype(next_c)::value;
    const bool two = kPair && (kNext || jb + 32 < j1);  // wave-uniform: the pair's second block has keys
    const int64_t jn = jb + (kPair ? 64 : 32);          // the next block
    if constexpr (kNext && !kPair) load_k(jn, 1 - KS);
    // ---- S^T = K Q^T over hd, two 32-key halves
    f32x16_t sc[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[sb][i] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u32x4_t qf = *(const u32x4_t*)&qs[ln][16 * j + 8 * g];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        if (sb == 1 && !two) break;
        if constexpr (DT == PE_DTYPE_F16)
          sc[sb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, kf[KS + sb][j]),
                                                          __builtin_bit_cast(f16x8_t, qf), sc[sb], 0, 0, 0);
        else
          sc[sb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[KS + sb][j]),
                                                           __builtin_bit_cast(bf16x8_t, qf), sc[sb], 0, 0, 0);
      }
    }
    if constexpr (kNext && kPair) load_k(jn, 0);
    // ---- mask, pair max (sc[sb][i] holds key jb + 32 sb + 8*(i/4) + 4*g + (i%4) of row ln).
    // The max is taken over the unscaled products (scale2 > 0, so it commutes
    // with the scaling) and each exponent is one fma; a masked key is -inf,
    // its probability exactly zero. Padding rows (past `rows`, zero Q) are
    // computed like the others and never stored.
    float bmax = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (sb == 1 && !two) break;
      const int64_t kb = jb + 32 * sb;
      if (kb + 32 <= min(P, j1) && (mask_mode == PE_MASK_TREE || kb + 32 <= P + 1)) {
        // a whole 32-key half of prefix keys: every key is visible to every node
#pragma unroll
        for (int i = 0; i < 16; ++i) bmax = fmaxf(bmax, sc[sb][i]);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int64_t kj = kb + 8 * (i >> 2) + 4 * g + (i & 3);
          const bool ok = kj < j1 && key_allowed(kj, P, t, mask_mode, nbits);
          sc[sb][i] = ok ? sc[sb][i] : -INFINITY;
          bmax = fmaxf(bmax, sc[sb][i]);
        }
      }
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64)) * scale2;
    const float mnew = fmaxf(m, bmax);
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    float psum = 0.f;
    uint32_t pb[2][8];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        if (sb == 1 && !two) {
          pb[sb][i >> 1] = 0u;
          continue;
        }
        const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[sb][i], scale2, -mnew));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[sb][i + 1], scale2, -mnew));
        psum += p0 + p1;
        pb[sb][i >> 1] = (DT == PE_DTYPE_F16)
                             ? ((uint32_t)f32_to_f16_bits(p0) | ((uint32_t)f32_to_f16_bits(p1) << 16))
                             : ((uint32_t)f32_to_bf16_bits(p0) | ((uint32_t)f32_to_bf16_bits(p1) << 16));
      }
    psum += __shfl_xor(psum, 32, 64);
    l = l * alpha + psum;
    // rescale O only if some row's running max moved (alpha == 1 leaves O as is)
    const bool rescale = __builtin_amdgcn_ballot_w64(mnew != m) != 0ull;
    m = mnew;
    if (!kFirst && rescale) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[h][i] *= alpha;
    }
    // ---- O^T += V^T P^T, one 32-key half at a time: V rows to LDS with 16-byte
    // stores, then ds_read_b64_tr_b16 hands each lane 4 consecutive keys of one
    // dim (within a 16-lane group, out lane i gets element i % 4 of the 8 bytes
    // at source lanes i / 4 + 4k, k < 4: source lane j points at key kb + j / 4,
    // dims db + 4 (j % 4), so out lane i holds dim db + i of keys kb .. kb + 3).
    const int qg = lane >> 4, jl = lane & 15;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (sb == 1 && !two) break;
      if (sb == 1) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) *(u32x4_t*)&vs[4 * c + (lane >> 4)][(lane & 15) * 8] = vf[sb][c];
      if constexpr (kNext)
        if (sb == (kPair ? 1 : 0)) load_v(jn, 0);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int cq = 0; cq < 2; ++cq) {
        const int c = 2 * sb + cq;  // 16-key quarter of the pair
        u32x4_t bp;
        bp[0] = pb[sb][4 * cq + 0];
        bp[1] = pb[sb][4 * cq + 1];
        bp[2] = pb[sb][4 * cq + 2];
        bp[3] = pb[sb][4 * cq + 3];
        // the P^T operand (from the S^T accumulator) holds keys 4g + {0..3} and
        // 8 + 4g + {0..3} of the quarter in lane group g; V^T follows the same order
        const int kb = 16 * cq + 4 * (qg >> 1) + (jl >> 2);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int db = 32 * h + 16 * (qg & 1) + 4 * (jl & 3);
          typedef short s4v_t __attribute__((__vector_size__(4 * sizeof(short))));
          typedef __attribute__((address_space(3))) s4v_t lds_s4v_t;
          const s4v_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v_t*)&vs[kb][db]);
          const s4v_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v_t*)&vs[kb + 8][db]);
          const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
          u32x4_t a;
          a[0] = l2.x;
          a[1] = l2.y;
          a[2] = h2.x;
          a[3] = h2.y;
          f32x16_t cin = o[h];
          if (kFirst && c == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) cin[i] = 0.f;
          }
          if constexpr (DT == PE_DTYPE_F16)
            o[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                          __builtin_bit_cast(f16x8_t, bp), cin, 0, 0, 0);
          else
            o[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                           __builtin_bit_cast(bf16x8_t, bp), cin, 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  constexpr std::integral_constant<int, 0> kK0{};
  constexpr std::integral_constant<int, 1> kK1{};
  if (b0 + 2 < b1) {
    // more blocks after the first pair: one block per round, the next block's
    // K and V in flight during each round (K slots alternate)
    process(ks0 + 32 * (int64_t)b0, std::true_type(), std::true_type(), kK0, std::true_type());
    int b = b0 + 2;
    for (; b + 2 < b1; b += 2) {
      process(ks0 + 32 * (int64_t)b, std::false_type(), std::false_type(), kK0, std::true_type());
      process(ks0 + 32 * (int64_t)b + 32, std::false_type(), std::false_type(), kK1, std::true_type());
    }
    if (b + 1 < b1) {
      process(ks0 + 32 * (int64_t)b, std::false_type(), std::false_type(), kK0, std::true_type());
      process(ks0 + 32 * (int64_t)b + 32, std::false_type(), std::false_type(), kK1, std::false_type());
    } else {
      process(ks0 + 32 * (int64_t)b, std::false_type(), std::false_type(), kK0, std::false_type());
    }
  } else if (b0 < b1) {
    process(ks0 + 32 * (int64_t)b0, std::true_type(), std::true_type(), kK0, std::false_type());
  } else {
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[h][i] = 0.f;
  }

  // ---- merge the waves (wave order) with all threads: thread (row, kDimsT-dim
  // chunk) sums its outputs over the waves; the merged (O, m, l) is this
  // workgroup's split partial (a single split writes the output).
  __syncthreads();  // every wave is done with Q and its V^T tile
  float* cmb = (float*)smem;                     // [wave][row][kCmbRow]: O of the wave's keys
  float* mlw = cmb + kAttnWaves * 32 * kCmbRow;  // [wave][row][2]: m, l
  // o[h][4c .. 4c + 3] are dims 32 h + 8 c + 4 g + 0..3 of row ln: 16-byte stores
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *(f32x4_t*)&cmb[(wave * 32 + ln) * kCmbRow + h * 32 + 8 * c + 4 * g] =
          f32x4_t{o[h][4 * c], o[h][4 * c + 1], o[h][4 * c + 2], o[h][4 * c + 3]};
  if (g == 0) {
    mlw[(wave * 32 + ln) * 2] = m;
    mlw[(wave * 32 + ln) * 2 + 1] = l;
  }
  __syncthreads();
  constexpr int kDimsT = HD * 32 / (64 * kAttnWaves);  // output dims per thread
  const int row = threadIdx.x / (HD / kDimsT), dc = (threadIdx.x % (HD / kDimsT)) * kDimsT;
  float M = kInitMax;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, mlw[(w * 32 + row) * 2]);
  float L = 0.f, acc[kDimsT];
#pragma unroll
  for (int k = 0; k < kDimsT; ++k) acc[k] = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) {
    const float wt = __builtin_amdgcn_exp2f(mlw[(w * 32 + row) * 2] - M);
    L += wt * mlw[(w * 32 + row) * 2 + 1];
#pragma unroll
    for (int k4 = 0; k4 < kDimsT / 4; ++k4) {
      const f32x4_t cv = *(const f32x4_t*)&cmb[(w * 32 + row) * kCmbRow + dc + 4 * k4];
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[4 * k4 + k] += wt * cv[k];
    }
  }
  const int rr = rt * 32 + row;
  auto write_out = [&](const float (&num)[kDimsT], float den) {
    if (rr >= rows) return;
    const int tt = rr / G + rbase, col0 = (kvh * G + rr % G) * HD + dc;
    typedef typename Elem<DT>::T Te;
    if (!out_units && ((ld_out & 3) || ((uintptr_t)out & 7))) {  // row-major output not 8-byte aligned
#pragma unroll
      for (int k = 0; k < kDimsT; ++k) Elem<DT>::store((Te*)out, (int64_t)tt * ld_out + col0 + k, num[k] / den);
      return;
    }
    // four consecutive dims per store (consecutive in either layout)
#pragma unroll
    for (int k4 = 0; k4 < kDimsT / 4; ++k4) {
      float o4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o4[i] = num[4 * k4 + i] / den;
      const int col = col0 + 4 * k4;
      Vec4<DT>::store((Te*)out + (out_units ? xtile_index(tt, col, out_units) : (int64_t)tt * ld_out + col), o4);
    }
  };
  if (splits == 1) {
    write_out(acc, L);
    return;
  }
  // partial[pair][split][row][128] and ml[pair][split][row][4] (m, l, -, -),
  // pair = kvh * row_tiles + rt
  const int row_tiles = bt.batch > 0 ? bt.row_tiles : rows_pad >> 5;
  const int nseq = bt.batch > 0 ? bt.batch : 1;
  const int pair = (seq * nkv + kvh) * row_tiles + rt;
  const uint32_t nrows = (uint32_t)(nseq * nkv * row_tiles * splits * 32);
  const __amdgpu_buffer_rsrc_t ro = agent_rsrc(opart, nrows * HD * 4), rm = agent_rsrc(mlpart, nrows * 16);
  auto prow = [&](int sp) -> uint32_t { return (uint32_t)((pair * splits + sp) * 32 + row); };
  if (rr < rows) {  // padding rows of the tile are neither stored nor combined
#pragma unroll
    for (int k = 0; k < kDimsT / 4; ++k)
      store_agent_x4(ro, (prow(split) * HD + dc) * 4 + 16 * k,
                     f32x4_t{acc[4 * k], acc[4 * k + 1], acc[4 * k + 2], acc[4 * k + 3]});
    if (dc == 0) store_agent_x4(rm, prow(split) * 16, f32x4_t{M, L, 0.f, 0.f});
  }
  // the stores are acknowledged at agent scope before this workgroup counts itself
  __builtin_amdgcn_s_waitcnt(0);
  // Each workgroup adds one to the pair's counter; the one that brings it to
  // `splits` is the last of this launch and, once it has written the output,
  // sets it back to zero (every other split has counted itself by then, so
  // nothing of this launch adds to it again, and the next launch starts after
  // this one ends; issued last, the store delays none of the combine's loads).
  __shared__ int s_arrived;
  __syncthreads();
  if (threadIdx.x == 0)
    s_arrived = __hip_atomic_fetch_add(counters + pair, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_arrived + 1 != splits) return;
  float Mx = kInitMax, den = 0.f, num[kDimsT];
#pragma unroll
  for (int k = 0; k < kDimsT; ++k) num[k] = 0.f;
  for (int c0 = 0; c0 < splits; c0 += 8) {  // up to 8 splits' loads in flight
    f32x4_t ov[8][kDimsT / 4], mv[8];
    // every load unconditional (a split past the last reads this workgroup's
    // own partial, a padding row its own slot; neither value is used), so all
    // of them are in flight together
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int sp = c0 + c < splits ? c0 + c : split;
#pragma unroll
      for (int k = 0; k < kDimsT / 4; ++k) ov[c][k] = load_agent_x4(ro, (prow(sp) * HD + dc) * 4 + 16 * k);
      mv[c] = load_agent_x4(rm, prow(sp) * 16);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int sp = c0 + c;
      if (sp >= splits) break;
      const float ms = sp == split ? M : mv[c][0], ls = sp == split ? L : mv[c][1];
      const float mn = fmaxf(Mx, ms);
      const float a = __builtin_amdgcn_exp2f(Mx - mn), wt = __builtin_amdgcn_exp2f(ms - mn);
      Mx = mn;
      den = den * a + wt * ls;
#pragma unroll
      for (int k = 0; k < kDimsT; ++k) num[k] = num[k] * a + wt * (sp == split ? acc[k] : ov[c][k >> 2][k & 3]);
    }
  }
  write_out(num, den);
  if (threadIdx.x == 0) __hip_atomic_store(counters + pair, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Batched attention with two row tiles per wave. One workgroup = 4 waves (one
// per SIMD, so a wave may hold up to 512 VGPRs) = one (KV head, sequence,
// pair of 32-row tiles); every key of the sequence in one split, each wave a
// quarter of the key blocks. Every K fragment feeds the S^T products of both
// tiles and every transposed V read the PV products of both, so each K/V byte
// a CU reads serves 64 query rows instead of 32, and a (sequence, KV head)
// with five row tiles (G = 5 query heads x 26 nodes) needs three workgroups
// instead of five. A pair's second tile may lie past the sequence's rows (the
// fifth of five): then only the first is computed. Each round: the next
// block's K (into the other of two K slots) and V (once this block's V is in
// LDS) in flight, every load unconditional (rows clamped to the wave's last
// key), so the waits are exact counts. The softmax arithmetic is
// attn_wg_kernel's; the waves' (O, m, l) are merged per tile in LDS in wave
// order.
constexpr int kPairWaves = 4;

template <int DT>
__global__ __launch_bounds__(64 * kPairWaves, 1) void attn_pair_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t cap,
    int nh, int nkv, const uint64_t* __restrict__ bits, int words, float scale, void* __restrict__ out,
    int64_t ld_out, int out_units, AttnBatch bt) {
  constexpr int HD = 128;
  constexpr int kQBytes = 32 * kQStride * 2;
  constexpr int kVtBytes = 32 * kVRow * 2;
  constexpr int kCmbBytes = kPairWaves * 32 * (kCmbRow + 2) * 4;
  constexpr int kMain = 2 * kQBytes + kPairWaves * kVtBytes;
  constexpr int kSmem = (kMain > kCmbBytes) ? kMain : kCmbBytes;
  __shared__ __align__(16) uint8_t smem[kSmem];
  const int kvh = blockIdx.x;
  const int tpairs = (bt.row_tiles + 1) / 2;
  const int pos = blockIdx.z / tpairs, tp = blockIdx.z - pos * tpairs;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ln = lane & 31, g = lane >> 5;
  int seq = pos;
  if (bt.batch <= 64) {  // longest prefix first, as attn_wg_kernel orders them
    int rank = -1;
    if (lane < bt.batch) {
      const int64_t pl = bt.seq_prefix[lane];
      rank = 0;
      for (int j = 0; j < bt.batch; ++j) {
        const int64_t pj = bt.seq_prefix[j];
        rank += (pj > pl || (pj == pl && j < lane)) ? 1 : 0;
      }
    }
    const uint64_t hit = __builtin_amdgcn_ballot_w64(rank == pos);
    seq = hit ? (int)__builtin_ctzll(hit) : pos;
  }
  const int rbase = bt.seq_row0[seq];
  const int T = bt.seq_row0[seq + 1] - rbase;
  const int64_t P = bt.seq_prefix[seq];
  const int G = nh / nkv, rows = T * G;
  const int rtA = 2 * tp, rtB = 2 * tp + 1;
  if (T <= 0 || rtA * 32 >= rows || T > bt.max_rows || P < 0 || P > bt.max_prefix) return;
  const bool two = rtB * 32 < rows;  // workgroup-uniform: one body per case
  auto body = [&](auto two_c) {
  constexpr bool TWO = decltype(two_c)::value;
  q += (int64_t)rbase * nh * HD;
  bits += (int64_t)rbase * words;
  kc += seq * bt.seq_stride;
  vc += seq * bt.seq_stride;
  const int64_t S = P + T;
  const int nb = (int)((S + 31) / 32);
  const int b0 = (nb * wave) / kPairWaves, b1 = (nb * (wave + 1)) / kPairWaves;
  const int64_t j1 = min(S, 32 * (int64_t)b1);
  const int jcl = (int)max(j1 - 1, (int64_t)0);  // a row index of one head: below cap < 2^24
  uint16_t(*qsA)[kQStride] = (uint16_t(*)[kQStride])smem;
  uint16_t(*qsB)[kQStride] = (uint16_t(*)[kQStride])(smem + kQBytes);
  uint16_t(*vs)[kVRow] = (uint16_t(*)[kVRow])(smem + 2 * kQBytes + wave * kVtBytes);
  const char* kbase = (const char*)(kc + (int64_t)kvh * cap * HD);
  const char* vbase = (const char*)(vc + (int64_t)kvh * cap * HD);
  u32x4_t kf[2][8], vf[8];
  auto load_k = [&](int jb, int slot) {
    const uint32_t ko = (uint32_t)min(jb + ln, jcl) * (HD * 2) + 16 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) kf[slot][j] = *(const u32x4_t*)(kbase + ko + 32 * j);
  };
  auto load_v = [&](int jb) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t vo = (uint32_t)min(jb + 4 * c + (lane >> 4), jcl) * (HD * 2) + (lane & 15) * 16;
      vf[c] = *(const u32x4_t*)(vbase + vo);
    }
  };
  // each lane's row in the two tiles, their ancestor bits, both tiles' Q
  // (rows past `rows` read row rows - 1 and stage zeros; never stored), then
  // the first block: all requested before anything waits
  const int rA = rtA * 32 + ln, rB = rtB * 32 + ln;
  const int tA = rA < rows ? rA / G : 0, tB = rB < rows ? rB / G : 0;
  uint64_t nbA[PE_TREE_MAX_WORDS], nbB[PE_TREE_MAX_WORDS];
#pragma unroll
  for (int w = 0; w < PE_TREE_MAX_WORDS; ++w) {
    nbA[w] = bits[(int64_t)tA * words + min(w, words - 1)];
    nbB[w] = bits[(int64_t)tB * words + min(w, words - 1)];
  }
  constexpr int kQChunks = 512 / (64 * kPairWaves);
  u32x4_t qv[2][kQChunks];
  bool qok[2][kQChunks];
#pragma unroll
  for (int tile = 0; tile < 2; ++tile)
#pragma unroll
    for (int c = 0; c < kQChunks; ++c) {
      const int chunk = c * 64 * kPairWaves + threadIdx.x;
      const int qr = chunk >> 4, dc = chunk & 15;
      const int rr0 = (tile ? rtB : rtA) * 32 + qr;
      qok[tile][c] = rr0 < rows;
      const int rr = min(rr0, rows - 1);
      qv[tile][c] = *(const u32x4_t*)(q + ((int64_t)(rr / G) * nh + kvh * G + rr % G) * HD + dc * 8);
    }
  load_k(32 * b0, 0);
  load_v(32 * b0);
  __builtin_amdgcn_sched_barrier(0);
  const u32x4_t zero4 = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int tile = 0; tile < 2; ++tile)
#pragma unroll
    for (int c = 0; c < kQChunks; ++c) {
      const int chunk = c * 64 * kPairWaves + threadIdx.x;
      uint16_t(*qs)[kQStride] = tile ? qsB : qsA;
      *(u32x4_t*)&qs[chunk >> 4][(chunk & 15) * 8] = qok[tile][c] ? qv[tile][c] : zero4;
    }
  f32x16_t oA[4], oB[4];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int i = 0; i < 16; ++i) oA[h][i] = oB[h][i] = 0.f;
  float mA = kInitMax, lA = 0.f, mB = kInitMax, lB = 0.f;
  __syncthreads();  // both Q tiles staged

  const float scale2 = scale * 1.44269504088896341f;  // natural-log scores -> base 2
  const int qg = lane >> 4, jl = lane & 15;
  // online softmax of one tile's 32 keys: returns the packed probabilities
  auto softmax = [&](f32x16_t& sc, int64_t jb, bool whole, const uint64_t (&nb)[PE_TREE_MAX_WORDS],
                     float& m, float& l, f32x16_t (&o)[4], uint32_t (&pb)[8]) {
    float bmax = -INFINITY;
    if (whole) {
#pragma unroll
      for (int i = 0; i < 16; ++i) bmax = fmaxf(bmax, sc[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t kj = jb + 8 * (i >> 2) + 4 * g + (i & 3);
        const bool ok = kj < j1 && tree_key_allowed(kj, P, nb);
        sc[i] = ok ? sc[i] : -INFINITY;
        bmax = fmaxf(bmax, sc[i]);
      }
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64)) * scale2;
    // a row keeps its running max until a block's exceeds it by more than
    // 2^8: its probabilities stay below 2^8 and O (held in the matrix-core
    // accumulators) is rescaled in a few rounds only
    const float mnew = bmax > m + 8.f ? bmax : m;
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[i], scale2, -mnew));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[i + 1], scale2, -mnew));
      psum += p0 + p1;
      pb[i >> 1] = pack2_16<DT>(p0, p1);
    }
    psum += __shfl_xor(psum, 32, 64);
    l = l * alpha + psum;
    // rescale O only if some row's running max moved (alpha == 1 leaves O as is)
    if (__builtin_amdgcn_ballot_w64(mnew != m) != 0ull) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[h][i] *= alpha;
    }
    m = mnew;
  };
  auto process = [&](int jb, auto ks_c, auto next_c) {
    constexpr int KS = decltype(ks_c)::value;
    constexpr bool kNext = decltype(next_c)::value;
    if constexpr (kNext) load_k(jb + 32, 1 - KS);
    f32x16_t scA, scB;
#pragma unroll
    for (int i = 0; i < 16; ++i) scA[i] = scB[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u32x4_t qa = *(const u32x4_t*)&qsA[ln][16 * j + 8 * g];
      const u32x4_t qb = *(const u32x4_t*)&qsB[ln][16 * j + 8 * g];
      if constexpr (DT == PE_DTYPE_F16) {
        scA = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, kf[KS][j]),
                                                     __builtin_bit_cast(f16x8_t, qa), scA, 0, 0, 0);
        if constexpr (TWO)
          scB = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, kf[KS][j]),
                                                       __builtin_bit_cast(f16x8_t, qb), scB, 0, 0, 0);
      } else {
        scA = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[KS][j]),
                                                      __builtin_bit_cast(bf16x8_t, qa), scA, 0, 0, 0);
        if constexpr (TWO)
          scB = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[KS][j]),
                                                        __builtin_bit_cast(bf16x8_t, qb), scB, 0, 0, 0);
      }
    }
    // a whole 32-key block of prefix keys: every key is visible to every node
    const bool whole = jb + 32 <= min(P, j1);
    uint32_t pbA[8], pbB[8] = {};
    softmax(scA, jb, whole, nbA, mA, lA, oA, pbA);
    if constexpr (TWO) softmax(scB, jb, whole, nbB, mB, lB, oB, pbB);
#pragma unroll
    for (int c = 0; c < 8; ++c) *(u32x4_t*)&vs[4 * c + (lane >> 4)][(lane & 15) * 8] = vf[c];
    if constexpr (kNext) load_v(jb + 32);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int cq = 0; cq < 2; ++cq) {
      u32x4_t bpA, bpB;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bpA[e] = pbA[4 * cq + e];
        bpB[e] = pbB[4 * cq + e];
      }
      const int kb = 16 * cq + 4 * (qg >> 1) + (jl >> 2);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int db = 32 * h + 16 * (qg & 1) + 4 * (jl & 3);
        typedef short s4v_t __attribute__((__vector_size__(4 * sizeof(short))));
        typedef __attribute__((address_space(3))) s4v_t lds_s4v_t;
        const s4v_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v_t*)&vs[kb][db]);
        const s4v_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v_t*)&vs[kb + 8][db]);
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        u32x4_t a;
        a[0] = l2.x;
        a[1] = l2.y;
        a[2] = h2.x;
        a[3] = h2.y;
        if constexpr (DT == PE_DTYPE_F16) {
          oA[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                         __builtin_bit_cast(f16x8_t, bpA), oA[h], 0, 0, 0);
          if constexpr (TWO)
            oB[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                           __builtin_bit_cast(f16x8_t, bpB), oB[h], 0, 0, 0);
        } else {
          oA[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                          __builtin_bit_cast(bf16x8_t, bpA), oA[h], 0, 0, 0);
          if constexpr (TWO)
            oB[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                            __builtin_bit_cast(bf16x8_t, bpB), oB[h], 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  constexpr std::integral_constant<int, 0> kK0{};
  constexpr std::integral_constant<int, 1> kK1{};
  if (b0 < b1) {
    int b = b0;
    for (; b + 2 < b1; b += 2) {
      process(32 * b, kK0, std::true_type());
      process(32 * b + 32, kK1, std::true_type());
    }
    if (b + 1 < b1) {
      process(32 * b, kK0, std::true_type());
      process(32 * b + 32, kK1, std::false_type());
    } else {
      process(32 * b, kK0, std::false_type());
    }
  }

  // ---- per tile: merge the waves (wave order) and write the rows
  constexpr int kDimsT = HD * 32 / (64 * kPairWaves);  // output dims per thread
  const int row = threadIdx.x / (HD / kDimsT), dc = (threadIdx.x % (HD / kDimsT)) * kDimsT;
  float* cmb = (float*)smem;                     // [wave][row][kCmbRow]
  float* mlw = cmb + kPairWaves * 32 * kCmbRow;  // [wave][row][2]
  typedef typename Elem<DT>::T Te;
  auto merge_tile = [&](const f32x16_t (&o)[4], float m, float l, int rt) {
    __syncthreads();  // every wave is done with Q, its V^T tile and the previous merge
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *(f32x4_t*)&cmb[(wave * 32 + ln) * kCmbRow + h * 32 + 8 * c + 4 * g] =
            f32x4_t{o[h][4 * c], o[h][4 * c + 1], o[h][4 * c + 2], o[h][4 * c + 3]};
    if (g == 0) {
      mlw[(wave * 32 + ln) * 2] = m;
      mlw[(wave * 32 + ln) * 2 + 1] = l;
    }
    __syncthreads();
    float M = kInitMax;
#pragma unroll
    for (int w = 0; w < kPairWaves; ++w) M = fmaxf(M, mlw[(w * 32 + row) * 2]);
    float L = 0.f, acc[kDimsT];
#pragma unroll
    for (int k = 0; k < kDimsT; ++k) acc[k] = 0.f;
#pragma unroll
    for (int w = 0; w < kPairWaves; ++w) {
      const float wt = __builtin_amdgcn_exp2f(mlw[(w * 32 + row) * 2] - M);
      L += wt * mlw[(w * 32 + row) * 2 + 1];
#pragma unroll
      for (int k4 = 0; k4 < kDimsT / 4; ++k4) {
        const f32x4_t cv = *(const f32x4_t*)&cmb[(w * 32 + row) * kCmbRow + dc + 4 * k4];
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[4 * k4 + k] += wt * cv[k];
      }
    }
    const int rr = rt * 32 + row;
    if (rr >= rows) return;
    const int tt = rr / G + rbase, col0 = (kvh * G + rr % G) * HD + dc;
    if (!out_units && ((ld_out & 3) || ((uintptr_t)out & 7))) {  // row-major output not 8-byte aligned
#pragma unroll
      for (int k = 0; k < kDimsT; ++k) Elem<DT>::store((Te*)out, (int64_t)tt * ld_out + col0 + k, acc[k] / L);
      return;
    }
#pragma unroll
    for (int k4 = 0; k4 < kDimsT / 4; ++k4) {
      float o4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o4[i] = acc[4 * k4 + i] / L;
      const int col = col0 + 4 * k4;
      Vec4<DT>::store((Te*)out + (out_units ? xtile_index(tt, col, out_units) : (int64_t)tt * ld_out + col), o4);
    }
  };
  merge_tile(oA, mA, lA, rtA);
  if constexpr (TWO) merge_tile(oB, mB, lB, rtB);
  };
  if (two)
    body(std::true_type());
  else
    body(std::false_type());
}

// Eager attention on the matrix cores (PE_ATTN_EAGER, the drafter's attention,
// src/pe/nn.py:84-87, 16-bit with hd = 128), one key split, so that a
// workgroup sees every key of its rows: one workgroup = 8 waves = one (KV head,
// 32-row tile), each wave a contiguous run of the tile's 32-key blocks, walked
// twice.
//   Pass 1: S^T = K Q^T on MFMA; each score rounded as the reference rounds it
//   (the product to the dtype, divided by sqrt(hd), to the dtype again; a
//   masked key is -inf); the row's max and the fp32 sum of exp(s - max) kept
//   online; the waves' (max, sum) merged in LDS in wave order.
//   Pass 2: the same scores again; each probability exp(s - M) / L rounded to
//   the dtype, as softmax(...).to(q.dtype) leaves it, and multiplied by V on
//   MFMA (fp32 accumulation and no rescaling: M is the row's final max); the
//   waves' sums added in wave order and rounded once.
// The next block's K (both passes) and V (pass 2) are in flight during each
// block; every load of those rounds is unconditional (rows clamped to the
// wave's last key), so the waits are exact counts.
template <int DT>
__global__ __launch_bounds__(64 * kAttnWaves, 1) void attn_eager_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t cap,
    int nh, int nkv, int T, int64_t P, int mask_mode, const uint64_t* __restrict__ bits, int words,
    void* __restrict__ out, int64_t ld_out) {
  typedef Elem<DT> E;
  constexpr int HD = 128;
  constexpr int kQBytes = 32 * kQStride * 2;
  constexpr int kVtBytes = 32 * kVRow * 2;
  constexpr int kCmbBytes = kAttnWaves * 32 * kCmbRow * 4;
  constexpr int kMain = kQBytes + kAttnWaves * kVtBytes;
  constexpr int kSmem = (kMain > kCmbBytes) ? kMain : kCmbBytes;
  __shared__ __align__(16) uint8_t smem[kSmem];
  __shared__ float s_ml[kAttnWaves][32][2];
  const int kvh = blockIdx.x, rt = blockIdx.z;
  const int G = nh / nkv, rows = T * G;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ln = lane & 31, g = lane >> 5;
  const int64_t S = P + T;
  const int64_t kvis = mask_mode == PE_MASK_CAUSAL ? P + min(T - 1, (rt * 32 + 31) / G) + 1 : S;
  const int64_t ks1 = min(S, kvis);
  const int nb = (int)((ks1 + 31) / 32);
  const int b0 = (nb * wave) / kAttnWaves, b1 = (nb * (wave + 1)) / kAttnWaves;
  const int64_t j1 = min(ks1, 32 * (int64_t)b1);  // end of this wave's keys
  const int jcl = (int)max(j1 - 1, (int64_t)0);    // a row index of one head: below cap < 2^24
  uint16_t(*qs)[kQStride] = (uint16_t(*)[kQStride])smem;
  uint16_t(*vs)[kVRow] = (uint16_t(*)[kVRow])(smem + kQBytes + wave * kVtBytes);
  const char* kbase = (const char*)(kc + (int64_t)kvh * cap * HD);
  const char* vbase = (const char*)(vc + (int64_t)kvh * cap * HD);
  u32x4_t kf[2][8], vf[8];
  auto load_k = [&](int jb, int slot) {
    const uint32_t ko = (uint32_t)min(jb + ln, jcl) * (HD * 2) + 16 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) kf[slot][j] = *(const u32x4_t*)(kbase + ko + 32 * j);
  };
  auto load_v = [&](int jb) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t vo = (uint32_t)min(jb + 4 * c + (lane >> 4), jcl) * (HD * 2) + (lane & 15) * 16;
      vf[c] = *(const u32x4_t*)(vbase + vo);
    }
  };
  // the row's ancestor bits and the row tile's Q (rows past `rows` read row
  // rows - 1 and stage zeros; their outputs are never stored)
  const int r = rt * 32 + ln;
  const int t = r < rows ? r / G : 0;
  uint64_t nbits[PE_TREE_MAX_WORDS];
  if (mask_mode == PE_MASK_TREE) {
#pragma unroll
    for (int w = 0; w < PE_TREE_MAX_WORDS; ++w) nbits[w] = bits[(int64_t)t * words + min(w, words - 1)];
  } else {
#pragma unroll
    for (int w = 0; w < PE_TREE_MAX_WORDS; ++w) nbits[w] = 0ull;
  }
  constexpr int kQChunks = 512 / (64 * kAttnWaves);
  {
    u32x4_t qv[kQChunks];
    bool qok[kQChunks];
#pragma unroll
    for (int c = 0; c < kQChunks; ++c) {
      const int chunk = c * 64 * kAttnWaves + threadIdx.x;
      const int qr = chunk >> 4, dc = chunk & 15;
      const int rr0 = rt * 32 + qr;
      qok[c] = rr0 < rows;
      const int rr = min(rr0, rows - 1);
      qv[c] = *(const u32x4_t*)(q + ((int64_t)(rr / G) * nh + kvh * G + rr % G) * HD + dc * 8);
    }
    const u32x4_t zero4 = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int c = 0; c < kQChunks; ++c) {
      const int chunk = c * 64 * kAttnWaves + threadIdx.x;
      *(u32x4_t*)&qs[chunk >> 4][(chunk & 15) * 8] = qok[c] ? qv[c] : zero4;
    }
  }
  __syncthreads();  // Q staged

  const float sqrt_hd = sqrtf((float)HD);
  // the rounded scores of one block (s[i]: key jb + 8*(i/4) + 4*g + (i%4) of row ln)
  auto scores = [&](int jb, int slot, float (&s)[16]) {
    f32x16_t sc;
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u32x4_t qf = *(const u32x4_t*)&qs[ln][16 * j + 8 * g];
      if constexpr (DT == PE_DTYPE_F16)
        sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, kf[slot][j]),
                                                    __builtin_bit_cast(f16x8_t, qf), sc, 0, 0, 0);
      else
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[slot][j]),
                                                     __builtin_bit_cast(bf16x8_t, qf), sc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t kj = jb + 8 * (i >> 2) + 4 * g + (i & 3);
      const bool ok = kj < j1 && key_allowed(kj, P, t, mask_mode, nbits);
      s[i] = ok ? E::round(__fdiv_rn(E::round(sc[i]), sqrt_hd)) : -INFINITY;
    }
  };
  constexpr std::integral_constant<int, 0> kK0{};
  constexpr std::integral_constant<int, 1> kK1{};

  // ---- pass 1: the row's max and sum
  float m = kInitMax, l = 0.f;
  auto pass1 = [&](int jb, auto ks_c, auto next_c) {
    constexpr int KS = decltype(ks_c)::value;
    if constexpr (decltype(next_c)::value) load_k(jb + 32, 1 - KS);
    float s[16];
    scores(jb, KS, s);
    float bmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) bmax = fmaxf(bmax, s[i]);
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float mnew = fmaxf(m, bmax);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) psum += expf(s[i] - mnew);
    psum += __shfl_xor(psum, 32, 64);
    l = l * expf(m - mnew) + psum;
    m = mnew;
  };
  if (b0 < b1) {
    load_k(32 * b0, 0);
    int b = b0;
    for (; b + 2 < b1; b += 2) {
      pass1(32 * b, kK0, std::true_type());
      pass1(32 * b + 32, kK1, std::true_type());
    }
    if (b + 1 < b1) {
      pass1(32 * b, kK0, std::true_type());
      pass1(32 * b + 32, kK1, std::false_type());
    } else {
      pass1(32 * b, kK0, std::false_type());
    }
  }
  if (g == 0) {
    s_ml[wave][ln][0] = m;
    s_ml[wave][ln][1] = l;
  }
  __syncthreads();
  float M = kInitMax;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, s_ml[w][ln][0]);
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) L += s_ml[w][ln][1] * expf(s_ml[w][ln][0] - M);
  const float invL = 1.0f / L;

  // ---- pass 2: O = sum_j round(exp(s_j - M) / L) v_j
  f32x16_t o[4];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[h][i] = 0.f;
  const int qg = lane >> 4, jl = lane & 15;
  auto pass2 = [&](int jb, auto ks_c, auto next_c) {
    constexpr int KS = decltype(ks_c)::value;
    constexpr bool kNext = decltype(next_c)::value;
    if constexpr (kNext) load_k(jb + 32, 1 - KS);
    float s[16];
    scores(jb, KS, s);
    uint32_t pb[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = E::round(expf(s[i] - M) * invL), p1 = E::round(expf(s[i + 1] - M) * invL);
      pb[i >> 1] = pack2_16<DT>(p0, p1);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) *(u32x4_t*)&vs[4 * c + (lane >> 4)][(lane & 15) * 8] = vf[c];
    if constexpr (kNext) load_v(jb + 32);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int cq = 0; cq < 2; ++cq) {
      u32x4_t bp;
      bp[0] = pb[4 * cq + 0];
      bp[1] = pb[4 * cq + 1];
      bp[2] = pb[4 * cq + 2];
      bp[3] = pb[4 * cq + 3];
      const int kb = 16 * cq + 4 * (qg >> 1) + (jl >> 2);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int db = 32 * h + 16 * (qg & 1) + 4 * (jl & 3);
        typedef short s4v_t __attribute__((__vector_size__(4 * sizeof(short))));
        typedef __attribute__((address_space(3))) s4v_t lds_s4v_t;
        const s4v_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v_t*)&vs[kb][db]);
        const s4v_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v_t*)&vs[kb + 8][db]);
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        u32x4_t a;
        a[0] = l2.x;
        a[1] = l2.y;
        a[2] = h2.x;
        a[3] = h2.y;
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
  };
  if (b0 < b1) {
    load_k(32 * b0, 0);
    load_v(32 * b0);
    int b = b0;
    for (; b + 2 < b1; b += 2) {
      pass2(32 * b, kK0, std::true_type());
      pass2(32 * b + 32, kK1, std::true_type());
    }
    if (b + 1 < b1) {
      pass2(32 * b, kK0, std::true_type());
      pass2(32 * b + 32, kK1, std::false_type());
    } else {
      pass2(32 * b, kK0, std::false_type());
    }
  }

  // ---- the waves' sums, in wave order, rounded once
  __syncthreads();  // every wave is done with Q and its V^T tile
  float* cmb = (float*)smem;  // [wave][row][kCmbRow]
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *(f32x4_t*)&cmb[(wave * 32 + ln) * kCmbRow + h * 32 + 8 * c + 4 * g] =
          f32x4_t{o[h][4 * c], o[h][4 * c + 1], o[h][4 * c + 2], o[h][4 * c + 3]};
  __syncthreads();
  constexpr int kDimsT = HD * 32 / (64 * kAttnWaves);
  const int row = threadIdx.x / (HD / kDimsT), dc = (threadIdx.x % (HD / kDimsT)) * kDimsT;
  const int rr = rt * 32 + row;
  if (rr >= rows) return;
  float acc[kDimsT];
#pragma unroll
  for (int k = 0; k < kDimsT; ++k) acc[k] = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w)
#pragma unroll
    for (int k4 = 0; k4 < kDimsT / 4; ++k4) {
      const f32x4_t cv = *(const f32x4_t*)&cmb[(w * 32 + row) * kCmbRow + dc + 4 * k4];
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[4 * k4 + k] += cv[k];
    }
  const int tt = rr / G, col0 = (kvh * G + rr % G) * HD + dc;
#pragma unroll
  for (int k = 0; k < kDimsT; ++k) E::store((typename E::T*)out, (int64_t)tt * ld_out + col0 + k, acc[k]);
}

// Generic path (fp32, any hd <= 256; and the eager semantics where
// attn_eager_kernel does not apply: fp32, or hd != 128): one block per (row t,
// query head), all keys.
// eager (PE_ATTN_EAGER, the drafter's attention, src/pe/nn.py:84-87): the
// score is the dot product rounded to the dtype, divided by sqrt(hd) and
// rounded again (the masked keys' -inf bias leaves them out); softmax in fp32;
// each probability is normalised and rounded to the dtype before the PV
// product, which accumulates in fp32 and is rounded once.
template <int DT>
__global__ __launch_bounds__(128) void attn_generic_kernel(
    const typename Elem<DT>::T* __restrict__ q, const typename Elem<DT>::T* __restrict__ kc,
    const typename Elem<DT>::T* __restrict__ vc, int64_t cap, int nh, int nkv, int hd, int T, int64_t P,
    int mask_mode, const uint64_t* __restrict__ bits, int words, float scale, int eager,
    typename Elem<DT>::T* __restrict__ out, int64_t ld_out, float* __restrict__ scores /* [T*nh][P+T] */) {
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
  __shared__ float qs[256];  // the query row, read by every thread
  for (int d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = E::load(qr, d);
  __syncthreads();
  float lmax = kInitMax;
  for (int64_t j = threadIdx.x; j < S; j += blockDim.x) {
    float v = kMaskedScore;
    if (key_allowed(j, P, t, mask_mode, nb)) {
      const typename E::T* kr = kc + ((int64_t)kvh * cap + j) * hd;
      float acc = 0.f;
#pragma unroll 8
      for (int d = 0; d < hd; ++d) acc = fmaf(qs[d], E::load(kr, d), acc);
      v = eager ? E::round(__fdiv_rn(E::round(acc), sqrtf((float)hd))) : acc * scale;
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
  const float invL = 1.0f / L;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.f;
    // every key row below S is cache memory, so the loads are unconditional
    // (independent, several in flight); masked keys (p == 0) add nothing
#pragma unroll 8
    for (int64_t j = 0; j < S; ++j) {
      const float p = sc[j];
      const float v = E::load(vc + ((int64_t)kvh * cap + j) * hd, d);
      const float pr = eager ? E::round(__fmul_rn(p, invL)) : E::round(p);
      acc = p != 0.f ? fmaf(pr, v, acc) : acc;
    }
    E::store(out, (int64_t)t * ld_out + (int64_t)hq * hd + d, eager ? acc : acc / L);
  }
}

// per-pair arrival counters: zero before first use and between launches
constexpr int64_t kAttnCounterBytes = 4096;

struct AttnPlan {
  int splits, keys_per_split, row_tiles, rows_pad;
  int64_t opart_bytes, ml_bytes;  // workspace: [counters | O partials | (m, l) partials]
};

AttnPlan attn_plan(int T, int nh, int nkv, int64_t S, int batch = 1) {
  AttnPlan p;
  const int rows = T * (nh / nkv);
  p.row_tiles = (rows + 31) / 32;
  p.rows_pad = p.row_tiles * 32;
  // about one 32-key block per wave (a wave takes up to a pair in one round),
  // with at most one workgroup per CU; longer caches give each wave more
  // rounds of pairs
  const int64_t pairs = (int64_t)batch * nkv * p.row_tiles;
  int64_t want = ((S + 31) / 32 + kAttnWaves - 1) / kAttnWaves;
  int64_t cap_splits = 256 / pairs;
  if (cap_splits > kAttnMaxSplits) cap_splits = kAttnMaxSplits;
  if (want > cap_splits) want = cap_splits;
  const int64_t pw = want > 1 ? want : 1;
  int64_t kps = (S + pw - 1) / pw;
  kps = ((kps + 31) / 32) * 32;
  p.keys_per_split = (int)kps;
  p.splits = (int)pw;
  p.opart_bytes = (int64_t)batch * nkv * p.splits * p.rows_pad * 128 * 4;
  p.ml_bytes = (int64_t)batch * nkv * p.splits * p.rows_pad * 4 * 4;
  return p;
}

// The chunk permutation of K / V row `row` in an LDS step buffer (physical
// chunk = logical chunk ^ swz_row(row)). With i = row % 4 and j = row / 4 % 4
// it is (2i ^ 4i ^ j) % 16: a bijection on 16 consecutive rows (so the K
// fragment reads, 16 bytes of one chunk from each of 16 consecutive rows, fall
// on distinct banks), and for four rows 4k .. 4k + 3 it moves bits 1-3 of the
// chunk differently per row, so that the transposed V reads (8 bytes from each
// of two or four neighbouring chunks of those four rows) do as well. Plain
// row % 16 left those V reads two- to four-way conflicted.
__device__ __forceinline__ int swz_row(int row) {
  const int i = row & 3, j = (row >> 2) & 3;
  return ((i << 1) ^ (i << 2) ^ j) & 15;
}

// Byte offset of 16-byte chunk `chunk` of a 256-byte K / V row in an LDS step
// buffer.
__device__ __forceinline__ uint32_t swz(int row, int chunk) { return (uint32_t)(row * 256 + ((chunk ^ swz_row(row)) << 4)); }

// Visibility of the 64 keys kb0 .. kb0 + 63 to one query row, as a bit mask
// (bit j: key kb0 + j), so that each score register tests a bit at an offset
// fixed at compile time. Built with wave-uniform branches only: a per-lane
// branch around each score (the tree test nested in the prefix test) was
// compiled for gfx950 into code that overwrote the first score register with
// the node index and left that score masked whenever the key was a node key.
// Tree rows: prefix keys (< P) visible, node key P + u visible when bit u of
// the row's ancestor bits nb (up to four words) is set.
__device__ __forceinline__ uint64_t tree_window(int64_t kb0, int64_t P, const uint64_t* nb) {
  const int64_t off = kb0 - P;  // node index of key kb0
  if (off <= -64) return ~0ull;
  if (off < 0) {
    const int j0 = (int)(-off);  // 1 .. 63: keys below kb0 + j0 are prefix keys
    return ((1ull << j0) - 1) | (nb[0] << j0);
  }
  if (off >= 64 * PE_TREE_MAX_WORDS) return 0ull;
  const int wi = (int)(off >> 6), sh = (int)(off & 63);
  static_assert(PE_TREE_MAX_WORDS == 4, "one select per word");
  const uint64_t a = wi == 0 ? nb[0] : wi == 1 ? nb[1] : wi == 2 ? nb[2] : nb[3];
  const uint64_t b = wi == 0 ? nb[1] : wi == 1 ? nb[2] : wi == 2 ? nb[3] : 0ull;
  return sh ? (a >> sh) | (b << (64 - sh)) : a;
}

// Causal rows: keys up to kvis visible.
__device__ __forceinline__ uint64_t causal_window(int64_t kb0, int64_t kvis) {
  const int64_t d = kvis - kb0;  // the last visible key's offset in the step
  return d >= 63 ? ~0ull : (d < 0 ? 0ull : (2ull << d) - 1);
}

// Keys at or past kend do not exist: clear their bits.
__device__ __forceinline__ uint64_t window_limit(uint64_t win, int64_t kb0, int64_t kend) {
  const int64_t lim = kend - kb0;
  return lim >= 64 ? win : (lim <= 0 ? 0ull : win & ((1ull << lim) - 1));
}

// ---------------------------------------------------------------------------
// Causal attention over many query rows (the prompt prefill)
// ---------------------------------------------------------------------------
// A KV head's query rows (T nodes x G query heads, row r = node r / G, query
// head r % G) are cut into blocks of 128 rows. Causally, block b sees about
// (b + 1) / nblk of the keys, so one workgroup takes the pair of blocks
// (nblk - 1 - i, i) in turn and every workgroup does the same work. Eight
// waves: wave w owns 32-row tile w % 4 of the block and, in key group w / 4,
// every other 64-key step (group 0 the even steps, group 1 the odd ones), so
// each SIMD runs two waves on independent work. The next iteration's two
// steps of K and V (128 keys) go straight from global memory into the other
// half of a four-step LDS ring (global_load_lds_dwordx4, rows unpadded, their
// 16-byte chunks swizzled by row as in attn_batch_rows_kernel) while every
// wave multiplies its tile by its step of this iteration: S^T = K Q^T
// (A = K from LDS, B = the wave's Q^T, held in registers), the online softmax
// in base 2 on the S^T accumulators (each lane one row and 16 keys of every
// 32-key half), O^T += V^T P^T (A = V^T by transposed LDS reads, B = P^T
// rounded to the compute dtype). At the end of a block group 1 hands its
// (O, m, l) to group 0 through LDS, which merges the two (group 0 first) and
// writes out = O / l. The arithmetic is attn_wg_kernel's: scores scaled by
// scale * log2 e, fp32 maxima and sums, probabilities rounded before PV. Keys
// past the visible range are masked to -inf (probability exactly zero); key
// rows past the cache fill (P + T) are read as row P + T - 1, so no
// uninitialised row reaches the products. Work item w of the nkv x npair grid
// runs on XCD w / (grid / 8) when the grid is a multiple of eight (workgroup
// b starts on XCD b % 8), so the row blocks of a KV head share one L2.
constexpr int kRowsWaves = 8;
constexpr int kRowsKeys = 64;            // keys per step
constexpr int kRowsStepBytes = 2 * kRowsKeys * 256;  // one step's K and V rows, unpadded (swizzled chunks)
constexpr int kRowsSmem = 4 * kRowsStepBytes;         // two iterations of two steps
// group 1's hand-over: per tile and lane 64 O values, m and l (rows of 68 floats: 16-byte aligned)
constexpr int kRowsMergeStride = 64 + 4;
constexpr int kRowsMergeBytes = 4 * 64 * kRowsMergeStride * 4;
static_assert(kRowsMergeBytes <= kRowsSmem, "the merge reuses the step buffers");
// causal passes of at least this many nodes take attn_rows_kernel
constexpr int kRowsMinNodes = 256;

template <int DT>
__global__ __launch_bounds__(64 * kRowsWaves, 1) void attn_rows_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t cap,
    int nh, int nkv, int T, int64_t P, float scale, int nblk, int npair, void* __restrict__ out, int64_t ld_out,
    int out_units) {
  constexpr int HD = 128;
  __shared__ __align__(1024) uint8_t smem[kRowsSmem];
  const int total = nkv * npair;
  const int b = blockIdx.x;
  const int w = (total & 7) ? b : (b & 7) * (total >> 3) + (b >> 3);
  const int kvh = w / npair, pair = w - kvh * npair;
  const int G = nh / nkv, rows = T * G;
  const int64_t S = P + T;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, ln = lane & 31, g = lane >> 5;
  const int tile = wave & 3, kg = wave >> 2;
  const uint16_t* kh = kc + (int64_t)kvh * cap * HD;
  const uint16_t* vh = vc + (int64_t)kvh * cap * HD;
  const float scale2 = scale * 1.44269504088896341f;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  // iteration it's two steps (2 it + group) go to step buffers 2 (it % 2) + group:
  // wave w loads step 2 it + w / 4, its loads 8 (w % 4) .. + 7 of the step's
  // 32 (K rows 4 i .. 4 i + 3 for i < 16, else V rows 4 (i - 16) ..), each
  // lane one 16-byte chunk, swizzled by row
  const int dsp = wave >> 2, dq = wave & 3;
  const uint16_t* dsrc = uniform_ptr(dq < 2 ? kh : vh);
  auto issue_pair = [&](int it) {
    const int64_t kb0 = (int64_t)(2 * it + dsp) * kRowsKeys;
    const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_base + (2 * (it & 1) + dsp) * kRowsStepBytes +
                                                        (dq < 2 ? 0 : 16384) + (dq & 1) * 8192);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int row = 32 * (dq & 1) + 4 * k + (lane >> 4);
      const uint32_t key = (uint32_t)min(kb0 + row, S - 1);
      lds_dma16(dsrc, key * (HD * 2) + (((lane & 15) ^ swz_row(row)) << 4), dst + k * 1024);
    }
  };

  for (int half = 0; half < 2; ++half) {
    const int blk = half == 0 ? nblk - 1 - pair : pair;
    if (half == 1 && blk == nblk - 1 - pair) break;  // the middle block of an odd count, done once
    const int r0 = blk * 128;
    // the last node of the block and of this wave's tile: keys up to P + node are visible
    const int tmax_blk = min(T - 1, (min(r0 + 127, rows - 1)) / G);
    const int64_t nkeys = P + tmax_blk + 1;
    const int nsteps = (int)((nkeys + kRowsKeys - 1) / kRowsKeys);
    const int iters = (nsteps + 1) / 2;
    const int rt0 = r0 + 32 * tile;
    const bool tile_live = rt0 < rows;
    const int64_t tile_last_key = tile_live ? P + min(T - 1, min(rt0 + 31, rows - 1) / G) : -1;
    const int64_t tile_first_vis = P + (int64_t)(min(rt0, rows - 1) / G);  // keys <= this: every row sees them
    const int r = rt0 + ln;
    const int rr = min(r, rows - 1);
    const int t = rr / G;
    const int64_t kvis = P + t;  // this lane's row sees keys <= kvis
    // the row's Q^T operand: k-step j holds dims 16 j + 8 g .. + 7
    u32x4_t qf[8];
    {
      const uint16_t* qrow = q + ((int64_t)t * nh + kvh * G + rr % G) * HD + 8 * g;
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[j] = *(const u32x4_t*)(qrow + 16 * j);
    }
    f32x16_t o[4];
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[h][i] = 0.f;
    float m = kInitMax, l = 0.f;

    __syncthreads();  // the previous block's buffers and hand-over are read by every wave
    __builtin_amdgcn_s_waitcnt(0);  // Q has landed: no wait of the compiler's covers the ring's loads
    issue_pair(0);
    for (int it = 0; it < iters; ++it) {
      __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of iteration it have landed
      __syncthreads();                // everyone's have, and iteration it - 1's buffers are free
      if (it + 1 < iters) issue_pair(it + 1);
      const int step = 2 * it + kg;
      const int64_t kb0 = (int64_t)step * kRowsKeys;
      const uint8_t* kbp = smem + (2 * (it & 1) + kg) * kRowsStepBytes;
      const uint8_t* vbp = kbp + 16384;
      if (tile_live && step < nsteps && kb0 <= tile_last_key) {  // wave-uniform: the tile sees a key of this step
        f32x16_t sc[2];
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) sc[sb][i] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) {
            const u32x4_t kf = *(const u32x4_t*)(kbp + swz(32 * sb + ln, 2 * j + g));
            if constexpr (DT == PE_DTYPE_F16)
              sc[sb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, kf),
                                                              __builtin_bit_cast(f16x8_t, qf[j]), sc[sb], 0, 0, 0);
            else
              sc[sb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                               __builtin_bit_cast(bf16x8_t, qf[j]), sc[sb], 0, 0, 0);
          }
        // sc[sb][i] is key kb0 + 32 sb + 8 (i / 4) + 4 g + i % 4 of row r
        float bmax = -INFINITY;
        const bool whole = kb0 + kRowsKeys - 1 <= tile_first_vis;  // visible to every row of the tile
        const uint64_t win = causal_window(kb0, kvis) >> (4 * g);
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            if (!whole) sc[sb][i] = ((win >> (32 * sb + 8 * (i >> 2) + (i & 3))) & 1ull) ? sc[sb][i] : -INFINITY;
            bmax = fmaxf(bmax, sc[sb][i]);
          }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64)) * scale2;
        const float mnew = fmaxf(m, bmax);
        const float alpha = __builtin_amdgcn_exp2f(m - mnew);
        float psum = 0.f;
        uint32_t pb[2][8];
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[sb][i], scale2, -mnew));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[sb][i + 1], scale2, -mnew));
            psum += p0 + p1;
            pb[sb][i >> 1] = (DT == PE_DTYPE_F16)
                                 ? ((uint32_t)f32_to_f16_bits(p0) | ((uint32_t)f32_to_f16_bits(p1) << 16))
                                 : ((uint32_t)f32_to_bf16_bits(p0) | ((uint32_t)f32_to_bf16_bits(p1) << 16));
          }
        psum += __shfl_xor(psum, 32, 64);
        l = l * alpha + psum;
        const bool rescale = __builtin_amdgcn_ballot_w64(mnew != m) != 0ull;
        m = mnew;
        if (rescale) {
#pragma unroll
          for (int h = 0; h < 4; ++h)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[h][i] *= alpha;
        }
        // O^T += V^T P^T over the four 16-key quarters of the step
        const int qg = lane >> 4, jl = lane & 15;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int sb = c >> 1, cq = c & 1;
          u32x4_t bp;
          bp[0] = pb[sb][4 * cq + 0];
          bp[1] = pb[sb][4 * cq + 1];
          bp[2] = pb[sb][4 * cq + 2];
          bp[3] = pb[sb][4 * cq + 3];
          const int kb = 16 * c + 4 * (qg >> 1) + (jl >> 2);
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const int db = 32 * h + 16 * (qg & 1) + 4 * (jl & 3);
            typedef short s4v_t __attribute__((__vector_size__(4 * sizeof(short))));
            typedef __attribute__((address_space(3))) s4v_t lds_s4v_t;
            const s4v_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s4v_t*)(vbp + swz(kb, db >> 3) + (db & 7) * 2));
            const s4v_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s4v_t*)(vbp + swz(kb + 8, db >> 3) + (db & 7) * 2));
            const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
            u32x4_t a;
            a[0] = l2.x;
            a[1] = l2.y;
            a[2] = h2.x;
            a[3] = h2.y;
            if constexpr (DT == PE_DTYPE_F16)
              o[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                            __builtin_bit_cast(f16x8_t, bp), o[h], 0, 0, 0);
            else
              o[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                             __builtin_bit_cast(bf16x8_t, bp), o[h], 0, 0, 0);
          }
        }
      }
    }
    __syncthreads();  // every wave is done with the step buffers
    // group 1 hands (O, m, l) to group 0
    float* mo = (float*)smem + (tile * 64 + lane) * kRowsMergeStride;
    if (kg == 1) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *(f32x4_t*)&mo[16 * h + 4 * c] = f32x4_t{o[h][4 * c], o[h][4 * c + 1], o[h][4 * c + 2], o[h][4 * c + 3]};
      mo[64] = m;
      mo[65] = l;
    }
    __syncthreads();
    if (kg == 0 && tile_live && r < rows) {
      const float m1 = mo[64], l1 = mo[65];
      const float mx = fmaxf(m, m1);
      const float a0 = __builtin_amdgcn_exp2f(m - mx), a1 = __builtin_amdgcn_exp2f(m1 - mx);
      const float den = a0 * l + a1 * l1;
      // out = O / l: o[h][4 c .. 4 c + 3] are dims 32 h + 8 c + 4 g + 0..3 of row r
      const int col0 = (kvh * G + r % G) * HD;
      typedef typename Elem<DT>::T Te;
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4_t o1 = *(const f32x4_t*)&mo[16 * h + 4 * c];
          float o4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) o4[i] = (a0 * o[h][4 * c + i] + a1 * o1[i]) / den;
          const int col = col0 + 32 * h + 8 * c + 4 * g;
          if (out_units)
            Vec4<DT>::store((Te*)out + xtile_index(t, col, out_units), o4);
          else if ((ld_out & 3) || ((uintptr_t)out & 7)) {
#pragma unroll
            for (int i = 0; i < 4; ++i) Elem<DT>::store((Te*)out, (int64_t)t * ld_out + col + i, o4[i]);
          } else {
            Vec4<DT>::store((Te*)out + (int64_t)t * ld_out + col, o4);
          }
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Batched tree attention with many rows per KV head (GQA batches)
// ---------------------------------------------------------------------------
// Sequence b's rows of a KV head are its T_b nodes x G query heads (row r =
// node r / G, query head r % G): up to eight tiles of 32 rows, tile w on wave
// w of an eight-wave workgroup. One workgroup = (key split, KV head,
// sequence); the sequence's P_b + T_b keys are cut into splits of `kps` keys
// (a multiple of 64), so a sequence has ceil((P_b + T_b) / kps) splits, every
// workgroup walks the same number of keys, and those past a sequence's split
// count leave at once. A split's keys are walked in 64-key steps through a
// ring of four LDS step buffers filled by direct global-to-LDS loads
// (global_load_lds_dwordx4: no registers, three steps in flight while one is
// multiplied); each step is 32 loads of 1 KiB (wave w the four of K rows
// 16 (w % 4) .. + 15 for w < 4, of V rows for w >= 4), one wait for this
// wave's loads of the step and one barrier. K and V rows are stored unpadded
// (256 bytes), their 16-byte chunks permuted by row (chunk c of key row k at
// c ^ swz_row(k)), so that the K fragment and transposed V reads fall on
// distinct banks. The arithmetic is attn_rows_kernel's, with
// the tree mask as a bit window. A sequence of one split writes its output;
// otherwise each tile stores its split's (O, m, l) and attn_combine_kernel
// (a second launch, one thread per row and 4-dim chunk) merges the splits in
// split order. Sequences whose device prefix or row count exceed the bounds
// of the launch are skipped by every workgroup alike (the K/V offsets kernel
// reports them).
constexpr int kBRowsWaves = 8;
constexpr int kBRowsMinWaves = 4;  // fewer row tiles: attn_pair_kernel / attn_wg_kernel
constexpr int kBRowsStep = 32 * 1024;  // one step's K and V, 64 keys x 256 bytes each
constexpr int kBRowsRing = 4;          // step buffers; three steps in flight
// s_waitcnt with vmcnt = 8 (expcnt and lgkmcnt left at their maxima): this
// wave's loads of the two later steps in flight may still be outstanding
constexpr int kWaitVm8 = 0x0F78;

template <int DT>
__global__ __launch_bounds__(64 * kBRowsWaves, 1) void attn_batch_rows_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t cap,
    int nh, int nkv, const uint64_t* __restrict__ bits, int words, float scale, int kps, int max_splits,
    int rows_pad, float* __restrict__ opart, float* __restrict__ mlpart, void* __restrict__ out, int64_t ld_out,
    int out_units, AttnBatch bt) {
  constexpr int HD = 128;
  __shared__ __align__(1024) uint8_t smem[kBRowsRing * kBRowsStep];
  const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int rbase = bt.seq_row0[seq];
  const int T = bt.seq_row0[seq + 1] - rbase;
  const int64_t P = bt.seq_prefix[seq];
  if (T <= 0 || T > bt.max_rows || P < 0 || P > bt.max_prefix) return;
  const int G = nh / nkv, rows = T * G;
  const int64_t S = P + T;
  const int nsplit = (int)((S + kps - 1) / kps);
  if (split >= nsplit) return;
  const int64_t k0 = (int64_t)split * kps, k1 = min(S, k0 + kps);
  const int nsteps = (int)((k1 - k0 + kRowsKeys - 1) / kRowsKeys);
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int ln = lane & 31, g = lane >> 5;
  const float scale2 = scale * 1.44269504088896341f;
  const uint16_t* kvbase = uniform_ptr((wave < 4 ? kc : vc) + seq * bt.seq_stride + (int64_t)kvh * cap * HD);
  // this wave's four loads of a step: rows 16 (wave % 4) + 4 i + lane / 16, physical chunk lane % 16
  const int prow0 = 16 * (wave & 3) + (lane >> 4), pch = lane & 15;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  auto issue = [&](int step) {
    const int64_t kb0 = k0 + (int64_t)step * kRowsKeys;
    const uint32_t dst = __builtin_amdgcn_readfirstlane(
        lds_base + (step % kBRowsRing) * kBRowsStep + (wave >= 4 ? 16384 : 0) + (wave & 3) * 4096);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = prow0 + 4 * i;
      const uint32_t key = (uint32_t)min(kb0 + row, S - 1);
      lds_dma16(kvbase, key * (HD * 2) + ((pch ^ swz_row(row)) << 4), dst + i * 1024);
    }
  };

  const bool tile_live = wave * 32 < rows;
  const int r = wave * 32 + ln;
  const int rr = min(r, rows - 1);
  const int t = rr / G;
  uint64_t nbits[PE_TREE_MAX_WORDS];
  u32x4_t qf[8];
  if (tile_live) {
#pragma unroll
    for (int w = 0; w < PE_TREE_MAX_WORDS; ++w) nbits[w] = bits[(int64_t)(rbase + t) * words + min(w, words - 1)];
    const uint16_t* qrow = q + ((int64_t)(rbase + t) * nh + kvh * G + rr % G) * HD + 8 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) qf[j] = *(const u32x4_t*)(qrow + 16 * j);
  }
  f32x16_t o[4];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[h][i] = 0.f;
  float m = kInitMax, l = 0.f;

  // Q and the bits have landed before the ring starts, so no wait of the
  // compiler's for them covers the ring's loads; then three steps in flight
  // ahead of the one multiplied (past the split's end the loads repeat its
  // last key row into buffers nobody reads)
  __builtin_amdgcn_s_waitcnt(0);
  issue(0);
  issue(1);
  issue(2);
  for (int st = 0; st < nsteps; ++st) {
    __builtin_amdgcn_s_waitcnt(kWaitVm8);  // this wave's loads of step st have landed
    __syncthreads();
    issue(st + 3);
    const int64_t kb0 = k0 + (int64_t)st * kRowsKeys;
    const uint8_t* kb = smem + (st % kBRowsRing) * kBRowsStep;
    const uint8_t* vb = kb + 16384;
    if (tile_live) {
      f32x16_t sc[2];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) sc[sb][i] = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          const u32x4_t kf = *(const u32x4_t*)(kb + swz(32 * sb + ln, 2 * j + g));
          if constexpr (DT == PE_DTYPE_F16)
            sc[sb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, kf),
                                                            __builtin_bit_cast(f16x8_t, qf[j]), sc[sb], 0, 0, 0);
          else
            sc[sb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                             __builtin_bit_cast(bf16x8_t, qf[j]), sc[sb], 0, 0, 0);
        }
      // sc[sb][i] is key kb0 + 32 sb + 8 (i / 4) + 4 g + i % 4 of row r
      float bmax = -INFINITY;
      const bool whole = kb0 + kRowsKeys <= min(P, k1);  // prefix keys of the split only: visible to every row
      const uint64_t win = window_limit(tree_window(kb0, P, nbits), kb0, k1) >> (4 * g);
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (!whole) sc[sb][i] = ((win >> (32 * sb + 8 * (i >> 2) + (i & 3))) & 1ull) ? sc[sb][i] : -INFINITY;
          bmax = fmaxf(bmax, sc[sb][i]);
        }
      bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64)) * scale2;
      const float mnew = fmaxf(m, bmax);
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      float psum = 0.f;
      uint32_t pb[2][8];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[sb][i], scale2, -mnew));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[sb][i + 1], scale2, -mnew));
          psum += p0 + p1;
          pb[sb][i >> 1] = pack2_16<DT>(p0, p1);
        }
      psum += __shfl_xor(psum, 32, 64);
      l = l * alpha + psum;
      const bool rescale = __builtin_amdgcn_ballot_w64(mnew != m) != 0ull;
      m = mnew;
      if (rescale) {
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[h][i] *= alpha;
      }
      // O^T += V^T P^T; lane (qg, jl) reads 8 bytes of key row kbr, dims db .. db + 3
      const int qg = lane >> 4, jl = lane & 15;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int sb = c >> 1, cq = c & 1;
        u32x4_t bp;
        bp[0] = pb[sb][4 * cq + 0];
        bp[1] = pb[sb][4 * cq + 1];
        bp[2] = pb[sb][4 * cq + 2];
        bp[3] = pb[sb][4 * cq + 3];
        const int kbr = 16 * c + 4 * (qg >> 1) + (jl >> 2);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int db = 32 * h + 16 * (qg & 1) + 4 * (jl & 3);
          typedef short s4v_t __attribute__((__vector_size__(4 * sizeof(short))));
          typedef __attribute__((address_space(3))) s4v_t lds_s4v_t;
          const s4v_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s4v_t*)(vb + swz(kbr, db >> 3) + (db & 7) * 2));
          const s4v_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s4v_t*)(vb + swz(kbr + 8, db >> 3) + (db & 7) * 2));
          const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
          u32x4_t a;
          a[0] = l2.x;
          a[1] = l2.y;
          a[2] = h2.x;
          a[3] = h2.y;
          if constexpr (DT == PE_DTYPE_F16)
            o[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                          __builtin_bit_cast(f16x8_t, bp), o[h], 0, 0, 0);
          else
            o[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                           __builtin_bit_cast(bf16x8_t, bp), o[h], 0, 0, 0);
        }
      }
    }
  }
  // the ring's last loads land before the workgroup ends
  __builtin_amdgcn_s_waitcnt(0);
  if (!tile_live || r >= rows) return;
  typedef typename Elem<DT>::T Te;
  // o[h][4 c .. 4 c + 3] are dims 32 h + 8 c + 4 g + 0..3 of row r
  if (nsplit == 1) {
    const int col0 = (kvh * G + r % G) * HD;
    const int64_t orow = rbase + t;
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float o4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = o[h][4 * c + i] / l;
        const int col = col0 + 32 * h + 8 * c + 4 * g;
        if (out_units)
          Vec4<DT>::store((Te*)out + xtile_index((int)orow, col, out_units), o4);
        else if ((ld_out & 3) || ((uintptr_t)out & 7)) {
#pragma unroll
          for (int i = 0; i < 4; ++i) Elem<DT>::store((Te*)out, orow * ld_out + col + i, o4[i]);
        } else {
          Vec4<DT>::store((Te*)out + orow * ld_out + col, o4);
        }
      }
    return;
  }
  const int64_t prow = ((int64_t)(seq * nkv + kvh) * max_splits + split) * rows_pad + r;
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *(f32x4_t*)(opart + prow * HD + 32 * h + 8 * c + 4 * g) =
          f32x4_t{o[h][4 * c], o[h][4 * c + 1], o[h][4 * c + 2], o[h][4 * c + 3]};
  if (g == 0) *(float2*)(mlpart + prow * 2) = float2{m, l};
}

// The split merge of attn_batch_rows_kernel: one thread per (sequence, KV
// head, row, 4-dim chunk), every split's partial requested at once (up to
// eight per round), merged in split order (running max, rescaled sums).
template <int DT>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ opart,
                                                           const float* __restrict__ mlpart, int nh, int nkv,
                                                           int kps, int max_splits, int rows_pad,
                                                           void* __restrict__ out, int64_t ld_out, int out_units,
                                                           AttnBatch bt) {
  constexpr int HD = 128;
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int chunk = (int)(item & 31);
  const int64_t rowid = item >> 5;  // (seq * nkv + kvh) * rows_pad + row
  const int row = (int)(rowid % rows_pad);
  const int pair = (int)(rowid / rows_pad);
  if (pair >= bt.batch * nkv) return;
  const int seq = pair / nkv, kvh = pair - seq * nkv;
  const int rbase = bt.seq_row0[seq];
  const int T = bt.seq_row0[seq + 1] - rbase;
  const int64_t P = bt.seq_prefix[seq];
  if (T <= 0 || T > bt.max_rows || P < 0 || P > bt.max_prefix) return;
  const int G = nh / nkv;
  if (row >= T * G) return;
  const int nsplit = (int)((P + T + kps - 1) / kps);
  if (nsplit <= 1) return;
  float Mx = kInitMax, den = 0.f, num[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < nsplit; c0 += 8) {
    f32x4_t ov[8];
    float2 mv[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int sp = min(c0 + c, nsplit - 1);
      const int64_t prow = ((int64_t)pair * max_splits + sp) * rows_pad + row;
      ov[c] = *(const f32x4_t*)(opart + prow * HD + chunk * 4);
      mv[c] = *(const float2*)(mlpart + prow * 2);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (c0 + c >= nsplit) break;
      const float mn = fmaxf(Mx, mv[c].x);
      const float a = __builtin_amdgcn_exp2f(Mx - mn), wt = __builtin_amdgcn_exp2f(mv[c].x - mn);
      Mx = mn;
      den = den * a + wt * mv[c].y;
#pragma unroll
      for (int k = 0; k < 4; ++k) num[k] = num[k] * a + wt * ov[c][k];
    }
  }
  float o4[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) o4[k] = num[k] / den;
  typedef typename Elem<DT>::T Te;
  const int64_t orow = rbase + row / G;
  const int col = (kvh * G + row % G) * HD + chunk * 4;
  if (out_units)
    Vec4<DT>::store((Te*)out + xtile_index((int)orow, col, out_units), o4);
  else if ((ld_out & 3) || ((uintptr_t)out & 7)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) Elem<DT>::store((Te*)out, orow * ld_out + col + i, o4[i]);
  } else {
    Vec4<DT>::store((Te*)out + orow * ld_out + col, o4);
  }
}

}  // namespace

int64_t attention_workspace_bytes(int T, int nh, int nkv, int hd, int64_t kv_len, int dtype, int attn_mode) {
  if (T <= 0 || nh <= 0 || nkv <= 0 || kv_len <= 0) return 0;
  if (dtype != PE_DTYPE_F32 && hd == 128) {
    if (attn_mode == PE_ATTN_EAGER) return kAttnCounterBytes;  // attn_eager_kernel: no scratch
    AttnPlan p = attn_plan(T, nh, nkv, kv_len);
    return kAttnCounterBytes + p.opart_bytes + p.ml_bytes;
  }
  return (int64_t)T * nh * kv_len * 4;
}

extern "C" int64_t pe_attention_workspace_bytes(int T, int nh, int nkv, int hd, int64_t kv_len, int dtype) {
  return attention_workspace_bytes(T, nh, nkv, hd, kv_len, dtype, PE_ATTN_SDPA);
}

int pe_internal_tree_attention(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap, int nh,
                               int nkv, int hd, int T, int64_t P, int mask_mode, const uint64_t* bits, int words,
                               float scale, int dtype, void* out, int64_t ld_out, int out_units, void* workspace,
                               int64_t workspace_bytes, int* counters, hipStream_t st, int attn_mode) {
  if (!q || !k_cache || !v_cache || !out || !workspace) return PE_ERR_ARG;
  if (out_units && (dtype == PE_DTYPE_F32 || hd != 128 || out_units * 128 != nh * hd)) return PE_ERR_ARG;
  if (T <= 0 || nh <= 0 || nkv <= 0 || nh % nkv || hd <= 0 || hd > 256 || P < 0) return PE_ERR_ARG;
  if (P + T > cache_cap) return PE_ERR_CAPACITY;
  if (mask_mode != PE_MASK_TREE && mask_mode != PE_MASK_CAUSAL) return PE_ERR_ARG;
  if (mask_mode == PE_MASK_TREE && (!bits || words <= 0 || words > PE_TREE_MAX_WORDS || T > 64 * words))
    return PE_ERR_TREE;
  const int64_t S = P + T;
  if (attn_mode != PE_ATTN_SDPA && attn_mode != PE_ATTN_EAGER) return PE_ERR_ARG;
  const int eager = attn_mode == PE_ATTN_EAGER;
  if (eager && out_units) return PE_ERR_ARG;
  if (workspace_bytes < attention_workspace_bytes(T, nh, nkv, hd, S, dtype, attn_mode)) return PE_ERR_WORKSPACE;
  if (dtype != PE_DTYPE_F32 && hd == 128 && !eager && mask_mode == PE_MASK_CAUSAL && T >= kRowsMinNodes) {
    // many causal rows (a prefill): row blocks in balanced pairs, no key splits
    if (!(scale > 0.f) || cache_cap >= kAttnMaxCap) return PE_ERR_ARG;
    const int nblk = (T * (nh / nkv) + 127) / 128, npair = (nblk + 1) / 2;
    const dim3 grid(nkv * npair);
    if (dtype == PE_DTYPE_BF16)
      attn_rows_kernel<PE_DTYPE_BF16><<<grid, 64 * kRowsWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, T, P, scale,
          nblk, npair, out, ld_out, out_units);
    else if (dtype == PE_DTYPE_F16)
      attn_rows_kernel<PE_DTYPE_F16><<<grid, 64 * kRowsWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, T, P, scale,
          nblk, npair, out, ld_out, out_units);
    else
      return PE_ERR_ARG;
    PE_CHECK_LAUNCH();
    return PE_OK;
  }
  if (dtype != PE_DTYPE_F32 && hd == 128 && !eager) {
    if (!(scale > 0.f) || cache_cap >= kAttnMaxCap) return PE_ERR_ARG;
    AttnPlan p = attn_plan(T, nh, nkv, S);
    if (p.splits > 1 && (int64_t)nkv * p.row_tiles * 4 > kAttnCounterBytes) return PE_ERR_ARG;
    if (!counters) counters = (int*)workspace;
    float* opart = (float*)((char*)workspace + kAttnCounterBytes);
    float* ml = (float*)((char*)workspace + kAttnCounterBytes + p.opart_bytes);
    dim3 grid(nkv, p.splits, p.row_tiles);
    if (dtype == PE_DTYPE_BF16) {
      attn_wg_kernel<PE_DTYPE_BF16><<<grid, 64 * kAttnWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, T, P, mask_mode,
          bits, words, scale, p.keys_per_split, p.splits, p.rows_pad, opart, ml, counters, out, ld_out, out_units,
          AttnBatch{0, 0, nullptr, nullptr, 0, 0, 0, 0});
    } else if (dtype == PE_DTYPE_F16) {
      attn_wg_kernel<PE_DTYPE_F16><<<grid, 64 * kAttnWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, T, P, mask_mode,
          bits, words, scale, p.keys_per_split, p.splits, p.rows_pad, opart, ml, counters, out, ld_out, out_units,
          AttnBatch{0, 0, nullptr, nullptr, 0, 0, 0, 0});
    } else {
      return PE_ERR_ARG;
    }
    PE_CHECK_LAUNCH();
    return PE_OK;
  }
  if (eager && dtype != PE_DTYPE_F32 && hd == 128) {
    // the matrix-core eager kernel: every key of a row tile in one workgroup
    if (cache_cap >= kAttnMaxCap) return PE_ERR_ARG;
    const dim3 grid(nkv, 1, (T * (nh / nkv) + 31) / 32);
    if (dtype == PE_DTYPE_BF16)
      attn_eager_kernel<PE_DTYPE_BF16><<<grid, 64 * kAttnWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, T, P,
          mask_mode, bits, words, out, ld_out);
    else
      attn_eager_kernel<PE_DTYPE_F16><<<grid, 64 * kAttnWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, T, P,
          mask_mode, bits, words, out, ld_out);
    PE_CHECK_LAUNCH();
    return PE_OK;
  }
  dim3 grid(T, nh);
  float* scores = (float*)workspace;
  switch (dtype) {
    case PE_DTYPE_F32:
      attn_generic_kernel<PE_DTYPE_F32><<<grid, 128, 0, st>>>((const float*)q, (const float*)k_cache,
                                                              (const float*)v_cache, cache_cap, nh, nkv, hd, T, P,
                                                              mask_mode, bits, words, scale, eager, (float*)out,
                                                              ld_out, scores);
      break;
    case PE_DTYPE_BF16:
      attn_generic_kernel<PE_DTYPE_BF16><<<grid, 128, 0, st>>>((const uint16_t*)q, (const uint16_t*)k_cache,
                                                               (const uint16_t*)v_cache, cache_cap, nh, nkv, hd, T,
                                                               P, mask_mode, bits, words, scale, eager,
                                                               (uint16_t*)out, ld_out, scores);
      break;
    case PE_DTYPE_F16:
      attn_generic_kernel<PE_DTYPE_F16><<<grid, 128, 0, st>>>((const uint16_t*)q, (const uint16_t*)k_cache,
                                                              (const uint16_t*)v_cache, cache_cap, nh, nkv, hd, T, P,
                                                              mask_mode, bits, words, scale, eager,
                                                              (uint16_t*)out, ld_out, scores);
      break;
    default:
      return PE_ERR_ARG;
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}

// attn_batch_rows_kernel's plan: keys per split a multiple of 64, sized so
// that a batch whose prefixes average half the longest fills about two
// workgroups per CU's worth of splits; sequences take as many splits as their
// own keys need.
struct BRowsPlan {
  bool use;
  int waves, kps, max_splits, rows_pad;
  int64_t opart_bytes, ml_bytes;
};

BRowsPlan brows_plan(int max_rows, int nh, int nkv, int64_t max_kv_len, int batch) {
  BRowsPlan p{};
  const int rows = max_rows * (nh / nkv);
  p.waves = (rows + 31) / 32;
  // opt-in (PE_ATTN_BATCH_ROWS=1): at the batched workload the kernel matches
  // attn_pair_kernel (39.2 against 39.1 us per launch) but its split combine
  // (a second launch, 8.2 us) and a partly filled second round of workgroups
  // leave the pass 0.3 ms slower
  static const bool enabled = [] {
    const char* v = getenv("PE_ATTN_BATCH_ROWS");
    return v && v[0] == '1';
  }();
  p.use = enabled && p.waves >= kBRowsMinWaves && p.waves <= kBRowsWaves;
  if (!p.use) return p;
  int64_t want = (512 + (int64_t)batch * nkv - 1) / ((int64_t)batch * nkv);
  want = want < 1 ? 1 : (want > 16 ? 16 : want);
  int64_t kps = (max_kv_len + want - 1) / want;
  kps = ((kps + kRowsKeys - 1) / kRowsKeys) * kRowsKeys;
  if (kps < kRowsKeys) kps = kRowsKeys;
  p.kps = (int)kps;
  p.max_splits = (int)((max_kv_len + kps - 1) / kps);
  p.rows_pad = p.waves * 32;
  p.opart_bytes = (int64_t)batch * nkv * p.max_splits * p.rows_pad * 128 * 4;
  p.ml_bytes = (int64_t)batch * nkv * p.max_splits * p.rows_pad * 2 * 4;
  return p;
}

int64_t pe_internal_attention_batch_bytes(int max_rows, int nh, int nkv, int64_t max_kv_len, int batch) {
  const AttnPlan p = attn_plan(max_rows, nh, nkv, max_kv_len, batch);
  const BRowsPlan r = brows_plan(max_rows, nh, nkv, max_kv_len, batch);
  const int64_t a = p.opart_bytes + p.ml_bytes, b = r.use ? r.opart_bytes + r.ml_bytes : 0;
  return kAttnCounterBytes + (a > b ? a : b);
}

int pe_internal_tree_attention_batch(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap,
                                     int64_t seq_stride, int nh, int nkv, int max_rows, int64_t max_prefix, int batch,
                                     const int32_t* seq_row0, const int64_t* seq_prefix, const uint64_t* bits,
                                     int words, float scale, int dtype, void* out, int64_t ld_out, int out_units,
                                     void* workspace, int64_t workspace_bytes, int* counters, hipStream_t st,
                                     int dyn_split) {
  if (!q || !k_cache || !v_cache || !out || !workspace || !seq_row0 || !seq_prefix || !bits) return PE_ERR_ARG;
  if (dtype == PE_DTYPE_F32 || batch <= 0 || max_rows <= 0 || nh <= 0 || nkv <= 0 || nh % nkv || max_prefix < 0)
    return PE_ERR_ARG;
  if (!(scale > 0.f) || cache_cap >= kAttnMaxCap) return PE_ERR_ARG;
  if (out_units && out_units * 128 != nh * 128) return PE_ERR_ARG;
  if (max_prefix + max_rows > cache_cap) return PE_ERR_CAPACITY;
  if (words <= 0 || words > PE_TREE_MAX_WORDS || max_rows > 64 * words) return PE_ERR_TREE;
  const int64_t S = max_prefix + max_rows;
  if (workspace_bytes < pe_internal_attention_batch_bytes(max_rows, nh, nkv, S, batch)) return PE_ERR_WORKSPACE;
  const AttnPlan p = attn_plan(max_rows, nh, nkv, S, batch);
  if (p.splits > 1 && (int64_t)batch * nkv * p.row_tiles * 4 > kAttnCounterBytes) return PE_ERR_ARG;
  if (!counters) counters = (int*)workspace;
  float* opart = (float*)((char*)workspace + kAttnCounterBytes);
  float* ml = (float*)((char*)workspace + kAttnCounterBytes + p.opart_bytes);
  const AttnBatch bt{batch, p.row_tiles, seq_row0, seq_prefix, seq_stride, max_prefix, max_rows, dyn_split};
  const BRowsPlan rp = brows_plan(max_rows, nh, nkv, S, batch);
  if (rp.use) {
    // K/V of a step staged once per workgroup for every row tile of the (sequence, KV head)
    float* op = (float*)((char*)workspace + kAttnCounterBytes);
    float* mp = (float*)((char*)workspace + kAttnCounterBytes + rp.opart_bytes);
    const dim3 gridr(rp.max_splits, nkv, batch);
    const int64_t items = (int64_t)batch * nkv * rp.rows_pad * 32;
    const dim3 gridc((unsigned)((items + 255) / 256));
    if (dtype == PE_DTYPE_BF16) {
      attn_batch_rows_kernel<PE_DTYPE_BF16><<<gridr, 64 * kBRowsWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, bits, words,
          scale, rp.kps, rp.max_splits, rp.rows_pad, op, mp, out, ld_out, out_units, bt);
      if (rp.max_splits > 1)
        attn_combine_kernel<PE_DTYPE_BF16><<<gridc, 256, 0, st>>>(op, mp, nh, nkv, rp.kps, rp.max_splits, rp.rows_pad,
                                                                  out, ld_out, out_units, bt);
    } else {
      attn_batch_rows_kernel<PE_DTYPE_F16><<<gridr, 64 * kBRowsWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, bits, words,
          scale, rp.kps, rp.max_splits, rp.rows_pad, op, mp, out, ld_out, out_units, bt);
      if (rp.max_splits > 1)
        attn_combine_kernel<PE_DTYPE_F16><<<gridc, 256, 0, st>>>(op, mp, nh, nkv, rp.kps, rp.max_splits, rp.rows_pad,
                                                                 out, ld_out, out_units, bt);
    }
    PE_CHECK_LAUNCH();
    return PE_OK;
  }
  const int tpairs = (p.row_tiles + 1) / 2;
  if (p.row_tiles >= 2 && (int64_t)batch * nkv * tpairs >= 128) {
    // two row tiles per wave: each K/V block read once for both
    const dim3 gridp(nkv, 1, batch * tpairs);
    if (dtype == PE_DTYPE_BF16)
      attn_pair_kernel<PE_DTYPE_BF16><<<gridp, 64 * kPairWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, bits, words,
          scale, out, ld_out, out_units, bt);
    else
      attn_pair_kernel<PE_DTYPE_F16><<<gridp, 64 * kPairWaves, 0, st>>>(
          (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, bits, words,
          scale, out, ld_out, out_units, bt);
    PE_CHECK_LAUNCH();
    return PE_OK;
  }
  const dim3 grid(nkv, p.splits, batch * p.row_tiles);
  if (dtype == PE_DTYPE_BF16)
    attn_wg_kernel<PE_DTYPE_BF16><<<grid, 64 * kAttnWaves, 0, st>>>(
        (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, max_rows,
        max_prefix, PE_MASK_TREE, bits, words, scale, p.keys_per_split, p.splits, p.rows_pad, opart, ml, counters,
        out, ld_out, out_units, bt);
  else
    attn_wg_kernel<PE_DTYPE_F16><<<grid, 64 * kAttnWaves, 0, st>>>(
        (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, cache_cap, nh, nkv, max_rows,
        max_prefix, PE_MASK_TREE, bits, words, scale, p.keys_per_split, p.splits, p.rows_pad, opart, ml, counters,
        out, ld_out, out_units, bt);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

extern "C" int64_t pe_attention_batch_workspace_bytes(int max_rows, int nh, int nkv, int64_t max_kv_len,
                                                      int batch) {
  if (max_rows <= 0 || nh <= 0 || nkv <= 0 || nh % nkv || batch <= 0 || max_kv_len <= 0) return 0;
  return pe_internal_attention_batch_bytes(max_rows, nh, nkv, max_kv_len, batch);
}

extern "C" int pe_tree_attention_batch(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap,
                                       int64_t seq_stride, int nh, int nkv, int max_rows, int64_t max_prefix,
                                       int batch, const int32_t* seq_row0, const int64_t* seq_prefix,
                                       const uint64_t* bits, int words, float scale, int dtype, void* out,
                                       int64_t ld_out, void* workspace, int64_t workspace_bytes, void* stream) {
  if (ld_out < (int64_t)nh * 128 || seq_stride < 0) return PE_ERR_ARG;
  return pe_internal_tree_attention_batch(q, k_cache, v_cache, cache_cap, seq_stride, nh, nkv, max_rows, max_prefix,
                                          batch, seq_row0, seq_prefix, bits, words, scale, dtype, out, ld_out, 0,
                                          workspace, workspace_bytes, nullptr, (hipStream_t)stream, 0);
}

extern "C" int pe_tree_attention(const void* q, const void* k_cache, const void* v_cache, int64_t cache_cap, int nh,
                                 int nkv, int hd, int T, int64_t P, int mask_mode, const uint64_t* bits, int words,
                                 float scale, int dtype, void* out, int64_t ld_out, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  return pe_internal_tree_attention(q, k_cache, v_cache, cache_cap, nh, nkv, hd, T, P, mask_mode, bits, words, scale,
                                    dtype, out, ld_out, 0, workspace, workspace_bytes, nullptr, (hipStream_t)stream,
                                    PE_ATTN_SDPA);
}
