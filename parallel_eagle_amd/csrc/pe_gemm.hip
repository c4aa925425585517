// Linear layers of the verification pass: Y[M][N] = X[M][K] . W^T, fp32 accumulate.
//
// The tree block is small (M = T = 26 rows at the 7B shape) and the weights are
// large, so every linear is bound by streaming W from HBM once and, for NF4, by
// the per-weight dequantisation that goes with it. The MFMA kernels:
//   * stream W in the tiled layouts of pe_format.hip: each wave load
//     instruction reads 1 KiB contiguous;
//   * use v_mfma_f32_32x32x16_{bf16,f16} with X as the A operand (32 rows per
//     M tile) and the weights as the B operand (32 columns per tile); a wave
//     owns NT = 2 column tiles, so every X fragment feeds two MFMAs;
//   * keep the next iteration's weights in flight in a second register set
//     while computing the current one, and fetch each X fragment of the next
//     iteration right after the MFMA that used the current one; the loop body
//     is straight-line (loads past the wave's range are clamped and their
//     contribution zeroed) so the compiler's wait counts never fall back to
//     waiting for the prefetch;
//   * split K across the 4 waves of a workgroup (summed in LDS in wave order)
//     and across S workgroups, with S chosen so that every launch has about
//     three 4-wave workgroups per CU. The S workgroups of a column group write
//     fp32 partials with agent-coherent stores, count themselves on a
//     per-group counter, and the last one to arrive sums the partials in split
//     order and applies the epilogue. Nobody waits for anybody: no spin loop,
//     no grid barrier, no device-scope cache write-back. Results are
//     deterministic (split order, then wave order) whatever the arrival order.
//
// NF4 dequantisation (bitsandbytes' dequantize_4bit, src/pe/target.py:55-62):
// in the tiled layout each lane owns one 64-element absmax block of one column
// per block pair, so it builds its own 16-entry table bf16_rne(NF4[c] *
// float(absmax)) in LDS and looks every code up there: the MFMA consumes
// exactly the bf16 weights the reference feeds its GEMM. Per lookup:
//   * one SDWA v_and/v_lshrrev writes the 4-bit code into bits 8..11 of an
//     address register that keeps the lane's table base (lane * 4) in its low
//     byte (dst_sel:BYTE_1, dst_unused:UNUSED_PRESERVE);
//   * one ds_read_u16 loads the bf16 weight; pairs are packed into the MFMA
//     operand with one v_lshl_or.
// Entry c of lane l sits at byte 256 c + 4 l of its tile's 4 KiB table, so the
// 32 lanes of a half-wave hit 32 distinct banks whatever the codes; the two
// 16-bit halves of each dword are the table slots of alternating block pairs.
// The per-wave and per-tile table offsets are instruction immediates, which is
// why the NF4 kernel body is instantiated once per wave index.

#include "pe_common.h"
#include "pe_internal.h"

#include <cstdlib>
#include <type_traits>

namespace {

// Internal epilogues: the q/k/v projection with bias, RoPE and the in-place KV
// append; and raw fp32 split partials, out[split][row][col] (ld = N), summed
// by the kernel that consumes them.
constexpr int kEpiRopeKV = 4;
constexpr int kEpiPartial = 5;
// PE_EPI_STORE plus, per row and column group, the argmax key of the group's
// stored values (amax_keys[row * amax_groups + group], arg_key64)
constexpr int kEpiArgmax = 6;

struct EpiArgs {
  int op;
  int M;
  int N;  // GEMM columns
  const void* bias;
  const void* resid;
  int64_t ld_resid;
  void* out;
  int64_t ld_out;
  int out_units;  // > 0: out is A-tiled with K = 128 * out_units (SwiGLU / store epilogues)
  // kEpiRopeKV: the q/k/v projection whose weight rows are in head-paired tile
  // order (see write_rope_kv); RoPE at positions[row], q to q_out [M][nh][hd],
  // k and v appended to the caches at rows row0 + row.
  const int64_t* positions;
  const void* cos_sin;  // [max_pos][hd] cos, then [max_pos][hd] sin
  int64_t max_pos;
  void* q_out;
  void* k_cache;
  void* v_cache;
  int64_t cap;
  int64_t row0;
  // batched passes: element offset of row `row`'s K/V slot in the caches
  // (sequence base + (prefix + local row) * hd; head h adds h * cap * hd), a
  // negative entry drops the row's K/V; null: rows row0 + row of one cache
  const int64_t* kv_off;
  int nh, nkv, hd;
  int32_t* status;
  uint64_t* amax_keys;  // kEpiArgmax: [M][amax_groups]
  int amax_groups;
};

__device__ __forceinline__ int64_t kv_row_elem(const EpiArgs& e, int row) {
  return e.kv_off ? e.kv_off[row] : (e.row0 + row) * (int64_t)e.hd;
}

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
    E::store(out, e.out_units ? xtile_index(row, col, e.out_units) : (int64_t)row * e.ld_out + col, v);
  }
}

template <int DT>
__device__ __forceinline__ void epi_swiglu(const EpiArgs& e, int row, int col, float gv, float uv) {
  typedef Elem<DT> E;
  float gr = E::round(gv), ur = E::round(uv);
  float s = E::round(silu_f(gr));
  E::store((typename E::T*)e.out, e.out_units ? xtile_index(row, col, e.out_units) : (int64_t)row * e.ld_out + col,
           __fmul_rn(s, ur));
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

// q/k/v projection epilogue (HF apply_rotary_pos_emb, modeling_llama.py:130-160,
// and the KV append of DynamicLayer.update, cache_utils.py:127-146). The
// weight rows are permuted at load time so that column group `group` holds,
// in its two tiles, dims [32 j, 32 j + 32) and [hd/2 + 32 j, hd/2 + 32 j + 32)
// of one head unit u (units: nh q heads, then nkv k heads, then nkv v heads;
// j = group % (hd / 64)). The two halves a RoPE pair needs are therefore in
// the same lane: o1 = r(r(x1 cos1) + r(-x2 sin1)), o2 = r(r(x2 cos2) + r(x1 sin2)).
// c1, s1, c2, s2: cos / sin at dims d1, d2 of position p (read by the caller;
// unused for v and for an out-of-range p).
template <int DT>
__device__ __forceinline__ void write_rope_kv_core(const EpiArgs& e, int group, int ln, int row, float a1, float a2,
                                                   int64_t p, float c1, float s1, float c2, float s2) {
  typedef Elem<DT> E;
  typedef typename E::T T;
  const int gpu = e.hd >> 6;  // column groups per head unit
  const int u = group / gpu, j = group % gpu;
  const int d1 = 32 * j + ln, d2 = d1 + (e.hd >> 1);
  float x1 = a1, x2 = a2;
  if (e.bias) {
    x1 = __fadd_rn(x1, E::load((const T*)e.bias, u * e.hd + d1));
    x2 = __fadd_rn(x2, E::load((const T*)e.bias, u * e.hd + d2));
  }
  x1 = E::round(x1);
  x2 = E::round(x2);
  const int64_t kvo = u >= e.nh ? kv_row_elem(e, row) : 0;
  if (kvo < 0) return;
  if (u >= e.nh + e.nkv) {  // v: appended as is
    T* dst = (T*)e.v_cache + (int64_t)(u - e.nh - e.nkv) * e.cap * e.hd + kvo;
    E::store(dst, d1, x1);
    E::store(dst, d2, x2);
    return;
  }
  if (p < 0 || p >= e.max_pos) {
    if (e.status) atomicOr(e.status, PE_ERR_CAPACITY);
    return;
  }
  const float o1 = __fadd_rn(E::round(__fmul_rn(x1, c1)), E::round(__fmul_rn(-x2, s1)));
  const float o2 = __fadd_rn(E::round(__fmul_rn(x2, c2)), E::round(__fmul_rn(x1, s2)));
  T* dst = (u < e.nh) ? (T*)e.q_out + ((int64_t)row * e.nh + u) * e.hd
                      : (T*)e.k_cache + (int64_t)(u - e.nh) * e.cap * e.hd + kvo;
  E::store(dst, d1, o1);
  E::store(dst, d2, o2);
}

// cos / sin of position p at dims d1, d2 (zeros for v heads or p out of range).
template <int DT>
__device__ __forceinline__ void rope_fetch(const EpiArgs& e, int group, int ln, int64_t p, float& c1, float& s1,
                                           float& c2, float& s2) {
  typedef Elem<DT> E;
  typedef typename E::T T;
  const int gpu = e.hd >> 6;
  const int u = group / gpu, j = group % gpu;
  c1 = s1 = c2 = s2 = 0.f;
  if (u >= e.nh + e.nkv || p < 0 || p >= e.max_pos) return;
  const int d1 = 32 * j + ln, d2 = d1 + (e.hd >> 1);
  const T* cosr = (const T*)e.cos_sin + p * e.hd;
  const T* sinr = (const T*)e.cos_sin + (e.max_pos + p) * e.hd;
  c1 = E::load(cosr, d1);
  s1 = E::load(sinr, d1);
  c2 = E::load(cosr, d2);
  s2 = E::load(sinr, d2);
}

template <int DT>
__device__ __forceinline__ void write_rope_kv(const EpiArgs& e, int group, int ln, int row, float a1, float a2) {
  const int gpu = e.hd >> 6;
  const bool v = group / gpu >= e.nh + e.nkv;
  const int64_t p = v ? 0 : e.positions[row];
  float c1, s1, c2, s2;
  rope_fetch<DT>(e, group, ln, p, c1, s1, c2, s2);
  write_rope_kv_core<DT>(e, group, ln, row, a1, a2, p, c1, s1, c2, s2);
}

// RoPE epilogue operands of a wave's output rows (rows 8 w + 4 g + j of each
// M tile), fetched while the GEMM runs: positions at kernel start, cos / sin
// once the wave's first loads are issued.
template <int MT>
struct RopePre {
  int64_t pos[MT][4];
  float c1[MT][4], s1[MT][4], c2[MT][4], s2[MT][4];
};


// ---------------------------------------------------------------------------
// NF4 lookup primitives
// ---------------------------------------------------------------------------
// Addresses (gfx950 assembly): the 8 codes of dword q go to bits 8..11 of 8
// address registers whose low byte holds the lane's table base (lane * 4).
// The table reads themselves are ordinary LDS loads the compiler schedules
// and counts: plain zero-extending ds_read_u16 (with SRAM ECC enabled, the
// MI355X default, d16 loads clear the other half of the register instead of
// preserving it), joined in pairs with one v_lshl_or.
#define PE_SDWA_LO(a, q, byte) \
  "v_and_b32_sdwa " a ", 15, " q " dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_" byte "\n\t"
#define PE_SDWA_HI(a, q, byte) \
  "v_lshrrev_b32_sdwa " a ", 4, " q " dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_" byte "\n\t"
#define PE_ADDR8(A, Q)                                                                                    \
  PE_SDWA_LO("%[" A "0]", "%[" Q "]", "0") PE_SDWA_HI("%[" A "1]", "%[" Q "]", "0")                     \
  PE_SDWA_LO("%[" A "2]", "%[" Q "]", "1") PE_SDWA_HI("%[" A "3]", "%[" Q "]", "1")                     \
  PE_SDWA_LO("%[" A "4]", "%[" Q "]", "2") PE_SDWA_HI("%[" A "5]", "%[" Q "]", "2")                     \
  PE_SDWA_LO("%[" A "6]", "%[" Q "]", "3") PE_SDWA_HI("%[" A "7]", "%[" Q "]", "3")

__device__ __forceinline__ void nf4_addr8(uint32_t q, uint32_t (&a)[8]) {
  asm(PE_ADDR8("a", "q")
      : [a0] "+v"(a[0]), [a1] "+v"(a[1]), [a2] "+v"(a[2]), [a3] "+v"(a[3]), [a4] "+v"(a[4]), [a5] "+v"(a[5]),
        [a6] "+v"(a[6]), [a7] "+v"(a[7])
      : [q] "v"(q));
}
#undef PE_ADDR8
#undef PE_SDWA_HI
#undef PE_SDWA_LO

// The table is written as dwords (two 16-bit slots) and read as 16-bit
// entries: the read type is may_alias (and the library is built with
// -fno-strict-aliasing), and the address is formed from the kernel's LDS
// array itself (smem + the address register + OFF), not from a bare integer.
// Otherwise the compiler may take the reads as independent of the table
// builds and move the next build's stores above reads of the current table.
typedef __attribute__((address_space(3), may_alias)) const uint16_t lds_u16_t;
typedef __attribute__((address_space(3))) const uint8_t lds_u8_t;

template <int OFF>
__device__ __forceinline__ void nf4_read8(const uint8_t* smem, const uint32_t (&a)[8], uint32_t (&r)[8]) {
  const lds_u8_t* base = (const lds_u8_t*)smem;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = *(lds_u16_t*)(base + a[i] + OFF);
}

__device__ __forceinline__ uint32_t pack16(uint32_t lo, uint32_t hi) { return lo | (hi << 16); }

// The lane's 16 table entries for two block pairs at once: entry c (at lane
// base + 256 c + OFF) holds bf16_rne(NF4[c] * scale0) in its low half and
// bf16_rne(NF4[c] * scale1) in its high half.
template <int OFF, bool AF>
__device__ __forceinline__ void nf4_build_table2(uint8_t* lanetab, uint32_t absmax0, uint32_t absmax1) {
  // AF: fp32 absmax (bitsandbytes' own), else fp16
  const float s0 = AF ? __uint_as_float(absmax0) : f16_bits_to_f32((uint16_t)absmax0);
  const float s1 = AF ? __uint_as_float(absmax1) : f16_bits_to_f32((uint16_t)absmax1);
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const f32x2_t v = {kNF4[c] * s0, kNF4[c] * s1};
    *(uint32_t*)(lanetab + c * 256 + OFF) = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  }
}

constexpr int kTabTile = 16 * 64 * 4;  // one tile's table: 16 codes x 64 lanes x dword (2 slots)

// Workgroup barrier that orders LDS accesses only: global loads still in
// flight (prefetches past the last unit) are not waited for.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}


// ---------------------------------------------------------------------------
// Workgroup output
// ---------------------------------------------------------------------------
constexpr int kWaves = 4;             // waves per GEMM workgroup (K slices)
constexpr int kCounterBytes = 32768;  // per-column-group arrival counters at the head of the workspace
constexpr int kMaxGroups = kGemmCounterInts;  // the rest of the counter area belongs to attention
constexpr int kMaxSplits = 16;

// Epilogue of one output row of a column group: v[nt] is the lane's column of
// tile nt (SwiGLU and RoPE pair tile 0 with tile 1 in the same lane).
template <int ADT, int NT>
__device__ __forceinline__ void epilogue_row(const EpiArgs& e, int group, int row, int ln, const float (&v)[NT]) {
  if (e.op == PE_EPI_SWIGLU) {
    if constexpr (NT == 2) epi_swiglu<ADT>(e, row, group * 32 + ln, v[0], v[1]);
  } else if (e.op == kEpiRopeKV) {
    if constexpr (NT == 2) write_rope_kv<ADT>(e, group, ln, row, v[0], v[1]);
  } else {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) epi_value<ADT>(e, row, (group * NT + nt) * 32 + ln, v[nt]);
  }
}

// Bytes of split-K partials of one launch: per split and column group, every
// wave stores its row quad of each (M tile, column tile) as 64 lanes x 4 floats.
__host__ __device__ constexpr int64_t partial_bytes_of(int S, int groups, int MT, int NT) {
  return S > 1 ? (int64_t)S * groups * MT * NT * kWaves * 64 * 16 : 0;
}

// The KW waves' K slices summed in LDS (wave order); wave w < 4 then owns rows
// 8 w + 4 g + j (j < 4) of every M tile. With S > 1 the workgroup publishes
// its sums as split `split` of the group's partials and the last workgroup of
// the group to arrive sums all S of them in split order. The caller has
// synchronised the workgroup if `red` had another use.
// LDS of the reduction: per (wave, tile, M tile) 64 lanes x kRedLane floats,
// the lane's 16 accumulators at a 20-float (80-byte) stride, so 16-byte
// accesses of 16 consecutive lanes hit 64 distinct banks.
constexpr int kRedLane = 20;
__host__ __device__ constexpr int red_floats(int KW, int NT, int MT) { return KW * NT * MT * 64 * kRedLane; }

template <int ADT, int NT, int MT, int KW = kWaves>
__device__ __forceinline__ void finish_tile(f32x16_t (&acc)[NT][MT], float* red, int group, int split, int S,
                                            float* __restrict__ partial, int* __restrict__ counters,
                                            const EpiArgs& e, const RopePre<MT>* rp = nullptr,
                                            bool use_rp = false) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 5, ln = lane & 31;
  auto slot = [&](int w, int nt, int mt) -> f32x4_t* {
    return (f32x4_t*)(red + ((((w * NT + nt) * MT + mt) * 64) + lane) * kRedLane);
  };
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        slot(wave, nt, mt)[q] = f32x4_t{acc[nt][mt][4 * q], acc[nt][mt][4 * q + 1], acc[nt][mt][4 * q + 2],
                                        acc[nt][mt][4 * q + 3]};
  lds_barrier();
  if (KW > kWaves && wave >= kWaves) return;
  float v[MT][4][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < KW; ++w) {
        const f32x4_t t = slot(w, nt, mt)[wave];
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] += t[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) v[mt][j][nt] = s[j];
    }

  if (e.op == kEpiPartial) {
    float* out = (float*)e.out + (int64_t)split * e.M * e.N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = mt * 32 + 8 * wave + 4 * g + j;
        if (row < e.M)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) out[(int64_t)row * e.N + (group * NT + nt) * 32 + ln] = v[mt][j][nt];
      }
    return;
  }
  if (S > 1) {
    const int groups = e.N / (32 * NT);
    // partial[split][group][mt][nt][wave][lane][4], agent-coherent 16-byte accesses
    const __amdgpu_buffer_rsrc_t rp = agent_rsrc(partial, (uint32_t)partial_bytes_of(S, groups, MT, NT));
    auto slot = [&](int sp, int mt, int nt) -> uint32_t {
      return (uint32_t)((((((int64_t)sp * groups + group) * MT + mt) * NT + nt) * kWaves + wave) * 64 + lane) * 16;
    };
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        store_agent_x4(rp, slot(split, mt, nt), f32x4_t{v[mt][0][nt], v[mt][1][nt], v[mt][2][nt], v[mt][3][nt]});
    // the stores are acknowledged at agent scope before this workgroup counts itself
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int* flag = (int*)red;
    if (threadIdx.x == 0)
      flag[0] = __hip_atomic_fetch_add(counters + group, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (flag[0] != S - 1) return;
    if (threadIdx.x == 0) __hip_atomic_store(counters + group, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float sum[MT][4][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) sum[mt][j][nt] = 0.f;
    // up to 8 splits' loads in flight at a time, summed in split order
    for (int c0 = 0; c0 < S; c0 += 8) {
      f32x4_t got[8][MT][NT];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int sp = c0 + c;
        if (sp < S && sp != split) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) got[c][mt][nt] = load_agent_x4(rp, slot(sp, mt, nt));
        }
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int sp = c0 + c;
        if (sp >= S) break;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int j = 0; j < 4; ++j) sum[mt][j][nt] += (sp == split) ? v[mt][j][nt] : got[c][mt][nt][j];
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) v[mt][j][nt] = sum[mt][j][nt];
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = mt * 32 + 8 * wave + 4 * g + j;
      if (row >= e.M) continue;
      if constexpr (NT == 2) {
        if (use_rp && e.op == kEpiRopeKV) {
          write_rope_kv_core<ADT>(e, group, ln, row, v[mt][j][0], v[mt][j][1], rp->pos[mt][j], rp->c1[mt][j],
                                  rp->s1[mt][j], rp->c2[mt][j], rp->s2[mt][j]);
          continue;
        }
      }
      epilogue_row<ADT, NT>(e, group, row, ln, v[mt][j]);
    }
  if (e.op == kEpiArgmax) {
    // the group's largest stored value of each row: the lane's NT columns, then
    // the 32 lanes of its half-wave (the row's 32 * NT columns)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint64_t best = 0;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const uint64_t k = arg_key64(Elem<ADT>::round(v[mt][j][nt]), (group * NT + nt) * 32 + ln);
          best = k > best ? k : best;
        }
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
          const uint64_t k = shfl_xor_u64(best, o);
          best = k > best ? k : best;
        }
        const int row = mt * 32 + 8 * wave + 4 * g + j;
        if (ln == 0 && row < e.M) e.amax_keys[(int64_t)row * e.amax_groups + group] = best;
      }
  }
}

// ---------------------------------------------------------------------------
// NF4 GEMM
// ---------------------------------------------------------------------------
// One wave's units [w0, w1) of column group `group` (a unit is 128 along K:
// the lane's 64-block of each tile, 8 MFMA k-steps); WV = this wave's index
// (compile time, so table offsets are immediates).
//   * codes of unit p + 1 are in flight while unit p is computed; X one unit
//     ahead (four k-steps with two M tiles), each fragment requested before
//     the codes loaded after the unit, so waiting for X never waits for them;
//   * table lookups go in batches of 8 reads (one tile, one k-step), the next
//     batch issued before the current one is waited for, which keeps the LDS
//     counter (15 outstanding at most) exact;
//   * one table build writes the entries of two units (low / high halves of
//     each dword), from absmax loaded a round ahead; a wave's tables are its
//     own, so no barrier is needed (a wave's LDS accesses run in order).
// The loop runs whole rounds of two units and is straight-line (prefetches
// past w1 are clamped to the last unit), so the compiler's wait counts stay
// exact; an odd last unit follows the loop.
// `mid` runs once the wave's first loads are issued (epilogue operands that
// do not depend on the product are requested there).
template <int MT, int NT, int WV, bool XT, bool AF, typename Mid>
__device__ __forceinline__ void nf4_wave_body(f32x16_t (&acc)[NT][MT], uint8_t* smem,
                                              const uint16_t* __restrict__ X, int64_t ldx,
                                              const uint8_t* __restrict__ W, const void* __restrict__ Wabs,
                                              int NP, int group, int w0, int w1, int M, uint32_t region, Mid&& mid) {
  constexpr int XD = MT == 1 ? 8 : 4;  // X k-steps in flight
  const int n = max(w1 - w0, 0);
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5, ln = lane & 31;
  constexpr int TB = WV * NT * kTabTile;  // this wave's table area
  uint8_t* lanetab = smem + region + lane * 4;
  // LDS address registers: the lane's table base in the low byte and the
  // table region (a multiple of 64 KiB) above bit 16 (the kernel's only LDS
  // object starts at offset 0, so bits 8..15 are free for the code).
  uint32_t addr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) addr[i] = region + (uint32_t)(lane * 4);

  // Rows at or beyond M read row M - 1: MFMA rows are independent and those
  // output rows are never stored.
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = X + (int64_t)min(mt * 32 + ln, M - 1) * ldx + 64 * g;

  u32x4_t qa[NT][2], qb[NT][2];  // codes of the lane's block in each tile (dword s = MFMA k-step s)
  uint32_t ac[2][NT];             // absmax bits of the next two units, for the next table build
  u32x4_t x[MT][XD];              // X fragments of k-steps s .. s + XD - 1

  const int wl = max(w1 - 1, 0);
  // The wave visits its units starting at a group-dependent rotation, so the
  // workgroups streaming at the same time touch different offsets of their
  // 64 KiB-aligned tiles. Unit p (w0 <= p, clamped to the last) -> stored unit.
  const int rot = n > 0 ? group % n : 0;
  auto unit_of = [&](int p) -> int {
    int r = min(p, wl) - w0 + rot;
    if (r >= n) r -= n;
    return n > 0 ? w0 + r : min(p, wl);
  };
  auto tile_of = [&](int nt, int p) -> int64_t { return (int64_t)(group * NT + nt) * NP + unit_of(p); };
  auto load_codes = [&](u32x4_t (&q)[NT][2], int p) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const u32x4_t* wp = (const u32x4_t*)(W + tile_of(nt, p) * 2048 + lane * 16);
      q[nt][0] = __builtin_nontemporal_load(wp);
      q[nt][1] = __builtin_nontemporal_load(wp + 64);
    }
  };
  auto load_abs = [&](int p) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int64_t ai = tile_of(nt, p + h) * 64 + lane;
        ac[h][nt] = AF ? ((const uint32_t*)Wabs)[ai] : (uint32_t)((const uint16_t*)Wabs)[ai];
      }
  };
  auto load_x = [&](int slot, int p, int s) {
    const int pc = unit_of(p);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (XT) x[mt][slot] = *(const u32x4_t*)(X + ((((int64_t)mt * NP + pc) * 8 + s) * 64 + lane) * 8);
      else x[mt][slot] = *(const u32x4_t*)(xrow[mt] + 128 * pc + 8 * s);
    }
  };
  auto unit = [&](const u32x4_t (&q)[NT][2], int p, auto slot_c, u32x4_t (&xs)[MT][XD], bool prefetch) {
    constexpr int SL = decltype(slot_c)::value;
    constexpr int NB = 8 * NT;  // batches: k-step b / NT, tile b % NT
    uint32_t r[2][8];
    auto issue = [&](int b, uint32_t (&rr)[8]) {
      const int s = b / NT, nt = b % NT;
      nf4_addr8(q[nt][s >> 2][s & 3], addr);
      if (nt == 0) nf4_read8<TB + SL>(smem, addr, rr);
      else nf4_read8<TB + kTabTile + SL>(smem, addr, rr);
    };
    issue(0, r[0]);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b + 1 < NB) issue(b + 1, r[(b + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      const int s = b / NT, nt = b % NT;
      const uint32_t (&cur)[8] = r[b & 1];
      const u32x4_t bv = {pack16(cur[0], cur[1]), pack16(cur[2], cur[3]), pack16(cur[4], cur[5]),
                          pack16(cur[6], cur[7])};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16<PE_DTYPE_BF16>(xs[mt][s % XD], bv, acc[nt][mt]);
      if (prefetch && nt == NT - 1) load_x(s % XD, p + ((s + XD) >> 3), (s + XD) & 7);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto build = [&]() {
    nf4_build_table2<TB, AF>(lanetab, ac[0][0], ac[1][0]);
    if constexpr (NT == 2) nf4_build_table2<TB + kTabTile, AF>(lanetab, ac[0][1], ac[1][1]);
  };
  constexpr std::integral_constant<int, 0> kLo{};
  constexpr std::integral_constant<int, 2> kHi{};

  if constexpr (MT == 1) {
    if (n <= 2) {
      // At most two units: every load of the wave is issued at once (absmax,
      // then codes and X of the first unit, then of the second), one table
      // build covers both, and each unit waits only for its own loads.
      u32x4_t xb[MT][XD];
      load_abs(w0);
      load_codes(qa, w0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < XD; ++s) load_x(s, w0, s);
      __builtin_amdgcn_sched_barrier(0);
      load_codes(qb, w0 + 1);
#pragma unroll
      for (int s = 0; s < XD; ++s) {
        const int pc = unit_of(w0 + 1);
        if constexpr (XT) xb[0][s] = *(const u32x4_t*)(X + (((int64_t)pc * 8 + s) * 64 + lane) * 8);
        else xb[0][s] = *(const u32x4_t*)(xrow[0] + 128 * pc + 8 * s);
      }
      __builtin_amdgcn_sched_barrier(0);
      build();
      mid();
      __builtin_amdgcn_sched_barrier(0);
      if (n > 0) unit(qa, w0, kLo, x, false);
      if (n > 1) unit(qb, w0 + 1, kHi, xb, false);
      return;
    }
  }
  // At the top of every round p the table holds units p, p + 1, and the loads
  // in flight are, in issue order, the codes of p, X k-steps 0 .. XD - 1 of p,
  // the codes of p + 1 and the absmax of p + 2, p + 3 (the codes of p already
  // arrived when the round is entered from the previous one). Each absmax load
  // is issued right after a table build has waited for the previous one, so a
  // build never waits for codes.
  load_abs(w0);
  load_codes(qa, w0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < XD; ++s) load_x(s, w0, s);
  __builtin_amdgcn_sched_barrier(0);
  load_codes(qb, w0 + 1);
  __builtin_amdgcn_sched_barrier(0);
  build();
  __builtin_amdgcn_sched_barrier(0);
  load_abs(w0 + 2);
  mid();
  const int rounds = n >> 1;
  int p = w0;
  for (int r = 0; r < rounds; ++r, p += 2) {
    __builtin_amdgcn_sched_barrier(0);
    unit(qa, p, kLo, x, true);
    load_codes(qa, p + 2);
    __builtin_amdgcn_sched_barrier(0);
    unit(qb, p + 1, kHi, x, true);
    load_codes(qb, p + 3);
    __builtin_amdgcn_sched_barrier(0);
    build();  // units p + 2, p + 3; the reads of p, p + 1 are all issued
    __builtin_amdgcn_sched_barrier(0);
    load_abs(p + 4);
  }
  if (n & 1) unit(qa, p, kLo, x, true);
}

// KW = 4 or 8 waves. Waves w and w + 4 run the same code (table offsets are
// immediates of wave index w % 4); the second four keep their tables 64 KiB
// higher, selected by bit 16 of the LDS address.
template <int MT, int NT, bool XT, int KW, bool AF>
__global__ __launch_bounds__(KW * 64, KW == 8 ? 1 : (MT == 1 ? 3 : 2)) void nf4_gemm_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, const uint8_t* __restrict__ W, const void* __restrict__ Wabs,
    int NP, int S, int pps, float* __restrict__ partial, int* __restrict__ counters, EpiArgs e, int nl, int tS,
    int tpps) {
  constexpr int kTabBytes = kWaves * NT * kTabTile;
  static_assert(kTabBytes <= 65536, "table offsets must fit the 16-bit LDS immediate");
  constexpr int kTabAll = KW == 8 ? 65536 + kTabBytes : kTabBytes;
  constexpr int kRedBytes = red_floats(KW, NT, MT) * 4;
  __shared__ __align__(256) uint8_t smem[kTabAll > kRedBytes ? kTabAll : kRedBytes];
  // nl > 0: workgroups [0, nl) take column groups [0, nl) whole; the rest take
  // the remaining groups in tS splits of tpps units each (split-K exchange)
  int group = blockIdx.x, split = blockIdx.y, Sg = S, ppsg = pps;
  if (nl > 0) {
    if ((int)blockIdx.x < nl) {
      split = 0;
      Sg = 1;
      ppsg = NP;
    } else {
      const int t = blockIdx.x - nl;
      group = nl + t / tS;
      split = t % tS;
      Sg = tS;
      ppsg = tpps;
    }
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p0 = split * ppsg;
  const int p1 = min(NP, p0 + ppsg);
  const int np = max(0, p1 - p0);
  const int w0 = p0 + (np * wave) / KW;
  const int w1 = p0 + (np * (wave + 1)) / KW;
  const uint32_t region = wave >= 4 ? 65536u : 0u;
  // eight-wave q/k/v launches fetch their RoPE operands while the GEMM runs
  const bool rope_pre = KW == 8 && NT == 2 && e.op == kEpiRopeKV && wave < kWaves;
  RopePre<MT> rp;
  {
    const int lane = threadIdx.x & 63, g = lane >> 5;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = mt * 32 + 8 * wave + 4 * g + j;
        rp.pos[mt][j] = (rope_pre && row < e.M) ? e.positions[row] : -1;
      }
  }
  auto mid = [&]() {
    if (!rope_pre) return;
    const int ln = threadIdx.x & 31;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        rope_fetch<PE_DTYPE_BF16>(e, group, ln, rp.pos[mt][j], rp.c1[mt][j], rp.s1[mt][j], rp.c2[mt][j],
                                  rp.s2[mt][j]);
  };

  f32x16_t acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nt][mt][r] = 0.f;

  switch (wave & 3) {
    case 0: nf4_wave_body<MT, NT, 0, XT, AF>(acc, smem, X, ldx, W, Wabs, NP, group, w0, w1, e.M, region, mid); break;
    case 1: nf4_wave_body<MT, NT, 1, XT, AF>(acc, smem, X, ldx, W, Wabs, NP, group, w0, w1, e.M, region, mid); break;
    case 2: nf4_wave_body<MT, NT, 2, XT, AF>(acc, smem, X, ldx, W, Wabs, NP, group, w0, w1, e.M, region, mid); break;
    default: nf4_wave_body<MT, NT, 3, XT, AF>(acc, smem, X, ldx, W, Wabs, NP, group, w0, w1, e.M, region, mid); break;
  }
  lds_barrier();  // every wave is done with its tables; smem becomes the reduction buffer
  finish_tile<PE_DTYPE_BF16, NT, MT, KW>(acc, (float*)smem, group, split, Sg, partial, counters, e, &rp, rope_pre);
}

// ---------------------------------------------------------------------------
// NF4 GEMM for many rows (the batched pass: 64 < M <= 256, A-tiled X)
// ---------------------------------------------------------------------------
// One workgroup = 8 waves = one group of four 32-column tiles (128 columns) x
// one K split; each 128-wide unit is dequantised once for every row.
// Waves 0-3 (producers) each dequantise tile w of every unit (the lane's own
// table, as in nf4_wave_body) into a two-slot LDS ring of bf16 MFMA B
// fragments; waves 4-7 (consumers) each multiply up to two M tiles by all
// four tiles of the unit in the other slot. Round t: the consumers multiply
// unit t (slot t % 2) while the producers fill unit t + 1 (slot (t + 1) % 2);
// one workgroup barrier ends the round. A SIMD holds one wave of each kind,
// so the lookups' VALU and LDS work and the matrix cores run at the same
// time, and each wave's in-order LDS counter covers one kind of access only
// (with both jobs in the same four waves, each MFMA waited for lookups issued
// after its operand). Both kinds run the same 1 + n barriers (n units; every
// condition below is uniform over the workgroup). Consumers split M, not K,
// so each accumulator holds the complete sum over the split's units; the
// result is written as fp32 split partials out[split][row][col] (plain
// stores), summed by the consumer kernels in split order.
constexpr int kBigNT = 4;
constexpr int kBigTab = 16 * 64 * 4;          // one producer's table: 16 codes x 64 lanes x dword (two units)
constexpr int kBigBufUnit = kBigNT * 8 * 64 * 16;  // B fragments of one unit: 4 tiles x 8 k-steps x 64 lanes x 16 B
constexpr int kBigSmem = kWaves * kBigTab + 2 * kBigBufUnit;

template <int WV>
__device__ __forceinline__ void bigws_producer(uint8_t* smem, const uint8_t* __restrict__ W,
                                               const uint16_t* __restrict__ Wabs, int NP, int group, int u0, int u1) {
  const int n = u1 - u0;
  const int lane = threadIdx.x & 63;
  constexpr int TB = WV * kBigTab;  // this wave's table
  uint8_t* lanetab = smem + lane * 4;
  uint32_t addr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) addr[i] = (uint32_t)(lane * 4);
  u32x4_t* bufs = (u32x4_t*)(smem + kWaves * kBigTab);
  const int64_t tile = (int64_t)group * kBigNT + WV;
  auto load_codes = [&](u32x4_t (&q)[2], int p) {
    const u32x4_t* wp = (const u32x4_t*)(W + (tile * NP + min(p, u1 - 1)) * 2048 + lane * 16);
    q[0] = __builtin_nontemporal_load(wp);
    q[1] = __builtin_nontemporal_load(wp + 64);
  };
  auto load_abs = [&](int p) -> uint32_t { return (uint32_t)Wabs[(tile * NP + min(p, u1 - 1)) * 64 + lane]; };
  // relative unit t (table half SL) into ring slot t % 2
  auto dequant = [&](const u32x4_t (&q)[2], int t, auto slot_c) {
    constexpr int SL = decltype(slot_c)::value;
    u32x4_t* dst = bufs + ((t & 1) * kBigNT + WV) * 8 * 64 + lane;
    uint32_t r[2][8];
    nf4_addr8(q[0][0], addr);
    nf4_read8<TB + SL>(smem, addr, r[0]);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s + 1 < 8) {
        nf4_addr8(q[(s + 1) >> 2][(s + 1) & 3], addr);
        nf4_read8<TB + SL>(smem, addr, r[(s + 1) & 1]);
      }
      const uint32_t (&cur)[8] = r[s & 1];
      dst[s * 64] = u32x4_t{pack16(cur[0], cur[1]), pack16(cur[2], cur[3]), pack16(cur[4], cur[5]),
                            pack16(cur[6], cur[7])};
    }
  };
  constexpr std::integral_constant<int, 0> kLo{};
  constexpr std::integral_constant<int, 2> kHi{};
  // qa holds the even relative units, qb the odd ones; a table build covers
  // an even unit (low halves) and the next (high halves)
  // Round r (r = 0 .. n, each ending with a barrier) fills relative unit r
  // while the consumers multiply unit r - 1.
  u32x4_t qa[2], qb[2];
  load_codes(qa, u0);
  load_codes(qb, u0 + 1);
  uint32_t a0 = load_abs(u0), a1 = load_abs(u0 + 1);
  for (int r = 0; r <= n; r += 2) {
    if (r < n) {
      nf4_build_table2<TB, false>(lanetab, a0, a1);  // the reads of units r - 2, r - 1 are issued
      a0 = load_abs(u0 + r + 2);
      a1 = load_abs(u0 + r + 3);
      dequant(qa, r, kLo);
      load_codes(qa, u0 + r + 2);
    }
    lds_barrier();
    if (r + 1 <= n) {
      if (r + 1 < n) {
        dequant(qb, r + 1, kHi);
        load_codes(qb, u0 + r + 3);
      }
      lds_barrier();
    }
  }
}

// SW: the launch has one split and stores the SwiGLU activation (a separate
// instance, so the split-partial launches carry no epilogue code)
template <int NMT, bool SW>
__device__ __forceinline__ void bigws_consumer(uint8_t* smem, const uint16_t* __restrict__ X, int NP, int group,
                                               int u0, int u1, int mt0, const EpiArgs& e, int split) {
  const int n = u1 - u0;
  constexpr int MA = NMT > 0 ? NMT : 1;  // array extents
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5, ln = lane & 31;
  const u32x4_t* bufs = (const u32x4_t*)(smem + kWaves * kBigTab);
  f32x16_t acc[kBigNT][MA];
#pragma unroll
  for (int nt = 0; nt < kBigNT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MA; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nt][mt][r] = 0.f;
  // X fragments in a ring of four k-steps, two k-steps ahead of their MFMAs
  u32x4_t x[4][MA];
  auto load_x = [&](int p, int s) {
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
      x[s & 3][mt] = *(const u32x4_t*)(X + ((((int64_t)(mt0 + mt) * NP + p) * 8 + s) * 64 + lane) * 8);
  };
  auto first_x = [&](int p) {
    load_x(p, 0);
    load_x(p, 1);
  };
  // relative unit t from ring slot t % 2: the four B fragments of k-step
  // s + 1 are requested before the MFMAs of k-step s; the next unit's first
  // X k-steps are requested before the round's barrier
  auto multiply = [&](int t) {
    const u32x4_t* src = bufs + (t & 1) * kBigNT * 8 * 64 + lane;
    u32x4_t b[2][kBigNT];
    auto load_b = [&](int s) {
#pragma unroll
      for (int nt = 0; nt < kBigNT; ++nt) b[s & 1][nt] = src[(nt * 8 + s) * 64];
    };
    if (NMT > 0) load_b(0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (NMT > 0 && s + 1 < 8) load_b(s + 1);
      if (s + 2 < 8) load_x(u0 + t, s + 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int nt = 0; nt < kBigNT; ++nt)
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) acc[nt][mt] = mfma16<PE_DTYPE_BF16>(x[s & 3][mt], b[s & 1][nt], acc[nt][mt]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (t + 1 < n) first_x(u0 + t + 1);
  };
  first_x(u0);
  lds_barrier();
  for (int t = 0; t < n; t += 2) {
    multiply(t);
    lds_barrier();
    if (t + 1 < n) {
      multiply(t + 1);
      lds_barrier();
    }
  }
  // row 32 mt + 8 q + 4 g + j, column (group * 4 + nt) * 32 + ln
  if constexpr (SW) {
    // One split (complete sums): tiles 2 p and 2 p + 1 are the gate and up
    // columns of activation columns (2 group + p) * 32 + c. After the last
    // barrier the LDS is free: each M tile goes through this wave's 16 KiB
    // (32 rows x 128 columns, fp32), and a rolled loop stores the activations.
    float* stage = (float*)smem + (threadIdx.x / 64 - kWaves) * 32 * 128;
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) {
#pragma unroll
      for (int nt = 0; nt < kBigNT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) stage[(8 * (r >> 2) + 4 * g + (r & 3)) * 128 + nt * 32 + ln] = acc[nt][mt][r];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll 1
      for (int it = 0; it < 32; ++it) {
        const int rr = it, c = lane;  // row of the tile, activation column of the group (pair c / 32)
        const int row = (mt0 + mt) * 32 + rr;
        const int pr = c >> 5, cl = c & 31;
        if (row < e.M)
          epi_swiglu<PE_DTYPE_BF16>(e, row, (2 * group + pr) * 32 + cl, stage[rr * 128 + 64 * pr + cl],
                                    stage[rr * 128 + 64 * pr + 32 + cl]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
  } else {
    // split partials
    float* out = (float*)e.out + (int64_t)split * e.M * e.N;
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = (mt0 + mt) * 32 + 8 * q4 + 4 * g + j;
          if (row < e.M)
#pragma unroll
            for (int nt = 0; nt < kBigNT; ++nt)
              out[(int64_t)row * e.N + (group * kBigNT + nt) * 32 + ln] = acc[nt][mt][4 * q4 + j];
        }
  }
}

constexpr int kWsWaves = 2 * kWaves;  // producers + consumers

template <bool SW>
__global__ __launch_bounds__(kWsWaves * 64, 1) void nf4_gemm_bigws_kernel(const uint16_t* __restrict__ X,
                                                                          const uint8_t* __restrict__ W,
                                                                          const uint16_t* __restrict__ Wabs, int NP,
                                                                          int pps, int mtiles, EpiArgs e) {
  __shared__ __align__(256) uint8_t smem[kBigSmem];
  const int group = blockIdx.x, split = blockIdx.y;
  const int u0 = split * pps, u1 = min(NP, u0 + pps);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (u0 >= u1) return;  // a whole workgroup: no barrier is left waiting
  if (wave < kWaves) {
    switch (wave) {
      case 0: bigws_producer<0>(smem, W, Wabs, NP, group, u0, u1); break;
      case 1: bigws_producer<1>(smem, W, Wabs, NP, group, u0, u1); break;
      case 2: bigws_producer<2>(smem, W, Wabs, NP, group, u0, u1); break;
      default: bigws_producer<3>(smem, W, Wabs, NP, group, u0, u1); break;
    }
    return;
  }
  // the consumers (the critical path) win issue arbitration over the
  // producers of their SIMD
  __builtin_amdgcn_s_setprio(2);
  // grid.z: blocks of eight 32-row tiles (a prefill of more than 256 rows)
  const int mt0 = blockIdx.z * 8 + (wave - kWaves) * 2;
  const int nmt = max(0, min(2, mtiles - mt0));
  if (nmt == 2) bigws_consumer<2, SW>(smem, X, NP, group, u0, u1, mt0, e, split);
  else if (nmt == 1) bigws_consumer<1, SW>(smem, X, NP, group, u0, u1, mt0, e, split);
  else bigws_consumer<0, SW>(smem, X, NP, group, u0, u1, mt0, e, split);
}

// ---------------------------------------------------------------------------
// Dense 16-bit GEMM for many rows (the batched pass's lm_head)
// ---------------------------------------------------------------------------
// Tiled bf16 / fp16 weights need no lookups, so the waves are not
// specialised: one workgroup = 4 waves = 128 columns x all of K; per 128-wide unit wave w
// copies tile w's MFMA B fragments of the unit (8 k-steps x 64 lanes x 16 B,
// requested two units ahead, in the k order of the A-tiled X) into the
// double-buffered LDS tile, and after one barrier multiplies its own M tiles
// by all four tiles.
// Each weight is read from HBM once for every row; the outputs are rounded
// once and stored in the dtype, row-major with leading dimension ld.
template <int DT, int NMT, int WV, bool F32OUT>
__device__ __forceinline__ void dense_bigm_wave(uint8_t* smem, const uint16_t* __restrict__ X,
                                                const uint16_t* __restrict__ W, int NP, int p0, int p1, int group,
                                                int mt0, int M, void* __restrict__ out, int64_t ld) {
  constexpr int MA = NMT > 0 ? NMT : 1;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5, ln = lane & 31;
  u32x4_t* bufs = (u32x4_t*)smem;
  const int64_t tile = (int64_t)group * kBigNT + WV;
  // A-tiled X gives k-step s of a unit the k = 64 g + 8 s + e (lane half g):
  // the two 64-wide halves interleaved, as the NF4 tiles order them. The dense
  // tiles hold k = 16 ks + 8 (lane / 32) + e, so lane (n, g) fetches its
  // fragment from k-step 8 p + 4 g + s / 2, lane n + 32 (s % 2) of the tile:
  // two 512-byte contiguous runs per load instruction.
  auto load_b = [&](u32x4_t (&b)[8], int p) {
    const int pc = min(p, p1 - 1);
    const u32x4_t* src = (const u32x4_t*)(W + ((tile * NP * 8 + 8 * pc + 4 * g) * 64 + ln) * 8);
#pragma unroll
    for (int s = 0; s < 8; ++s) b[s] = __builtin_nontemporal_load(src + (s >> 1) * 64 + 32 * (s & 1));
  };
  auto store_b = [&](const u32x4_t (&b)[8], int p) {
    u32x4_t* dst = bufs + ((p & 1) * kBigNT + WV) * 8 * 64 + lane;
#pragma unroll
    for (int s = 0; s < 8; ++s) dst[s * 64] = b[s];
  };
  f32x16_t acc[kBigNT][MA];
#pragma unroll
  for (int nt = 0; nt < kBigNT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MA; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nt][mt][r] = 0.f;
  u32x4_t x[4][MA];
  auto load_x = [&](int p, int s) {
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
      x[s & 3][mt] = *(const u32x4_t*)(X + ((((int64_t)(mt0 + mt) * NP + p) * 8 + s) * 64 + lane) * 8);
  };
  auto multiply = [&](int p) {
    const u32x4_t* src = bufs + (p & 1) * kBigNT * 8 * 64 + lane;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s + 2 < 8) load_x(p, s + 2);
#pragma unroll
      for (int nt = 0; nt < kBigNT; ++nt) {
        const u32x4_t b = src[(nt * 8 + s) * 64];
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) acc[nt][mt] = mfma16<DT>(x[s & 3][mt], b, acc[nt][mt]);
      }
    }
  };
  u32x4_t ba[8], bb[8];
  load_b(ba, p0);
  load_b(bb, p0 + 1);
  for (int p = p0; p < p1; p += 2) {
    load_x(p, 0);
    load_x(p, 1);
    store_b(ba, p);
    load_b(ba, p + 2);
    lds_barrier();  // unit p's fragments are complete; the other slot is free
    multiply(p);
    if (p + 1 < p1) {  // the same for every wave of the workgroup
      load_x(p + 1, 0);
      load_x(p + 1, 1);
      store_b(bb, p + 1);
      load_b(bb, p + 3);
      lds_barrier();
      multiply(p + 1);
    }
  }
  typedef typename Elem<DT>::T Te;
#pragma unroll
  for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = (mt0 + mt) * 32 + 8 * q4 + 4 * g + j;
        if (row < M)
#pragma unroll
          for (int nt = 0; nt < kBigNT; ++nt) {
            const int64_t o = (int64_t)row * ld + (group * kBigNT + nt) * 32 + ln;
            if constexpr (F32OUT)
              ((float*)out)[(int64_t)blockIdx.z * M * ld + o] = acc[nt][mt][4 * q4 + j];
            else
              Elem<DT>::store((Te*)out, o, acc[nt][mt][4 * q4 + j]);
          }
      }
}

// F32OUT: the fp32 sums are stored as they are, split partials
// out[split][row][col] for the prefill's epilogue kernels (grid.z: K splits of
// ceil(NP / splits) units, each non-empty); grid.y runs over blocks of eight
// 32-row tiles.
template <int DT, bool F32OUT>
__global__ __launch_bounds__(kWaves * 64, 2) void dense_gemm_bigm_kernel(const uint16_t* __restrict__ X,
                                                                        const uint16_t* __restrict__ W, int NP,
                                                                        int mtiles, int M, void* __restrict__ out,
                                                                        int64_t ld) {
  __shared__ __align__(256) uint8_t smem[2 * kBigBufUnit];
  const int group = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int mt0 = blockIdx.y * 8 + wave * 2;
  const int nmt = max(0, min(2, mtiles - mt0));
  const int ups = (NP + gridDim.z - 1) / gridDim.z;
  const int p0 = blockIdx.z * ups, p1 = min(NP, p0 + ups);
#define PE_DBIGM_WAVE(N)                                                                                  \
  switch (wave) {                                                                                         \
    case 0: dense_bigm_wave<DT, N, 0, F32OUT>(smem, X, W, NP, p0, p1, group, mt0, M, out, ld); break;     \
    case 1: dense_bigm_wave<DT, N, 1, F32OUT>(smem, X, W, NP, p0, p1, group, mt0, M, out, ld); break;     \
    case 2: dense_bigm_wave<DT, N, 2, F32OUT>(smem, X, W, NP, p0, p1, group, mt0, M, out, ld); break;     \
    default: dense_bigm_wave<DT, N, 3, F32OUT>(smem, X, W, NP, p0, p1, group, mt0, M, out, ld); break;    \
  }
  if (nmt == 2) {
    PE_DBIGM_WAVE(2)
  } else if (nmt == 1) {
    PE_DBIGM_WAVE(1)
  } else {
    PE_DBIGM_WAVE(0)
  }
#undef PE_DBIGM_WAVE
}

// ---------------------------------------------------------------------------
// Dense 16-bit GEMM over many rows: 256 x 256 output tiles
// ---------------------------------------------------------------------------
// One workgroup = 4 waves = 256 rows (eight 32-row tiles of the A-tiled X) x
// 256 columns (eight 32-column weight tiles); wave w owns rows 128 (w / 2) ..
// + 127 and columns 128 (w % 2) .. + 127: 4 x 4 MFMA tiles, 256 fp32
// accumulators. K is walked in stages of two MFMA k-steps. A stage's 16 A
// fragments (8 M tiles x 2 k-steps) and 16 B fragments (8 N tiles x 2
// k-steps), 1 KiB each, go straight from global memory into a four-stage LDS
// ring (global_load_lds_dwordx4: three stages in flight while one is
// multiplied); wave w loads fragments 8 w .. 8 w + 7 of the stage (A for
// w < 2, B otherwise). A fragments are copied as stored (the A-tiled layout is
// MFMA fragment order). The B fragment for k-step s of unit p is gathered lane
// by lane from weight k-step 8 p + 4 g + s / 2, lane n + 32 (s % 2) of the
// tiled weights, so that both operands hold the same k in the same place. Per
// stage a wave reads its 4 + 4 fragments of each k-step (ds_read_b128 at the
// lane's 16 bytes: conflict-free) and issues 32 MFMAs. One vmcnt wait and one
// barrier per stage; loads past the split's last stage repeat its last unit
// into buffers nobody reads. Work item w of the grid (column tile w / mblocks,
// row block w % mblocks) runs on XCD w / (grid / 8) when the grid is a
// multiple of eight, so the row blocks of a column tile share its weights in
// one L2. grid.y: K splits (fp32 partials out[split][row][col]).
constexpr int kT256Stage = 32 * 1024;
constexpr int kT256Ring = 4;
// s_waitcnt with vmcnt = 16 (expcnt and lgkmcnt at their maxima): this wave's
// loads of the two later stages in flight may still be outstanding
constexpr int kWaitVm16 = (16 & 15) | (7 << 4) | (15 << 8) | ((16 >> 4) << 14);

template <int DT, bool F32OUT>
__global__ __launch_bounds__(256, 1) void dense_gemm_t256_kernel(const uint16_t* __restrict__ X,
                                                                 const uint16_t* __restrict__ W, int units,
                                                                 int ups, int mtiles, int mblocks, int M,
                                                                 void* __restrict__ out, int64_t ld, int64_t N) {
  __shared__ __align__(1024) uint8_t smem[kT256Ring * kT256Stage];
  const int total = gridDim.x;
  const int b = blockIdx.x;
  const int w = (total & 7) ? b : (b & 7) * (total >> 3) + (b >> 3);
  const int ntile = w / mblocks, mblock = w - ntile * mblocks;
  const int split = blockIdx.y;
  const int u0 = split * ups, u1 = min(units, u0 + ups);
  if (u0 >= u1) return;
  const int nstages = (u1 - u0) * 4;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int ln = lane & 31, g = lane >> 5;
  const int KS = units * 8;  // weight k-steps
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  const uint16_t* xb = uniform_ptr(X);
  const uint16_t* wb = uniform_ptr(W);
  // this wave's eight fragments of a stage
  auto issue = [&](int t) {
    const int tc = min(t, nstages - 1);
    const int p = u0 + tc / 4, s0 = 2 * (tc % 4);
    const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_base + (t % kT256Ring) * kT256Stage + wave * 8192);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f = 8 * (wave & 1) + i;  // fragment of the operand: tile f / 2, k-step s0 + f % 2
      const int s = s0 + (f & 1);
      uint32_t off;
      if (wave < 2) {
        const int mt = min(mblock * 8 + (f >> 1), mtiles - 1);
        off = (uint32_t)((((mt * units + p) * 8 + s) * 64 + lane) * 16);
      } else {
        const int nt = ntile * 8 + (f >> 1);
        off = (uint32_t)((((int64_t)nt * KS + 8 * p + 4 * g + (s >> 1)) * 64 + ln + 32 * (s & 1)) * 16);
      }
      lds_dma16(wave < 2 ? (const void*)xb : (const void*)wb, off, dst + i * 1024);
    }
  };
  const int wm = wave >> 1, wn = wave & 1;
  f32x16_t acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;
  issue(0);
  issue(1);
  issue(2);
  for (int t = 0; t < nstages; ++t) {
    __builtin_amdgcn_s_waitcnt(kWaitVm16);  // this wave's loads of stage t have landed
    __syncthreads();                        // everyone's have; stage t - 1's buffer is free
    issue(t + 3);
    const uint8_t* st = smem + (t % kT256Ring) * kT256Stage + lane * 16;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      u32x4_t a[4], bf[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) a[mi] = *(const u32x4_t*)(st + ((4 * wm + mi) * 2 + sl) * 1024);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) bf[ni] = *(const u32x4_t*)(st + 16384 + ((4 * wn + ni) * 2 + sl) * 1024);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma16<DT>(a[mi], bf[ni], acc[mi][ni]);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the ring's last loads land before the workgroup ends
  typedef typename Elem<DT>::T Te;
  const int64_t base = F32OUT ? (int64_t)split * M * ld : 0;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = mblock * 256 + 128 * wm + 32 * mi + 8 * (r >> 2) + 4 * g + (r & 3);
      if (row >= M) continue;
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        const int64_t o = base + (int64_t)row * ld + ntile * 256 + 128 * wn + 32 * ni + ln;
        if constexpr (F32OUT)
          ((float*)out)[o] = acc[mi][ni][r];
        else
          Elem<DT>::store((Te*)out, o, acc[mi][ni][r]);
      }
    }
  (void)N;
}

// ---------------------------------------------------------------------------
// Dense 16-bit GEMM: one iteration = 4 MFMA k-steps (64 along K) of NT tiles.
// Same pipeline as the NF4 kernel; a padded iteration multiplies a zero X.
// XT: X is A-tiled (xtile_index). Weight k-step 4u + j holds, in lane half
// g, k = 64u + 16j + 8g .. + 7; in the A-tiled X those eight elements of row
// 32 mt + ln are chunk 2j + g of 128-column unit u / 2 at lane ln + 32 (u % 2),
// so each X load reads two 512-byte runs (whole cache lines) instead of
// 32 bytes from each of 32 rows.
// ---------------------------------------------------------------------------
template <int FMT, int MT, int NT, bool XT>
__global__ __launch_bounds__(kWaves * 64, 3) void dense_gemm_kernel(const uint16_t* __restrict__ X, int64_t ldx,
                                                                    int K, const uint16_t* __restrict__ W, int S,
                                                                    int ups, float* __restrict__ partial,
                                                                    int* __restrict__ counters, EpiArgs e) {
  __shared__ __align__(16) float red[red_floats(kWaves, NT, MT)];
  const int group = blockIdx.x, split = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 5, ln = lane & 31;
  const int NU = K >> 6, KS = K >> 4;
  const int u0 = split * ups;
  const int u1 = min(NU, u0 + ups);
  const int nu = max(0, u1 - u0);
  const int w0 = u0 + (nu * wave) / kWaves;
  const int w1 = u0 + (nu * (wave + 1)) / kWaves;

  f32x16_t acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nt][mt][r] = 0.f;

  const int n = w1 - w0;
  if (n > 0) {
    const uint16_t* xrow[MT];
    const int xunits = K >> 7;  // XT: 128-column units of a tiled row block
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      xrow[mt] = XT ? X + ((int64_t)mt * xunits * 8 + g) * 512 + ln * 8
                    : X + (int64_t)min(mt * 32 + ln, e.M - 1) * ldx + 8 * g;
    u32x4_t ba[NT][4], bb[NT][4], x[MT][4];
    auto load_w = [&](u32x4_t (&b)[NT][4], int u) {
      const int uc = min(u, w1 - 1);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          b[nt][j] = *(const u32x4_t*)(W + (((int64_t)(group * NT + nt) * KS + 4 * uc + j) * 64 + lane) * 8);
    };
    auto load_x = [&](int j, int u) {
      const int uc = min(u, w1 - 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        x[mt][j] = XT ? *(const u32x4_t*)(xrow[mt] + (((int64_t)(uc >> 1) * 8 + 2 * j) * 64 + 32 * (uc & 1)) * 8)
                      : *(const u32x4_t*)(xrow[mt] + 64 * uc + 16 * j);
    };
    auto iter = [&](const u32x4_t (&b)[NT][4], int u) {
      const uint32_t keep = u < w1 ? 0xffffffffu : 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const u32x4_t xa = x[mt][j] & keep;
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) acc[nt][mt] = mfma16<FMT>(xa, b[nt][j], acc[nt][mt]);
        }
        load_x(j, u + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    load_w(ba, w0);
#pragma unroll
    for (int j = 0; j < 4; ++j) load_x(j, w0);
    load_w(bb, w0 + 1);
    const int rounds = (n + 1) >> 1;
    for (int r = 0; r < rounds; ++r) {
      const int u = w0 + 2 * r;
      __builtin_amdgcn_sched_barrier(0);
      iter(ba, u);
      load_w(ba, u + 2);
      __builtin_amdgcn_sched_barrier(0);
      iter(bb, u + 1);
      load_w(bb, u + 3);
    }
  }
  finish_tile<FMT, NT, MT>(acc, red, group, split, S, partial, counters, e);
}

// fp32 linear (VALU): one wave per output column (with SwiGLU, the column's
// gate and up weight rows), lanes strided across K so that every weight and X
// load is 256 contiguous bytes; 8 rows per workgroup, each row's 64 lane sums
// reduced across the wave.
template <bool SW>
__global__ __launch_bounds__(256) void f32_gemm_kernel(const float* __restrict__ X, int64_t ldx, int M, int K,
                                                       const float* __restrict__ W, int n_out, EpiArgs e) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = blockIdx.x * 4 + wave;
  const int m0 = blockIdx.y * 8;
  if (col >= n_out) return;  // no workgroup barrier below
  const int wrow = SW ? (col >> 5) * 64 + (col & 31) : col;
  const float* wg = W + (int64_t)wrow * K;
  const float* wu = W + (int64_t)(wrow + 32) * K;
  const int nrow = min(8, M - m0);
  float a[8], b[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) a[r] = b[r] = 0.f;
  for (int k = lane; k < K; k += 64) {
    const float w1 = wg[k];
    const float w2 = SW ? wu[k] : 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (r < nrow) {
        const float x = X[(int64_t)(m0 + r) * ldx + k];
        a[r] = fmaf(x, w1, a[r]);
        if constexpr (SW) b[r] = fmaf(x, w2, b[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    a[r] = wave_sum(a[r]);
    if constexpr (SW) b[r] = wave_sum(b[r]);
  }
  if (lane != 0) return;
  for (int r = 0; r < nrow; ++r) {
    if constexpr (SW) epi_swiglu<PE_DTYPE_F32>(e, m0 + r, col, a[r], b[r]);
    else epi_value<PE_DTYPE_F32>(e, m0 + r, col, a[r]);
  }
}


// ---------------------------------------------------------------------------
// Consumers of split partials (partial[S][M][N] fp32, summed in split order)
// ---------------------------------------------------------------------------
// Thread (row, column group, quad q): columns 64 group + 4q .. + 3 and the same
// 32 further on are the halves a RoPE pair (q/k/v) or a gate/up pair (SwiGLU)
// combines; four columns per thread make every access 16 (fp32) or 8 bytes.
__device__ __forceinline__ void sum_partials4(const float* __restrict__ pr, int S, int64_t sstride, float (&a)[4],
                                              float (&b)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = b[i] = 0.f;
#pragma unroll 4
  for (int sp = 0; sp < S; ++sp) {
    const float4 t = *(const float4*)(pr + sp * sstride);
    const float4 u = *(const float4*)(pr + sp * sstride + 32);
    a[0] += t.x; a[1] += t.y; a[2] += t.z; a[3] += t.w;
    b[0] += u.x; b[1] += u.y; b[2] += u.z; b[3] += u.w;
  }
}

// write_rope_kv for four consecutive dims d1 .. d1 + 3 (and d1 + hd/2 ..).
template <int DT>
__device__ __forceinline__ void write_rope_kv4(const EpiArgs& e, int group, int ln0, int row, const float (&a1)[4],
                                               const float (&a2)[4]) {
  typedef Elem<DT> E;
  typedef typename E::T T;
  typedef Vec4<DT> V;
  const int gpu = e.hd >> 6;
  const int u = group / gpu, j = group % gpu;
  const int d1 = 32 * j + ln0, d2 = d1 + (e.hd >> 1);
  float x1[4], x2[4];
  if (e.bias) {
    float b1[4], b2[4];
    V::load((const T*)e.bias + u * e.hd + d1, b1);
    V::load((const T*)e.bias + u * e.hd + d2, b2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x1[i] = E::round(__fadd_rn(a1[i], b1[i]));
      x2[i] = E::round(__fadd_rn(a2[i], b2[i]));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x1[i] = E::round(a1[i]);
      x2[i] = E::round(a2[i]);
    }
  }
  const int64_t kvo = u >= e.nh ? kv_row_elem(e, row) : 0;
  if (kvo < 0) return;
  if (u >= e.nh + e.nkv) {  // v: appended as is
    T* dst = (T*)e.v_cache + (int64_t)(u - e.nh - e.nkv) * e.cap * e.hd + kvo;
    V::store(dst + d1, x1);
    V::store(dst + d2, x2);
    return;
  }
  const int64_t p = e.positions[row];
  if (p < 0 || p >= e.max_pos) {
    if (e.status) atomicOr(e.status, PE_ERR_CAPACITY);
    return;
  }
  const T* cosr = (const T*)e.cos_sin + p * e.hd;
  const T* sinr = (const T*)e.cos_sin + (e.max_pos + p) * e.hd;
  float c1[4], c2[4], s1[4], s2[4], o1[4], o2[4];
  V::load(cosr + d1, c1);
  V::load(cosr + d2, c2);
  V::load(sinr + d1, s1);
  V::load(sinr + d2, s2);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o1[i] = E::round(__fadd_rn(E::round(__fmul_rn(x1[i], c1[i])), E::round(__fmul_rn(-x2[i], s1[i]))));
    o2[i] = E::round(__fadd_rn(E::round(__fmul_rn(x2[i], c2[i])), E::round(__fmul_rn(x1[i], s2[i]))));
  }
  T* dst = (u < e.nh) ? (T*)e.q_out + ((int64_t)row * e.nh + u) * e.hd
                      : (T*)e.k_cache + (int64_t)(u - e.nh) * e.cap * e.hd + kvo;
  V::store(dst + d1, o1);
  V::store(dst + d2, o2);
}

template <int DT>
__global__ __launch_bounds__(256) void rope_kv_partials_kernel(const float* __restrict__ partial, int S, EpiArgs e) {
  const int quads = e.N >> 3;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= e.M * quads) return;
  const int row = idx / quads, rem = idx - row * quads;
  const int group = rem >> 3, ln0 = (rem & 7) * 4;
  float a1[4], a2[4];
  sum_partials4(partial + (int64_t)row * e.N + group * 64 + ln0, S, (int64_t)e.M * e.N, a1, a2);
  write_rope_kv4<DT>(e, group, ln0, row, a1, a2);
}

template <int DT>
__global__ __launch_bounds__(256) void swiglu_partials_kernel(const float* __restrict__ partial, int S, EpiArgs e) {
  typedef Elem<DT> E;
  typedef typename E::T T;
  const int quads = e.N >> 3;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= e.M * quads) return;
  const int row = idx / quads, rem = idx - row * quads;
  const int group = rem >> 3, ln0 = (rem & 7) * 4;
  float gv[4], uv[4], o[4];
  sum_partials4(partial + (int64_t)row * e.N + group * 64 + ln0, S, (int64_t)e.M * e.N, gv, uv);
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = E::round(__fmul_rn(E::round(silu_f(E::round(gv[i]))), E::round(uv[i])));
  const int col = group * 32 + ln0;
  T* out = (T*)e.out;
  Vec4<DT>::store(out + (e.out_units ? xtile_index(row, col, e.out_units) : (int64_t)row * e.ld_out + col), o);
}

// ---------------------------------------------------------------------------
// Launch planning
// ---------------------------------------------------------------------------
constexpr int kMaxChunkRows = 64;  // M rows per launch (MT <= 2)

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v ? atoi(v) : dflt;
}

struct Plan {
  int NT, MT, S, per_split, groups, units;
  // NF4 hybrid launch (column groups between one and two per CU): nl whole
  // groups, the other groups in tS splits of tpps units; nl = 0 otherwise
  int nl, tS, tpps;
  int KW;  // NF4 waves per workgroup (4, or 8 for an unsplit launch of at most one workgroup per CU)
  int64_t partial_bytes;
};

// units: 128-wide K units (NF4) or 64-wide K steps (dense).
// NF4 split partials: as many splits as one round of one workgroup per CU
// holds (at least two units per wave); with more column groups than CUs (one
// M tile) K / 1024 splits, two units per wave.
// NF4 otherwise: the fewest splits that give at least `min_wgs` workgroups
// (one CU pulls under 1/128 of the HBM bandwidth), keeping every wave at least
// `min_units` units; at the 7B shapes q/k/v and gate/up get one split (the
// epilogue runs in the GEMM, no exchange).
// Dense q/k/v (split exchange) and o/down (split partials): as many splits as
// keep the launch within one workgroup per CU. Other dense launches: S spreads
// the work over about `wave_slots` waves (256 CUs x 3 four-wave workgroups), a
// wave getting at least 2 units.
// Either way the splits are balanced to differ by at most one unit per wave.
// CUs of the current device (256 on MI355X), queried once.
int cu_count() {
  static const int n = [] {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                  hipSuccess || cus <= 0)
      cus = 256;
    return cus;
  }();
  return n;
}

Plan make_plan(int M, int N, int K, bool nf4, int epi) {
  // dense linears: about 1792 waves' worth of units per launch (the 14B fp16
  // linears then run 400-480 workgroups in 4-6 K splits; 3072 gave 7-9
  // splits and a pass 6% slower)
  static const int wave_slots = env_int("PE_GEMM_WAVE_SLOTS", 1792);
  static const int nf4_min_wgs = env_int("PE_NF4_MIN_WGS", 128);
  static const int nf4_min_units = env_int("PE_NF4_MIN_UNITS", 2);
  static const int min_units = env_int("PE_GEMM_MIN_UNITS", 2);
  static const int nf4_upw = env_int("PE_NF4_UNITS_PER_WAVE", 2) == 1 ? 1 : 2;
  static const int nf4_wide_groups = env_int("PE_NF4_WIDE_GROUPS", 256);
  static const bool nf4_hybrid = env_int("PE_NF4_HYBRID", 1) != 0;
  static const int nf4_hybrid_ts = env_int("PE_NF4_HYBRID_TS", 2);
  static const int nf4_hybrid_less = env_int("PE_NF4_HYBRID_LESS", 0);
  Plan p;
  p.NT = (epi == PE_EPI_SWIGLU || epi == kEpiRopeKV || N % 64 == 0) ? 2 : 1;
  p.MT = M > 32 ? 2 : 1;
  p.groups = N / (32 * p.NT);
  p.units = nf4 ? K / 128 : K / 64;
  int S;
  if (nf4 && epi == kEpiPartial && p.groups <= cu_count()) {
    // split partials: as many splits as fill one round of one workgroup per
    // CU, each wave at least two units (the 7B o and down projections at 26
    // and at 64 rows: 4 splits, 256 workgroups; down had 11 splits of two units
    // per wave, 704 workgroups, at 26 rows and 2 at 64: 3% and 6% of the
    // passes)
    S = cu_count() / p.groups;
    const int s_units = p.units / (kWaves * nf4_min_units);
    if (S > s_units) S = s_units;
  } else if (nf4 && p.MT == 1 && epi == kEpiPartial && p.units <= kMaxSplits * kWaves * nf4_upw) {
    // split partials, at most two units per wave: the wave issues all of its
    // loads at once
    S = (p.units + kWaves * nf4_upw - 1) / (kWaves * nf4_upw);
  } else if (nf4) {
    S = (nf4_min_wgs + p.groups - 1) / p.groups;
    const int s_units = p.units / (kWaves * nf4_min_units);
    if (S > s_units) S = s_units;
  } else if (epi == kEpiRopeKV || epi == kEpiPartial) {
    // dense split exchange (q/k/v) or split partials (o, down): at most one
    // round of one workgroup per CU; a second, partly filled round costs more
    // than the splits save
    S = cu_count() / p.groups;
    const int s_units = p.units / (kWaves * min_units);
    if (S > s_units) S = s_units;
  } else {
    const int64_t total = (int64_t)p.groups * p.units;
    int per_wave = (int)((total + wave_slots - 1) / wave_slots);
    if (per_wave < min_units) per_wave = min_units;
    S = (p.units + per_wave * kWaves - 1) / (per_wave * kWaves);
  }
  if (S > kMaxSplits) S = kMaxSplits;
  if (S < 1) S = 1;
  p.per_split = (p.units + S - 1) / S;
  p.S = (p.units + p.per_split - 1) / p.per_split;
  p.partial_bytes = partial_bytes_of(p.S, p.groups, p.MT, p.NT);
  // Fewer column groups than CUs: eight waves per workgroup, two per SIMD, so
  // one wave's waits overlap the other's issue.
  p.KW = (nf4 && p.MT == 1 && p.NT == 2 && p.S == 1 && p.groups <= nf4_wide_groups) ? 8 : 4;
  // Between one and two column groups per CU (unsplit): one whole group per
  // CU, the rest split in halves, so each CU carries one whole group and at
  // most one half group instead of one or two whole ones; the halves finish
  // early and their exchange is off the critical path. (Quarters, thirds and
  // more or fewer whole groups measured slower in the 7B pass.)
  p.nl = p.tS = p.tpps = 0;
  const int ncu = cu_count();
  if (nf4 && p.NT == 2 && p.S == 1 && epi != kEpiPartial && nf4_hybrid && p.groups > ncu &&
      p.groups < 2 * ncu && p.units >= 4 * kWaves) {
    p.nl = ncu - nf4_hybrid_less;
    p.tS = nf4_hybrid_ts;
    p.tpps = (p.units + p.tS - 1) / p.tS;
    p.partial_bytes = partial_bytes_of(p.tS, p.groups, p.MT, p.NT);
  }
  return p;
}

int64_t workspace_of(const Plan& p) { return kCounterBytes + p.partial_bytes; }

// fmt: -1 = NF4 (bf16 compute), else PE_DTYPE_BF16 / PE_DTYPE_F16 dense.
// ws: [counters | partials]; the counters are zero on entry and left zero.
// NF4 format codes of launch_gemm / mfma_gemm (dtype codes are >= 0)
constexpr int kFmtNF4 = -1;     // fp16 absmax
constexpr int kFmtNF4F32 = -2;  // fp32 absmax
int nf4_fmt(int wfmt) { return wfmt == PE_WFMT_NF4_F32ABS ? kFmtNF4F32 : kFmtNF4; }

template <bool AF>
void launch_nf4(const Plan& p, dim3 grid, hipStream_t st, const uint16_t* x, int64_t ldx, bool x_tiled,
                const void* w, const void* wabs, float* partial, int* counters, const EpiArgs& e) {
#define PE_NF4(MT_, NT_, XT_)                                                                                       \
  nf4_gemm_kernel<MT_, NT_, XT_, kWaves, AF><<<grid, kWaves * 64, 0, st>>>(x, ldx, (const uint8_t*)w, wabs, p.units, \
                                                                            p.S, p.per_split, partial, counters, e,  \
                                                                            p.nl, p.tS, p.tpps)
  if (x_tiled) {
    if (p.NT == 2 && p.MT == 1 && p.KW == 8)
      nf4_gemm_kernel<1, 2, true, 8, AF><<<grid, 8 * 64, 0, st>>>(x, ldx, (const uint8_t*)w, wabs, p.units, p.S,
                                                                   p.per_split, partial, counters, e, p.nl, p.tS,
                                                                   p.tpps);
    else if (p.NT == 2) { if (p.MT == 1) PE_NF4(1, 2, true); else PE_NF4(2, 2, true); }
    else { if (p.MT == 1) PE_NF4(1, 1, true); else PE_NF4(2, 1, true); }
  } else {
    if (p.NT == 2) { if (p.MT == 1) PE_NF4(1, 2, false); else PE_NF4(2, 2, false); }
    else { if (p.MT == 1) PE_NF4(1, 1, false); else PE_NF4(2, 1, false); }
  }
#undef PE_NF4
}

int launch_gemm(int fmt, const Plan& p, hipStream_t st, const uint16_t* x, int64_t ldx, bool x_tiled, int K,
                const void* w, const void* wabs, void* ws, const EpiArgs& e) {
  if (p.groups > kMaxGroups) return PE_ERR_ARG;
  dim3 grid(p.groups, p.S);
  if (p.nl > 0) grid = dim3(p.nl + (p.groups - p.nl) * p.tS, 1);
  int* counters = (int*)ws;
  float* partial = (float*)((char*)ws + kCounterBytes);
  if (fmt < 0) {
    if (fmt == kFmtNF4F32)
      launch_nf4<true>(p, grid, st, x, ldx, x_tiled, w, wabs, partial, counters, e);
    else
      launch_nf4<false>(p, grid, st, x, ldx, x_tiled, w, wabs, partial, counters, e);
  } else {
    if (x_tiled && K % 128) return PE_ERR_ARG;
#define PE_DENSE(F, MT_, NT_)                                                                                         \
  do {                                                                                                               \
    if (x_tiled)                                                                                                     \
      dense_gemm_kernel<F, MT_, NT_, true><<<grid, kWaves * 64, 0, st>>>(x, ldx, K, (const uint16_t*)w, p.S,        \
                                                                         p.per_split, partial, counters, e);       \
    else                                                                                                             \
      dense_gemm_kernel<F, MT_, NT_, false><<<grid, kWaves * 64, 0, st>>>(x, ldx, K, (const uint16_t*)w, p.S,       \
                                                                          p.per_split, partial, counters, e);      \
  } while (0)
    if (fmt == PE_DTYPE_F16) {
      if (p.NT == 2) { if (p.MT == 1) PE_DENSE(PE_DTYPE_F16, 1, 2); else PE_DENSE(PE_DTYPE_F16, 2, 2); }
      else { if (p.MT == 1) PE_DENSE(PE_DTYPE_F16, 1, 1); else PE_DENSE(PE_DTYPE_F16, 2, 1); }
    } else {
      if (p.NT == 2) { if (p.MT == 1) PE_DENSE(PE_DTYPE_BF16, 1, 2); else PE_DENSE(PE_DTYPE_BF16, 2, 2); }
      else { if (p.MT == 1) PE_DENSE(PE_DTYPE_BF16, 1, 1); else PE_DENSE(PE_DTYPE_BF16, 2, 1); }
    }
#undef PE_DENSE
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}

int check_gemm_args(const void* x, int M, int K, const void* w, int N, int epi, const void* resid, const void* out) {
  if (!x || !w || !out || M <= 0 || K <= 0 || N <= 0 || K % 128 || N % 32) return PE_ERR_ARG;
  if (epi == PE_EPI_SWIGLU && N % 64) return PE_ERR_ARG;
  if (epi == PE_EPI_RESIDUAL && !resid) return PE_ERR_ARG;
  if (epi < 0 || epi > PE_EPI_SWIGLU) return PE_ERR_ARG;
  return PE_OK;
}

EpiArgs make_epi(int epi, int mc, int N, const void* bias, const void* resid, int64_t ld_resid, void* out,
                 int64_t ld_out) {
  EpiArgs e;
  e.op = epi;
  e.M = mc;
  e.N = N;
  e.bias = bias;
  e.resid = resid;
  e.ld_resid = ld_resid;
  e.out = out;
  e.ld_out = ld_out;
  e.out_units = 0;
  e.positions = nullptr;
  e.cos_sin = nullptr;
  e.max_pos = 0;
  e.q_out = e.k_cache = e.v_cache = nullptr;
  e.cap = e.row0 = 0;
  e.kv_off = nullptr;
  e.nh = e.nkv = e.hd = 0;
  e.status = nullptr;
  e.amax_keys = nullptr;
  e.amax_groups = 0;
  return e;
}

// M is processed in chunks of up to 64 rows, one launch each.
// x_tiled: X is A-tiled (M <= 64, one launch); out_units > 0: out is A-tiled.
int mfma_gemm(int fmt, const void* x, int64_t ldx, int M, int K, const void* w, const void* wabs, int N,
              int epi, const void* bias, const void* resid, int64_t ld_resid, void* out, int64_t ld_out,
              void* ws, int64_t ws_bytes, hipStream_t st, bool x_tiled = false, int out_units = 0,
              uint64_t* amax_keys = nullptr) {
  int rc = check_gemm_args(x, M, K, w, N, epi, resid, out);
  if (rc != PE_OK) return rc;
  if (amax_keys && (epi != PE_EPI_STORE || out_units)) return PE_ERR_ARG;
  const bool nf4 = fmt < 0;
  if ((x_tiled || out_units) && M > kMaxChunkRows) return PE_ERR_ARG;
  if (out_units && epi == PE_EPI_RESIDUAL) return PE_ERR_ARG;
  int done = 0;
  while (done < M) {
    const int mc = (M - done > kMaxChunkRows) ? kMaxChunkRows : (M - done);
    Plan p = make_plan(mc, N, K, nf4, amax_keys ? kEpiArgmax : epi);
    if (!ws || ws_bytes < workspace_of(p)) return PE_ERR_WORKSPACE;
    const size_t esz = 2;
    EpiArgs e = make_epi(epi, mc, N, bias, resid ? (const char*)resid + (size_t)done * ld_resid * esz : nullptr,
                         ld_resid, (char*)out + (size_t)done * ld_out * esz, ld_out);
    e.out_units = out_units;
    if (amax_keys) {
      e.op = kEpiArgmax;
      e.amax_groups = p.groups;
      e.amax_keys = amax_keys + (int64_t)done * p.groups;
    }
    const uint16_t* xc = x_tiled ? (const uint16_t*)x : (const uint16_t*)x + (size_t)done * ldx;
    rc = launch_gemm(fmt, p, st, xc, ldx, x_tiled, K, w, wabs, ws, e);
    if (rc != PE_OK) return rc;
    done += mc;
  }
  return PE_OK;
}

}  // namespace

// The q/k/v projection with its RoPE + KV-append epilogue (weight rows in
// head-paired tile order; hd % 64 == 0), one launch over M <= 64 rows.
int pe_internal_gemm_rope_kv(int wfmt, int dtype, const void* x, int64_t ldx, int M, int K, const void* w,
                             const void* wabs, int nh, int nkv, int hd, const void* bias,
                             const int64_t* positions, const void* cos_sin, int64_t max_pos, void* q_out,
                             void* k_cache, void* v_cache, int64_t cap, int64_t row0, int32_t* status, void* ws,
                             int64_t ws_bytes, bool x_tiled, hipStream_t st, const int64_t* kv_off) {
  const int N = (nh + 2 * nkv) * hd;
  if (M > kMaxChunkRows || hd % 64 || !positions || !cos_sin || !q_out || !k_cache || !v_cache) return PE_ERR_ARG;
  if (!kv_off && (row0 < 0 || row0 + M > cap)) return PE_ERR_CAPACITY;
  int rc = check_gemm_args(x, M, K, w, N, PE_EPI_SWIGLU, nullptr, q_out);
  if (rc != PE_OK) return rc;
  const bool nf4 = pe_wfmt_nf4(wfmt);
  Plan p = make_plan(M, N, K, nf4, kEpiRopeKV);
  if (!ws || ws_bytes < workspace_of(p)) return PE_ERR_WORKSPACE;
  EpiArgs e = make_epi(kEpiRopeKV, M, N, bias, nullptr, 0, nullptr, 0);
  e.positions = positions;
  e.cos_sin = cos_sin;
  e.max_pos = max_pos;
  e.q_out = q_out;
  e.k_cache = k_cache;
  e.v_cache = v_cache;
  e.cap = cap;
  e.row0 = row0;
  e.kv_off = kv_off;
  e.nh = nh;
  e.nkv = nkv;
  e.hd = hd;
  e.status = status;
  return launch_gemm(nf4 ? nf4_fmt(wfmt) : dtype, p, st, (const uint16_t*)x, ldx, x_tiled, K, w, wabs, ws, e);
}

int pe_internal_linear(int wfmt, int dtype, const void* x, int64_t ldx, bool x_tiled, int M, int K, const void* w,
                       const void* wabs, int N, int epi, const void* bias, const void* resid, int64_t ld_resid,
                       void* out, int64_t ld_out, int out_units, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (pe_wfmt_nf4(wfmt)) {
    if (!wabs) return PE_ERR_ARG;
    return mfma_gemm(nf4_fmt(wfmt), x, ldx, M, K, w, wabs, N, epi, bias, resid, ld_resid, out, ld_out, ws, ws_bytes, st,
                     x_tiled, out_units);
  }
  if (dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16) return PE_ERR_ARG;
  return mfma_gemm(dtype, x, ldx, M, K, w, nullptr, N, epi, bias, resid, ld_resid, out, ld_out, ws, ws_bytes, st,
                   x_tiled, out_units);
}

int64_t pe_internal_gemm_rope_kv_bytes(int M, int N, int K, int wfmt) {
  // callers with more rows launch 64-row chunks and a shorter last one
  const bool nf4 = pe_wfmt_nf4(wfmt);
  int64_t w = workspace_of(make_plan(M > kMaxChunkRows ? kMaxChunkRows : M, N, K, nf4, kEpiRopeKV));
  if (M > kMaxChunkRows && M % kMaxChunkRows) {
    const int64_t wr = workspace_of(make_plan(M % kMaxChunkRows, N, K, nf4, kEpiRopeKV));
    if (wr > w) w = wr;
  }
  return w;
}

// Y = X . W^T as split partials partial[S][M][N] (fp32, plain stores: no
// exchange between workgroups, the consumer sums them); one launch, M <= 64.
int pe_internal_linear_partials(int wfmt, int dtype, const void* x, int64_t ldx, bool x_tiled, int M, int K,
                                const void* w, const void* wabs, int N, float* partial, int64_t partial_bytes,
                                int* splits, hipStream_t st) {
  if (M > kMaxChunkRows || !partial || !splits) return PE_ERR_ARG;
  int rc = check_gemm_args(x, M, K, w, N, PE_EPI_STORE, nullptr, partial);
  if (rc != PE_OK) return rc;
  const bool nf4 = pe_wfmt_nf4(wfmt);
  if (nf4 ? !wabs : (dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16)) return PE_ERR_ARG;
  const Plan p = make_plan(M, N, K, nf4, kEpiPartial);
  if (partial_bytes < (int64_t)p.S * M * N * 4) return PE_ERR_WORKSPACE;
  EpiArgs e = make_epi(kEpiPartial, M, N, nullptr, nullptr, 0, partial, N);
  *splits = p.S;
  return launch_gemm(nf4 ? nf4_fmt(wfmt) : dtype, p, st, (const uint16_t*)x, ldx, x_tiled, K, w, wabs, nullptr, e);
}

int64_t pe_internal_linear_partials_bytes(int M, int N, int K, int wfmt) {
  if (M > kMaxChunkRows) M = kMaxChunkRows;
  return (int64_t)make_plan(M, N, K, pe_wfmt_nf4(wfmt), kEpiPartial).S * M * N * 4;
}

// The q/k/v epilogue (bias, RoPE at positions[row], q to q_out, K/V appended
// at cache rows row0 + row) applied to S split partials of the projection.
int pe_internal_rope_kv_partials(const float* partial, int S, int M, int nh, int nkv, int hd, const void* bias,
                                 const int64_t* positions, const void* cos_sin, int64_t max_pos, void* q_out,
                                 void* k_cache, void* v_cache, int64_t cap, int64_t row0, int32_t* status, int dtype,
                                 hipStream_t st, const int64_t* kv_off) {
  if (!partial || S < 1 || M <= 0 || hd <= 0 || hd % 64 || !positions || !cos_sin || !q_out || !k_cache ||
      !v_cache)
    return PE_ERR_ARG;
  if (!kv_off && (row0 < 0 || row0 + M > cap)) return PE_ERR_CAPACITY;
  const int N = (nh + 2 * nkv) * hd;
  EpiArgs e = make_epi(kEpiRopeKV, M, N, bias, nullptr, 0, nullptr, 0);
  e.positions = positions;
  e.cos_sin = cos_sin;
  e.max_pos = max_pos;
  e.q_out = q_out;
  e.k_cache = k_cache;
  e.v_cache = v_cache;
  e.cap = cap;
  e.row0 = row0;
  e.kv_off = kv_off;
  e.nh = nh;
  e.nkv = nkv;
  e.hd = hd;
  e.status = status;
  const int grid = pe_cdiv((int64_t)M * (N / 8), 256);
  if (dtype == PE_DTYPE_BF16) rope_kv_partials_kernel<PE_DTYPE_BF16><<<grid, 256, 0, st>>>(partial, S, e);
  else if (dtype == PE_DTYPE_F16) rope_kv_partials_kernel<PE_DTYPE_F16><<<grid, 256, 0, st>>>(partial, S, e);
  else return PE_ERR_ARG;
  PE_CHECK_LAUNCH();
  return PE_OK;
}

// SwiGLU of S split partials of the interleaved gate/up projection (N columns,
// N / 2 outputs), row-major or A-tiled (out_units > 0).
int pe_internal_swiglu_partials(const float* partial, int S, int M, int N, void* out, int64_t ld_out, int out_units,
                                int dtype, hipStream_t st) {
  if (!partial || !out || S < 1 || M <= 0 || N <= 0 || N % 64) return PE_ERR_ARG;
  EpiArgs e = make_epi(PE_EPI_SWIGLU, M, N, nullptr, nullptr, 0, out, ld_out);
  e.out_units = out_units;
  const int grid = pe_cdiv((int64_t)M * (N / 8), 256);
  if (dtype == PE_DTYPE_BF16) swiglu_partials_kernel<PE_DTYPE_BF16><<<grid, 256, 0, st>>>(partial, S, e);
  else if (dtype == PE_DTYPE_F16) swiglu_partials_kernel<PE_DTYPE_F16><<<grid, 256, 0, st>>>(partial, S, e);
  else return PE_ERR_ARG;
  PE_CHECK_LAUNCH();
  return PE_OK;
}

// The many-row NF4 GEMM (A-tiled X of M rows, 64 < M <= 256, N % 128 == 0):
// split partials [S][M][N]; S chosen for about two workgroups per CU.
namespace {
struct BigPlan {
  int groups, units, S, pps;
};
BigPlan big_plan(int N, int K) {
  BigPlan p;
  p.groups = N / (32 * kBigNT);
  p.units = K / 128;
  // At most one workgroup per CU (one eight-wave workgroup fills a CU's
  // registers), all resident at once: every further split adds M x N x 4
  // bytes of partials that the consuming kernel re-reads, and a launch past
  // the CU count runs a second, mostly idle round (gate/up at 216 groups
  // takes one split).
  static const int forced = env_int("PE_BIGM_SPLITS", 0);
  const int cu = cu_count();
  int S = cu / p.groups;
  if (S < 1) S = 1;
  if (forced > 0) S = forced;
  if (S > kMaxSplits) S = kMaxSplits;
  if (S > p.units) S = p.units;
  if (S < 1) S = 1;
  p.pps = (p.units + S - 1) / S;
  p.S = (p.units + p.pps - 1) / p.pps;
  return p;
}
}  // namespace

int64_t pe_internal_nf4_bigm_partials_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K < 128 || N % (32 * kBigNT) || K % 128) return 0;
  return (int64_t)big_plan(N, K).S * M * N * 4;
}

int pe_internal_dense_bigm(const void* x_tiled, int M, int K, const void* w, int dtype, int N, void* out,
                           int64_t ld_out, hipStream_t st, bool f32_out, int* splits) {
  if (!x_tiled || !w || !out || M <= 0 || K % 128 || N % (32 * kBigNT) || ld_out < N) return PE_ERR_ARG;
  if (splits) *splits = 1;
  const int mtiles0 = (M + 31) / 32;
  // 256 x 256 tiles from an LDS ring when the tiles fill at least two rounds
  // of one workgroup per CU (offsets within X and W below 4 GiB). With fewer
  // tiles the 128-column kernel, two workgroups per CU, measured faster (a
  // 2047-row drafter context: q/k/v 226 against 258 us, the 4096-column
  // linears 212 against 285; gate/up, 688 tiles, 403 against 442)
  const int mblocks0 = (M + 255) / 256;
  if (M > 256 && N % 256 == 0 && (int64_t)(N / 256) * mblocks0 >= 512 && (int64_t)N * K * 2 < (int64_t(1) << 32) &&
      (int64_t)mtiles0 * 32 * K * 2 < (int64_t(1) << 32)) {
    const int units = K / 128, mblocks = mblocks0;
    const dim3 grid((unsigned)(N / 256 * mblocks), 1);
#define PE_T256_LAUNCH(D, F)                                                                                   \
  dense_gemm_t256_kernel<D, F><<<grid, 256, 0, st>>>((const uint16_t*)x_tiled, (const uint16_t*)w, units, units, \
                                                     mtiles0, mblocks, M, out, ld_out, N)
    if (dtype == PE_DTYPE_BF16 && f32_out)
      PE_T256_LAUNCH(PE_DTYPE_BF16, true);
    else if (dtype == PE_DTYPE_BF16)
      PE_T256_LAUNCH(PE_DTYPE_BF16, false);
    else if (dtype == PE_DTYPE_F16 && f32_out)
      PE_T256_LAUNCH(PE_DTYPE_F16, true);
    else if (dtype == PE_DTYPE_F16)
      PE_T256_LAUNCH(PE_DTYPE_F16, false);
    else
      return PE_ERR_ARG;
#undef PE_T256_LAUNCH
    PE_CHECK_LAUNCH();
    return PE_OK;
  }
  const int np = K / 128;
  const int mtiles = (M + 31) / 32;
  // fp32 partials for a caller that sums splits: two K splits when the column
  // groups x row blocks would fill fewer than two workgroups per CU
  int S = 1;
  if (f32_out && splits && (int64_t)(N / (32 * kBigNT)) * ((mtiles + 7) / 8) < 512 && np >= 4) S = 2;
  if (splits) *splits = S;
  const dim3 grid(N / (32 * kBigNT), (mtiles + 7) / 8, S);
#define PE_DBIGM_LAUNCH(D, F)                                                                             \
  dense_gemm_bigm_kernel<D, F><<<grid, kWaves * 64, 0, st>>>((const uint16_t*)x_tiled, (const uint16_t*)w, np, \
                                                             mtiles, M, out, ld_out)
  if (dtype == PE_DTYPE_BF16 && f32_out)
    PE_DBIGM_LAUNCH(PE_DTYPE_BF16, true);
  else if (dtype == PE_DTYPE_BF16)
    PE_DBIGM_LAUNCH(PE_DTYPE_BF16, false);
  else if (dtype == PE_DTYPE_F16 && f32_out)
    PE_DBIGM_LAUNCH(PE_DTYPE_F16, true);
  else if (dtype == PE_DTYPE_F16)
    PE_DBIGM_LAUNCH(PE_DTYPE_F16, false);
  else
    return PE_ERR_ARG;
#undef PE_DBIGM_LAUNCH
  PE_CHECK_LAUNCH();
  return PE_OK;
}

// The prefill's NF4 linears: all M rows (A-tiled) in blocks of 256 rows on
// grid.z, one K split, each weight dequantised once per row block. SwiGLU
// (out_units > 0, bf16): the activation stored A-tiled; otherwise fp32 sums
// y[M][N] (one split of partials).
int pe_internal_nf4_prefill(const void* x_tiled, int M, int K, const void* w, const void* wabs, int N, float* y,
                            void* act, int out_units, hipStream_t st) {
  if (!x_tiled || !w || !wabs || M <= 0 || K % 128 || N % (32 * kBigNT)) return PE_ERR_ARG;
  if (out_units ? (!act || out_units * 128 != N / 2) : !y) return PE_ERR_ARG;
  const int units = K / 128, groups = N / (32 * kBigNT), mtiles = (M + 31) / 32;
  const dim3 grid(groups, 1, (mtiles + 7) / 8);
  if (out_units) {
    EpiArgs e = make_epi(PE_EPI_SWIGLU, M, N, nullptr, nullptr, 0, act, 0);
    e.out_units = out_units;
    nf4_gemm_bigws_kernel<true><<<grid, kWsWaves * 64, 0, st>>>((const uint16_t*)x_tiled, (const uint8_t*)w,
                                                                (const uint16_t*)wabs, units, units, mtiles, e);
  } else {
    EpiArgs e = make_epi(kEpiPartial, M, N, nullptr, nullptr, 0, y, N);
    nf4_gemm_bigws_kernel<false><<<grid, kWsWaves * 64, 0, st>>>((const uint16_t*)x_tiled, (const uint8_t*)w,
                                                                 (const uint16_t*)wabs, units, units, mtiles, e);
  }
  PE_CHECK_LAUNCH();
  return PE_OK;
}

int pe_internal_nf4_bigm_partials(const void* x_tiled, int M, int K, const void* w, const void* wabs, int N,
                                  float* partial, int64_t partial_bytes, int* splits, hipStream_t st) {
  if (!x_tiled || !w || !wabs || !partial || !splits || M <= 0 || M > 8 * 32 || K % 128 || N % (32 * kBigNT))
    return PE_ERR_ARG;
  const BigPlan p = big_plan(N, K);
  if (partial_bytes < (int64_t)p.S * M * N * 4) return PE_ERR_WORKSPACE;
  EpiArgs e = make_epi(kEpiPartial, M, N, nullptr, nullptr, 0, partial, N);
  *splits = p.S;
  const int mtiles = (M + 31) / 32;
  nf4_gemm_bigws_kernel<false><<<dim3(p.groups, p.S), kWsWaves * 64, 0, st>>>(
      (const uint16_t*)x_tiled, (const uint8_t*)w, (const uint16_t*)wabs, p.units, p.pps, mtiles, e);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

int pe_internal_nf4_bigm_swiglu(const void* x_tiled, int M, int K, const void* w, const void* wabs, int N, void* out,
                                int out_units, int dtype, float* partial, int64_t partial_bytes, int* splits,
                                hipStream_t st) {
  if (!x_tiled || !w || !wabs || !out || !splits || M <= 0 || M > 8 * 32 || K % 128 || N % (32 * kBigNT) ||
      out_units * 128 != N / 2)
    return PE_ERR_ARG;
  const BigPlan p = big_plan(N, K);
  if (p.S > 1 || dtype != PE_DTYPE_BF16)
    return pe_internal_nf4_bigm_partials(x_tiled, M, K, w, wabs, N, partial, partial_bytes, splits, st);
  EpiArgs e = make_epi(PE_EPI_SWIGLU, M, N, nullptr, nullptr, 0, out, 0);
  e.out_units = out_units;
  *splits = 0;
  const int mtiles = (M + 31) / 32;
  nf4_gemm_bigws_kernel<true><<<dim3(p.groups, 1), kWsWaves * 64, 0, st>>>(
      (const uint16_t*)x_tiled, (const uint8_t*)w, (const uint16_t*)wabs, p.units, p.pps, mtiles, e);
  PE_CHECK_LAUNCH();
  return PE_OK;
}

// A dense 16-bit pe_dense_gemm of more than 256 rows without bias or residual
// packs X A-tiled into its workspace and runs the many-row kernel.
static bool dense_many_rows(int M, int N, int K, int epilogue, const void* bias) {
  return M > 4 * kMaxChunkRows && epilogue == PE_EPI_STORE && !bias && K % 128 == 0 && N % (32 * kBigNT) == 0;
}

extern "C" int64_t pe_gemm_workspace_bytes(int M, int N, int K, int wfmt, int dtype, int epilogue) {
  if (dtype == PE_DTYPE_F32 && wfmt == PE_WFMT_DENSE) return 0;
  // the packed rows go after the counters, which other calls sharing the workspace rely on
  if (wfmt == PE_WFMT_DENSE && dense_many_rows(M, N, K, epilogue, nullptr)) return kCounterBytes + xtile_bytes(M, K);
  if (M <= 0 || N <= 0 || K < 128) return kCounterBytes;
  // M runs as 64-row launches plus a shorter last one, whose plan (one M tile
  // instead of two) can need more split partials; the many-row SwiGLU linear
  // of pe_nf4_gemm_tiled needs its split partials when its plan splits K
  const bool nf4 = pe_wfmt_nf4(wfmt);
  const int64_t big = nf4 && epilogue == PE_EPI_SWIGLU && M > kMaxChunkRows && M <= 8 * 32
                          ? pe_internal_nf4_bigm_partials_bytes(M, N, K)
                          : 0;
  const int mc = M > kMaxChunkRows ? kMaxChunkRows : M;
  int64_t w = workspace_of(make_plan(mc, N, K, nf4, epilogue));
  const int rem = M % kMaxChunkRows;
  if (M > kMaxChunkRows && rem) {
    const int64_t wr = workspace_of(make_plan(rem, N, K, nf4, epilogue));
    if (wr > w) w = wr;
  }
  return w > big ? w : big;
}

extern "C" int pe_nf4_gemm(const void* x, int64_t ldx, int M, int K, const uint8_t* w_tiled,
                           const uint16_t* absmax_tiled, int N, int epilogue, const void* bias,
                           const void* resid, int64_t ld_resid, void* out, int64_t ld_out, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  if (!absmax_tiled) return PE_ERR_ARG;
  return mfma_gemm(kFmtNF4, x, ldx, M, K, w_tiled, absmax_tiled, N, epilogue, bias, resid, ld_resid, out,
                   ld_out, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int pe_nf4_gemm_f32abs(const void* x, int64_t ldx, int M, int K, const uint8_t* w_tiled,
                                  const float* absmax_tiled, int N, int epilogue, const void* bias,
                                  const void* resid, int64_t ld_resid, void* out, int64_t ld_out, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  if (!absmax_tiled) return PE_ERR_ARG;
  return mfma_gemm(kFmtNF4F32, x, ldx, M, K, w_tiled, absmax_tiled, N, epilogue, bias, resid, ld_resid, out,
                   ld_out, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int pe_nf4_gemm_tiled(const void* x_tiled, int M, int K, const uint8_t* w_tiled,
                                 const uint16_t* absmax_tiled, int N, int epilogue, const void* bias,
                                 const void* resid, int64_t ld_resid, void* out, int64_t ld_out, int out_units,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  if (!absmax_tiled || out_units < 0) return PE_ERR_ARG;
  if (M > kMaxChunkRows) {
    // many rows: the gate/up linear of the batched pass (A-tiled activation out)
    if (M > 8 * 32 || epilogue != PE_EPI_SWIGLU || bias || out_units * 256 != N) return PE_ERR_ARG;
    int S = 0;
    const hipStream_t st = (hipStream_t)stream;
    int rc = pe_internal_nf4_bigm_swiglu(x_tiled, M, K, w_tiled, absmax_tiled, N, out, out_units, PE_DTYPE_BF16,
                                         (float*)workspace, workspace_bytes, &S, st);
    if (rc == PE_OK && S > 0)
      rc = pe_internal_swiglu_partials((const float*)workspace, S, M, N, out, ld_out, out_units, PE_DTYPE_BF16, st);
    return rc;
  }
  return mfma_gemm(kFmtNF4, x_tiled, K, M, K, w_tiled, absmax_tiled, N, epilogue, bias, resid, ld_resid, out, ld_out,
                   workspace, workspace_bytes, (hipStream_t)stream, true, out_units);
}

extern "C" int64_t pe_nf4_gemm_partials_bytes(int M, int N, int K) {
  if (M > kMaxChunkRows && M <= 8 * 32) return pe_internal_nf4_bigm_partials_bytes(M, N, K);
  if (M <= 0 || M > kMaxChunkRows || N <= 0 || K < 128) return 0;
  return pe_internal_linear_partials_bytes(M, N, K, PE_WFMT_NF4);
}

extern "C" int pe_nf4_gemm_partials(const void* x, int64_t ldx, int x_tiled, int M, int K, const uint8_t* w_tiled,
                                    const uint16_t* absmax_tiled, int N, float* partials, int64_t partial_bytes,
                                    int* splits, void* stream) {
  if (M > kMaxChunkRows) {  // the many-row kernel: A-tiled X, N % 128 == 0
    if (!x_tiled) return PE_ERR_ARG;
    return pe_internal_nf4_bigm_partials(x, M, K, w_tiled, absmax_tiled, N, partials, partial_bytes, splits,
                                         (hipStream_t)stream);
  }
  return pe_internal_linear_partials(PE_WFMT_NF4, PE_DTYPE_BF16, x, x_tiled ? K : ldx, x_tiled != 0, M, K, w_tiled,
                                     absmax_tiled, N, partials, partial_bytes, splits, (hipStream_t)stream);
}

extern "C" int pe_dense_gemm_argmax_groups(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K < 128 || K % 128 || N % 32) return 0;
  return make_plan(M > kMaxChunkRows ? kMaxChunkRows : M, N, K, false, kEpiArgmax).groups;
}

// The lm_head of the fused pass over its A-tiled final norm rows (M <= 64):
// the logits stored in the dtype and, with keys, each row's argmax keys.
int pe_internal_dense_gemm_tiled(const void* x_tiled, int M, int K, const void* w, int dtype, int N, void* out,
                                 int64_t ld_out, uint64_t* keys, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16) return PE_ERR_ARG;
  return mfma_gemm(dtype, x_tiled, 0, M, K, w, nullptr, N, PE_EPI_STORE, nullptr, nullptr, 0, out, ld_out, ws,
                   ws_bytes, st, true, 0, keys);
}

extern "C" int pe_dense_gemm_argmax(const void* x, int64_t ldx, int M, int K, const void* w, int dtype, int N,
                                    void* out, int64_t ld_out, uint64_t* keys, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  if (!keys || (dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16)) return PE_ERR_ARG;
  return mfma_gemm(dtype, x, ldx, M, K, w, nullptr, N, PE_EPI_STORE, nullptr, nullptr, 0, out, ld_out, workspace,
                   workspace_bytes, (hipStream_t)stream, false, 0, keys);
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
    EpiArgs e = make_epi(epilogue, M, N, bias, resid, ld_resid, out, ld_out);
    const int n_out = epilogue == PE_EPI_SWIGLU ? N / 2 : N;
    dim3 grid((n_out + 3) / 4, (M + 7) / 8);
    if (epilogue == PE_EPI_SWIGLU)
      f32_gemm_kernel<true><<<grid, 256, 0, st>>>((const float*)x, ldx, M, K, (const float*)w, n_out, e);
    else
      f32_gemm_kernel<false><<<grid, 256, 0, st>>>((const float*)x, ldx, M, K, (const float*)w, n_out, e);
    PE_CHECK_LAUNCH();
    return PE_OK;
  }
  if (dtype != PE_DTYPE_BF16 && dtype != PE_DTYPE_F16) return PE_ERR_ARG;
  if (dense_many_rows(M, N, K, epilogue, bias) && workspace && workspace_bytes >= kCounterBytes + xtile_bytes(M, K)) {
    // every weight read once per 256 rows instead of once per 64-row launch;
    // the A-tiled rows after the workspace's counters
    if (!x || !w || !out || ld_out < N || ldx < K) return PE_ERR_ARG;
    void* xt = (char*)workspace + kCounterBytes;
    int rc = pe_internal_to_xtile(x, ldx, M, K, xt, st);
    if (rc != PE_OK) return rc;
    return pe_internal_dense_bigm(xt, M, K, w, dtype, N, out, ld_out, st);
  }
  return mfma_gemm(dtype, x, ldx, M, K, w, nullptr, N, epilogue, bias, resid, ld_resid, out, ld_out, workspace,
                   workspace_bytes, st);
}
