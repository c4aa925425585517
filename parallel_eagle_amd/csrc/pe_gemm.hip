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
//   * prefetch the next iteration's weights and X fragments into registers
//     before computing the current one;
//   * split K across the waves of a workgroup (reduced in LDS, fixed order)
//     and, when there are too few column tiles to fill 256 CUs, across S
//     workgroups. Split-K workgroups never synchronise with each other (a
//     device-scope fence costs more than a kernel boundary on a multi-XCD
//     part): each writes an fp32 partial [split][M][N], and the consumer sums
//     the S partials in split order. The consumer is either the reduction
//     kernel here (pe_nf4_gemm / pe_dense_gemm) or, inside pe_forward, the next
//     kernel of the layer (attention prologue, residual + RMSNorm). Results are
//     deterministic and independent of M.
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

constexpr int64_t kGemmWsAlign = 256;
// Internal epilogues: write the fp32 accumulators to partial[split] even when
// S == 1; and the q/k/v projection with bias, RoPE and the in-place KV append.
constexpr int kEpiPartial = 3;
constexpr int kEpiRopeKV = 4;

struct EpiArgs {
  int op;
  int M;
  int N;  // GEMM columns
  const void* bias;
  const void* resid;
  int64_t ld_resid;
  void* out;
  int64_t ld_out;
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
  int nh, nkv, hd;
  int32_t* status;
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
template <int DT>
__device__ __forceinline__ void write_rope_kv(const EpiArgs& e, int group, int row, float a1, float a2) {
  typedef Elem<DT> E;
  typedef typename E::T T;
  const int lane = threadIdx.x & 63, ln = lane & 31;
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
  if (u >= e.nh + e.nkv) {  // v: appended as is
    T* dst = (T*)e.v_cache + ((int64_t)(u - e.nh - e.nkv) * e.cap + e.row0 + row) * e.hd;
    E::store(dst, d1, x1);
    E::store(dst, d2, x2);
    return;
  }
  const int64_t p = e.positions[row];
  if (p < 0 || p >= e.max_pos) {
    if (e.status) atomicOr(e.status, PE_ERR_CAPACITY);
    return;
  }
  const T* cosr = (const T*)e.cos_sin + p * e.hd;
  const T* sinr = (const T*)e.cos_sin + (e.max_pos + p) * e.hd;
  const float o1 = __fadd_rn(E::round(__fmul_rn(x1, E::load(cosr, d1))), E::round(__fmul_rn(-x2, E::load(sinr, d1))));
  const float o2 = __fadd_rn(E::round(__fmul_rn(x2, E::load(cosr, d2))), E::round(__fmul_rn(x1, E::load(sinr, d2))));
  T* dst = (u < e.nh) ? (T*)e.q_out + ((int64_t)row * e.nh + u) * e.hd
                      : (T*)e.k_cache + ((int64_t)(u - e.nh) * e.cap + e.row0 + row) * e.hd;
  E::store(dst, d1, o1);
  E::store(dst, d2, o2);
}

// Output of a GEMM workgroup, after its waves' K slices are summed.
//   S == 1: the epilogue writes the final values.
//   S > 1: rows < M of the tile go to partial[split][M][N] (fp32).
template <int ADT, int NT, int MT>
__device__ __forceinline__ void write_tile(f32x16_t (&acc)[NT][MT], int group, int split, int S,
                                           float* __restrict__ partial, const EpiArgs& e) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5, ln = lane & 31;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = mt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
      if (row >= e.M) continue;
      if (S > 1 || e.op == kEpiPartial) {
        float* prow = partial + ((int64_t)split * e.M + row) * e.N;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) prow[(group * NT + nt) * 32 + ln] = acc[nt][mt][r];
      } else if (e.op == PE_EPI_SWIGLU) {
        if constexpr (NT == 2) epi_swiglu<ADT>(e, row, group * 32 + ln, acc[0][mt][r], acc[1][mt][r]);
      } else if (e.op == kEpiRopeKV) {
        if constexpr (NT == 2) write_rope_kv<ADT>(e, group, row, acc[0][mt][r], acc[1][mt][r]);
      } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) epi_value<ADT>(e, row, (group * NT + nt) * 32 + ln, acc[nt][mt][r]);
      }
    }
  }
}

// Sum the waves' K slices in LDS in wave order, then wave 0 writes the tile.
// `red` needs (WAVES - 1) * 16 * 64 floats; the caller has synchronised the
// workgroup if that memory had another use.
template <int ADT, int NT, int MT, int WAVES>
__device__ __forceinline__ void reduce_waves_and_write(f32x16_t (&acc)[NT][MT], float* red, int group, int split,
                                                       int S, float* __restrict__ partial, const EpiArgs& e) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[((wave - 1) * 16 + r) * 64 + lane] = acc[nt][mt][r];
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int w = 0; w < WAVES - 1; ++w)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[nt][mt][r] += red[(w * 16 + r) * 64 + lane];
      }
      __syncthreads();
    }
  }
  if (wave == 0) write_tile<ADT, NT, MT>(acc, group, split, S, partial, e);
}

// ---------------------------------------------------------------------------
// NF4 lookup primitive (gfx950 assembly)
// ---------------------------------------------------------------------------
// One MFMA k-step of NT tiles: the 8 codes of q[nt] become 8 bf16 table
// entries, packed in pairs into the MFMA operand. Address updates, loads and
// the wait are one asm block, so the compiler never touches a register whose
// load is still in flight; every load is issued at least 8 instructions after
// the SDWA that wrote its address. The loads are plain zero-extending
// ds_read_u16: with SRAM ECC enabled (the MI355X default) d16 loads clear the
// other half of the register instead of preserving it, so the two halves are
// joined with one v_lshl_or after the wait.
#define PE_SDWA_LO(a, q, byte) \
  "v_and_b32_sdwa " a ", 15, " q " dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_" byte "\n\t"
#define PE_SDWA_HI(a, q, byte) \
  "v_lshrrev_b32_sdwa " a ", 4, " q " dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:BYTE_" byte "\n\t"
#define PE_ADDR8(A, Q)                                                                                    \
  PE_SDWA_LO("%[" A "0]", "%[" Q "]", "0") PE_SDWA_HI("%[" A "1]", "%[" Q "]", "0")                     \
  PE_SDWA_LO("%[" A "2]", "%[" Q "]", "1") PE_SDWA_HI("%[" A "3]", "%[" Q "]", "1")                     \
  PE_SDWA_LO("%[" A "4]", "%[" Q "]", "2") PE_SDWA_HI("%[" A "5]", "%[" Q "]", "2")                     \
  PE_SDWA_LO("%[" A "6]", "%[" Q "]", "3") PE_SDWA_HI("%[" A "7]", "%[" Q "]", "3")
#define PE_READ1(D, A, O) "ds_read_u16 %[" D "], %[" A "] offset:%[" O "]\n\t"
#define PE_READ8(D, A, O)                                                                                    \
  PE_READ1(D "0", A "0", O) PE_READ1(D "1", A "1", O) PE_READ1(D "2", A "2", O) PE_READ1(D "3", A "3", O)     \
  PE_READ1(D "4", A "4", O) PE_READ1(D "5", A "5", O) PE_READ1(D "6", A "6", O) PE_READ1(D "7", A "7", O)

__device__ __forceinline__ uint32_t pack16(uint32_t lo, uint32_t hi) { return lo | (hi << 16); }

template <int NT, int OFF0, int OFF1>
__device__ __forceinline__ void nf4_lookup_step(const uint32_t (&q)[NT], uint32_t (&a)[NT][8], u32x4_t (&bv)[NT]) {
  uint32_t x[8];
  if constexpr (NT == 2) {
    uint32_t y[8];
    asm volatile(PE_ADDR8("a", "q0") PE_ADDR8("c", "q1") PE_READ8("x", "a", "o0") PE_READ8("y", "c", "o1")
                 "s_waitcnt lgkmcnt(0)"
                 : [x0] "=&v"(x[0]), [x1] "=&v"(x[1]), [x2] "=&v"(x[2]), [x3] "=&v"(x[3]), [x4] "=&v"(x[4]),
                   [x5] "=&v"(x[5]), [x6] "=&v"(x[6]), [x7] "=&v"(x[7]), [y0] "=&v"(y[0]), [y1] "=&v"(y[1]),
                   [y2] "=&v"(y[2]), [y3] "=&v"(y[3]), [y4] "=&v"(y[4]), [y5] "=&v"(y[5]), [y6] "=&v"(y[6]),
                   [y7] "=&v"(y[7]), [a0] "+v"(a[0][0]), [a1] "+v"(a[0][1]), [a2] "+v"(a[0][2]),
                   [a3] "+v"(a[0][3]), [a4] "+v"(a[0][4]), [a5] "+v"(a[0][5]), [a6] "+v"(a[0][6]),
                   [a7] "+v"(a[0][7]), [c0] "+v"(a[1][0]), [c1] "+v"(a[1][1]), [c2] "+v"(a[1][2]),
                   [c3] "+v"(a[1][3]), [c4] "+v"(a[1][4]), [c5] "+v"(a[1][5]), [c6] "+v"(a[1][6]),
                   [c7] "+v"(a[1][7])
                 : [q0] "v"(q[0]), [q1] "v"(q[1]), [o0] "i"(OFF0), [o1] "i"(OFF1)
                 : "memory");
    bv[1] = u32x4_t{pack16(y[0], y[1]), pack16(y[2], y[3]), pack16(y[4], y[5]), pack16(y[6], y[7])};
  } else {
    asm volatile(PE_ADDR8("a", "q0") PE_READ8("x", "a", "o0") "s_waitcnt lgkmcnt(0)"
                 : [x0] "=&v"(x[0]), [x1] "=&v"(x[1]), [x2] "=&v"(x[2]), [x3] "=&v"(x[3]), [x4] "=&v"(x[4]),
                   [x5] "=&v"(x[5]), [x6] "=&v"(x[6]), [x7] "=&v"(x[7]), [a0] "+v"(a[0][0]), [a1] "+v"(a[0][1]),
                   [a2] "+v"(a[0][2]), [a3] "+v"(a[0][3]), [a4] "+v"(a[0][4]), [a5] "+v"(a[0][5]),
                   [a6] "+v"(a[0][6]), [a7] "+v"(a[0][7])
                 : [q0] "v"(q[0]), [o0] "i"(OFF0)
                 : "memory");
  }
  bv[0] = u32x4_t{pack16(x[0], x[1]), pack16(x[2], x[3]), pack16(x[4], x[5]), pack16(x[6], x[7])};
}
#undef PE_READ8
#undef PE_READ1
#undef PE_ADDR8
#undef PE_SDWA_HI
#undef PE_SDWA_LO

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// The lane's 16 table entries bf16_rne(NF4[c] * scale), entry c at lane base + 256 c + OFF.
template <int OFF>
__device__ __forceinline__ void nf4_build_table(uint8_t* lanetab, uint16_t absmax) {
  const float sc = f16_bits_to_f32(absmax);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f32x2_t v = {kNF4[2 * i] * sc, kNF4[2 * i + 1] * sc};
    const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    *(uint16_t*)(lanetab + (2 * i) * 256 + OFF) = (uint16_t)w;
    *(uint16_t*)(lanetab + (2 * i + 1) * 256 + OFF) = (uint16_t)(w >> 16);
  }
}

constexpr int kTabTile = 16 * 64 * 4;  // one tile's table: 16 codes x 64 lanes x dword (2 slots)

template <int MT, int NT>
struct NF4Regs {
  u32x4_t q[NT][2];  // codes of the lane's block in each tile (dword s = MFMA k-step s)
  u32x4_t x[MT][8];  // X fragments of the 8 MFMA k-steps
  uint16_t a[NT];    // absmax of the lane's block in each tile
};

// One wave's share of a workgroup's block-pair range; WV = this wave's index
// (compile time, so table offsets are immediates). Codes, absmax and X
// fragments of the next block pair are loaded into a second register set
// while the current pair is computed; tables alternate between the two
// 16-bit slots of each entry.
template <int MT, int NT, int WAVES, int WV>
__device__ __forceinline__ void nf4_wave_body(f32x16_t (&acc)[NT][MT], uint8_t* smem,
                                              const uint16_t* __restrict__ X, int64_t ldx,
                                              const uint8_t* __restrict__ W, const uint16_t* __restrict__ Wabs,
                                              int NP, int group, int w0, int w1, int M) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5, ln = lane & 31;
  constexpr int TB = WV * NT * kTabTile;  // this wave's table area
  uint8_t* lanetab = smem + lane * 4;
  // LDS address registers: the lane's table base in the low byte (the kernel's
  // only LDS object starts at offset 0, so bits 8..15 are free for the code).
  uint32_t addr[NT][8];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int i = 0; i < 8; ++i) addr[nt][i] = (uint32_t)(lane * 4);

  // Rows at or beyond M read row M - 1: MFMA rows are independent and those
  // output rows are never stored, so no masking is needed.
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = X + (int64_t)min(mt * 32 + ln, M - 1) * ldx + 64 * g;

  auto load = [&](NF4Regs<MT, NT>& R, int p) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int64_t ts = (int64_t)(group * NT + nt) * NP + p;
      const uint8_t* wp = W + ts * 2048 + lane * 16;
      R.q[nt][0] = *(const u32x4_t*)(wp);
      R.q[nt][1] = *(const u32x4_t*)(wp + 1024);
      R.a[nt] = Wabs[ts * 64 + lane];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < 8; ++s) R.x[mt][s] = *(const u32x4_t*)(xrow[mt] + 128 * p + 8 * s);
  };
  auto compute = [&](const NF4Regs<MT, NT>& R, auto slot_c) {
    constexpr int SL = decltype(slot_c)::value;
    nf4_build_table<TB + SL>(lanetab, R.a[0]);
    if constexpr (NT == 2) nf4_build_table<TB + kTabTile + SL>(lanetab, R.a[1]);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      uint32_t qs[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) qs[nt] = R.q[nt][s >> 2][s & 3];
      u32x4_t bv[NT];
      nf4_lookup_step<NT, TB + SL, TB + kTabTile + SL>(qs, addr, bv);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16<PE_DTYPE_BF16>(R.x[mt][s], bv[nt], acc[nt][mt]);
    }
  };

  NF4Regs<MT, NT> A, B;
  if (w0 < w1) load(A, w0);
  for (int p = w0; p < w1; p += 2) {
    if (p + 1 < w1) load(B, p + 1);
    compute(A, std::integral_constant<int, 0>());
    if (p + 1 >= w1) break;
    if (p + 2 < w1) load(A, p + 2);
    compute(B, std::integral_constant<int, 2>());
  }
}

template <int MT, int NT, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void nf4_gemm_kernel(const uint16_t* __restrict__ X, int64_t ldx,
                                                              const uint8_t* __restrict__ W,
                                                              const uint16_t* __restrict__ Wabs, int NP, int S,
                                                              int pps, float* __restrict__ partial, EpiArgs e) {
  constexpr int kTabBytes = WAVES * NT * kTabTile;
  constexpr int kRedBytes = (WAVES - 1) * 16 * 64 * 4;
  static_assert(kTabBytes <= 65536, "table offsets must fit the 16-bit LDS immediate");
  __shared__ __align__(256) uint8_t smem[kTabBytes > kRedBytes ? kTabBytes : kRedBytes];
  const int group = blockIdx.x, split = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p0 = split * pps;
  const int p1 = min(NP, p0 + pps);
  const int np = max(0, p1 - p0);
  const int w0 = p0 + (np * wave) / WAVES;
  const int w1 = p0 + (np * (wave + 1)) / WAVES;

  f32x16_t acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nt][mt][r] = 0.f;

  switch (wave) {
#define PE_WAVE_CASE(i)                                                                              \
  case i:                                                                                            \
    if constexpr (i < WAVES) nf4_wave_body<MT, NT, WAVES, i>(acc, smem, X, ldx, W, Wabs, NP, group, w0, w1, e.M); \
    break;
    PE_WAVE_CASE(0)
    PE_WAVE_CASE(1)
    PE_WAVE_CASE(2)
    PE_WAVE_CASE(3)
    PE_WAVE_CASE(4)
    PE_WAVE_CASE(5)
    PE_WAVE_CASE(6)
    PE_WAVE_CASE(7)
#undef PE_WAVE_CASE
    default:
      break;
  }
  __syncthreads();  // every wave is done with its tables; smem becomes the reduction buffer
  reduce_waves_and_write<PE_DTYPE_BF16, NT, MT, WAVES>(acc, (float*)smem, group, split, S, partial, e);
}

// ---------------------------------------------------------------------------
// Dense 16-bit: one iteration = 4 MFMA k-steps (64 along K) of NT column tiles.
// ---------------------------------------------------------------------------
template <int FMT, int MT, int NT>
__global__ __launch_bounds__(256) void dense_gemm_kernel(const uint16_t* __restrict__ X, int64_t ldx, int K,
                                                         const uint16_t* __restrict__ W, int S, int ups,
                                                         float* __restrict__ partial, EpiArgs e) {
  constexpr int WAVES = 4;
  __shared__ __align__(16) float red[(WAVES - 1) * 16 * 64];
  const int group = blockIdx.x, split = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 5, ln = lane & 31;
  const int NU = K >> 6, KS = K >> 4;
  const int u0 = split * ups;
  const int u1 = min(NU, u0 + ups);
  const int nu = max(0, u1 - u0);
  const int w0 = u0 + (nu * wave) / WAVES;
  const int w1 = u0 + (nu * (wave + 1)) / WAVES;

  f32x16_t acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nt][mt][r] = 0.f;

  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = X + (int64_t)min(mt * 32 + ln, e.M - 1) * ldx + 8 * g;

  u32x4_t bn[NT][4], xn[MT][4];
  auto load = [&](int u) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bn[nt][j] = *(const u32x4_t*)(W + (((int64_t)(group * NT + nt) * KS + 4 * u + j) * 64 + lane) * 8);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) xn[mt][j] = *(const u32x4_t*)(xrow[mt] + 64 * u + 16 * j);
  };

  if (w0 < w1) load(w0);
  for (int u = w0; u < w1; ++u) {
    u32x4_t bc[NT][4], xc[MT][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) bc[nt][j] = bn[nt][j];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xc[mt][j] = xn[mt][j];
    }
    if (u + 1 < w1) load(u + 1);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16<FMT>(xc[mt][j], bc[nt][j], acc[nt][mt]);
  }
  reduce_waves_and_write<FMT, NT, MT, WAVES>(acc, red, group, split, S, partial, e);
}

// Sum S fp32 partials [S][M][N] in split order, then the epilogue. One thread
// per output (swiglu: per gate/up pair).
template <int DT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partial, int S, EpiArgs e) {
  const int n_out = e.op == PE_EPI_SWIGLU ? e.N / 2 : e.N;
  const int64_t total = (int64_t)e.M * n_out;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int row = (int)(i / n_out), col = (int)(i % n_out);
    if (e.op == PE_EPI_SWIGLU) {
      const int gcol = (col >> 5) * 64 + (col & 31);
      float gv = 0.f, uv = 0.f;
      for (int s = 0; s < S; ++s) {
        const float* p = partial + ((int64_t)s * e.M + row) * e.N;
        gv += p[gcol];
        uv += p[gcol + 32];
      }
      epi_swiglu<DT>(e, row, col, gv, uv);
    } else {
      float v = 0.f;
      for (int s = 0; s < S; ++s) v += partial[((int64_t)s * e.M + row) * e.N + col];
      epi_value<DT>(e, row, col, v);
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

// ---------------------------------------------------------------------------
// Launch planning
// ---------------------------------------------------------------------------
constexpr int kMaxChunkRows = 64;  // M rows per launch (MT <= 2)
constexpr int kMaxSplits = 16;     // split-K partials a consumer sums (residual RMSNorm's limit)

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v ? atoi(v) : dflt;
}

struct Plan {
  int NT, MT, S, per_split, groups, units, waves;
  int64_t partial_bytes;  // [S][M][N] fp32 when S > 1
};

// units: block pairs (NF4) or 64-wide K steps (dense). With allow_split false
// the GEMM covers all of K in one workgroup per column group (S == 1);
// otherwise S gives about `target_wg` workgroups (one per CU).
Plan make_plan(int M, int N, int K, bool nf4, int epi, bool allow_split) {
  static const int target_wg = env_int("PE_GEMM_TARGET_WG", 256);
  Plan p;
  p.NT = (epi == PE_EPI_SWIGLU || N % 64 == 0) ? 2 : 1;
  p.MT = M > 32 ? 2 : 1;
  p.groups = N / (32 * p.NT);
  p.units = nf4 ? K / 128 : K / 64;
  int S = allow_split ? (target_wg + p.groups - 1) / p.groups : 1;
  // An unsplit NF4 GEMM with few column groups splits K over 8 waves instead of 4.
  // (only when the workgroups fit in one round at one 8-wave workgroup per CU)
  static const int wide_groups = env_int("PE_GEMM_WIDE_GROUPS", 257);
  p.waves = (nf4 && S <= 1 && p.groups < wide_groups && p.units >= 16) ? 8 : 4;
  const int waves = p.waves;
  int smax = p.units / waves;
  if (smax < 1) smax = 1;
  if (S > smax) S = smax;
  if (S > kMaxSplits) S = kMaxSplits;
  if (S < 1) S = 1;
  p.per_split = (p.units + S - 1) / S;
  p.S = (p.units + p.per_split - 1) / p.per_split;
  p.partial_bytes = (p.S > 1) ? (int64_t)p.S * M * N * 4 : 0;
  return p;
}

// fmt: -1 = NF4 (bf16 compute), else PE_DTYPE_BF16 / PE_DTYPE_F16 dense.
int launch_gemm(int fmt, const Plan& p, hipStream_t st, const uint16_t* x, int64_t ldx, int K, const void* w,
                const uint16_t* wabs, float* partial, const EpiArgs& e) {
  dim3 grid(p.groups, p.S);
  if (fmt < 0) {
#define PE_NF4(MT_, NT_, WV_)                                                                              \
  nf4_gemm_kernel<MT_, NT_, WV_><<<grid, WV_ * 64, 0, st>>>(x, ldx, (const uint8_t*)w, wabs, p.units, p.S, \
                                                           p.per_split, partial, e)
    if (p.waves == 8) {
      if (p.NT == 2) { if (p.MT == 1) PE_NF4(1, 2, 8); else PE_NF4(2, 2, 8); }
      else { if (p.MT == 1) PE_NF4(1, 1, 8); else PE_NF4(2, 1, 8); }
    } else {
      if (p.NT == 2) { if (p.MT == 1) PE_NF4(1, 2, 4); else PE_NF4(2, 2, 4); }
      else { if (p.MT == 1) PE_NF4(1, 1, 4); else PE_NF4(2, 1, 4); }
    }
#undef PE_NF4
  } else {
#define PE_DENSE(F, MT_, NT_)                                                                                 \
  dense_gemm_kernel<F, MT_, NT_><<<grid, 256, 0, st>>>(x, ldx, K, (const uint16_t*)w, p.S, p.per_split, partial, \
                                                       e)
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
  e.positions = nullptr;
  e.cos_sin = nullptr;
  e.max_pos = 0;
  e.q_out = e.k_cache = e.v_cache = nullptr;
  e.cap = e.row0 = 0;
  e.nh = e.nkv = e.hd = 0;
  e.status = nullptr;
  return e;
}

// The standalone GEMM: split-K partials (if any) are summed by splitk_reduce_kernel.
int mfma_gemm(int fmt, const void* x, int64_t ldx, int M, int K, const void* w, const uint16_t* wabs, int N,
              int epi, const void* bias, const void* resid, int64_t ld_resid, void* out, int64_t ld_out,
              void* ws, int64_t ws_bytes, hipStream_t st) {
  int rc = check_gemm_args(x, M, K, w, N, epi, resid, out);
  if (rc != PE_OK) return rc;
  const bool nf4 = fmt < 0;
  const int adt = nf4 ? PE_DTYPE_BF16 : fmt;
  int done = 0;
  while (done < M) {
    const int mc = (M - done > kMaxChunkRows) ? kMaxChunkRows : (M - done);
    Plan p = make_plan(mc, N, K, nf4, epi, true);
    if (p.S > 1 && (!ws || ws_bytes < p.partial_bytes)) return PE_ERR_WORKSPACE;
    const size_t esz = 2;
    EpiArgs e = make_epi(epi, mc, N, bias, resid ? (const char*)resid + (size_t)done * ld_resid * esz : nullptr,
                         ld_resid, (char*)out + (size_t)done * ld_out * esz, ld_out);
    const uint16_t* xc = (const uint16_t*)x + (size_t)done * ldx;
    rc = launch_gemm(fmt, p, st, xc, ldx, K, w, wabs, (float*)ws, e);
    if (rc != PE_OK) return rc;
    if (p.S > 1) {
      const int n_out = epi == PE_EPI_SWIGLU ? N / 2 : N;
      int blocks = (int)(((int64_t)mc * n_out + 255) / 256);
      if (blocks > 4096) blocks = 4096;
      if (adt == PE_DTYPE_F16) splitk_reduce_kernel<PE_DTYPE_F16><<<blocks, 256, 0, st>>>((const float*)ws, p.S, e);
      else splitk_reduce_kernel<PE_DTYPE_BF16><<<blocks, 256, 0, st>>>((const float*)ws, p.S, e);
      PE_CHECK_LAUNCH();
    }
    done += mc;
  }
  return PE_OK;
}

constexpr int kFmtNF4 = -1;

}  // namespace

// Internal entries used by pe_forward (one launch over M <= 64 rows of a
// 16-bit dtype). pe_internal_gemm_partials always writes fp32 partials
// [S][M][N] to `partial` (S >= 1, reported in S_out) for a consumer kernel to
// sum; pe_internal_gemm_epilogue covers all of K in each workgroup and applies
// the epilogue itself.
int pe_internal_gemm_partials(int wfmt, int dtype, const void* x, int64_t ldx, int M, int K, const void* w,
                              const uint16_t* wabs, int N, float* partial, int64_t partial_bytes, int* S_out,
                              hipStream_t st) {
  if (M > kMaxChunkRows || !partial) return PE_ERR_ARG;
  int rc = check_gemm_args(x, M, K, w, N, PE_EPI_STORE, nullptr, partial);
  if (rc != PE_OK) return rc;
  const bool nf4 = wfmt == PE_WFMT_NF4;
  Plan p = make_plan(M, N, K, nf4, PE_EPI_STORE, true);
  if (partial_bytes < (int64_t)p.S * M * N * 4) return PE_ERR_WORKSPACE;
  EpiArgs e = make_epi(kEpiPartial, M, N, nullptr, nullptr, 0, partial, N);
  *S_out = p.S;
  return launch_gemm(nf4 ? kFmtNF4 : dtype, p, st, (const uint16_t*)x, ldx, K, w, wabs, partial, e);
}

int pe_internal_gemm_epilogue(int wfmt, int dtype, const void* x, int64_t ldx, int M, int K, const void* w,
                              const uint16_t* wabs, int N, int epi, const void* bias, const void* resid,
                              int64_t ld_resid, void* out, int64_t ld_out, hipStream_t st) {
  if (M > kMaxChunkRows) return PE_ERR_ARG;
  int rc = check_gemm_args(x, M, K, w, N, epi, resid, out);
  if (rc != PE_OK) return rc;
  const bool nf4 = wfmt == PE_WFMT_NF4;
  Plan p = make_plan(M, N, K, nf4, epi, false);
  EpiArgs e = make_epi(epi, M, N, bias, resid, ld_resid, out, ld_out);
  return launch_gemm(nf4 ? kFmtNF4 : dtype, p, st, (const uint16_t*)x, ldx, K, w, wabs, nullptr, e);
}

// The q/k/v projection with its RoPE + KV-append epilogue (weight rows in
// head-paired tile order; hd % 64 == 0). Covers all of K per workgroup.
int pe_internal_gemm_rope_kv(int wfmt, int dtype, const void* x, int64_t ldx, int M, int K, const void* w,
                             const uint16_t* wabs, int nh, int nkv, int hd, const void* bias,
                             const int64_t* positions, const void* cos_sin, int64_t max_pos, void* q_out,
                             void* k_cache, void* v_cache, int64_t cap, int64_t row0, int32_t* status,
                             hipStream_t st) {
  const int N = (nh + 2 * nkv) * hd;
  if (M > kMaxChunkRows || hd % 64 || !positions || !cos_sin || !q_out || !k_cache || !v_cache) return PE_ERR_ARG;
  if (row0 < 0 || row0 + M > cap) return PE_ERR_CAPACITY;
  int rc = check_gemm_args(x, M, K, w, N, PE_EPI_SWIGLU, nullptr, q_out);
  if (rc != PE_OK) return rc;
  const bool nf4 = wfmt == PE_WFMT_NF4;
  Plan p = make_plan(M, N, K, nf4, PE_EPI_SWIGLU, false);  // NT = 2, S = 1
  EpiArgs e = make_epi(kEpiRopeKV, M, N, bias, nullptr, 0, nullptr, 0);
  e.positions = positions;
  e.cos_sin = cos_sin;
  e.max_pos = max_pos;
  e.q_out = q_out;
  e.k_cache = k_cache;
  e.v_cache = v_cache;
  e.cap = cap;
  e.row0 = row0;
  e.nh = nh;
  e.nkv = nkv;
  e.hd = hd;
  e.status = status;
  return launch_gemm(nf4 ? kFmtNF4 : dtype, p, st, (const uint16_t*)x, ldx, K, w, wabs, nullptr, e);
}

int64_t pe_internal_gemm_partial_bytes(int M, int N, int K, int wfmt) {
  if (M > kMaxChunkRows) M = kMaxChunkRows;
  const Plan p = make_plan(M, N, K, wfmt == PE_WFMT_NF4, PE_EPI_STORE, true);
  return (int64_t)p.S * M * N * 4;
}

extern "C" int64_t pe_gemm_workspace_bytes(int M, int N, int K, int wfmt, int dtype, int epilogue) {
  if (dtype == PE_DTYPE_F32 && wfmt == PE_WFMT_DENSE) return 0;
  if (M <= 0 || N <= 0 || K < 128) return kGemmWsAlign;
  const int mc = M > kMaxChunkRows ? kMaxChunkRows : M;
  const int64_t b = make_plan(mc, N, K, wfmt == PE_WFMT_NF4, epilogue, true).partial_bytes;
  return b > kGemmWsAlign ? b : kGemmWsAlign;
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
    EpiArgs e = make_epi(epilogue, M, N, bias, resid, ld_resid, out, ld_out);
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
