// exl3_device.h -- device-side pieces shared by the EXL3 kernels (gfx950, wave64).
//
// The EXL3 trellis format (paths relative to /root/reference/plugins/):
//  * a linear is stored as 16x16 tiles, trellis [in/16][out/16][n] u16 with
//    n = 16K halfwords per tile (sushi_ds41/src/sushi/exl3/expert_exl3.zig:176-245);
//  * u32 word m of a tile is hw[2m] | hw[2m+1] << 16, i.e. the little-endian
//    dword at byte 4m (expert_exl3.zig:313-315), and stream bit b is bit
//    31 - b%32 of word b/32 (expert_exl3.zig:1065-1066);
//  * codeword t is the 16 stream bits ending at floor((t+1) n / 16), circular
//    over the tile's 16n bits (expert_exl3.zig:202-205, 317-336);
//  * codeword p = 8t+j sits at row rows[j%4], column t/4 + (j<4 ? 0 : 8) of the
//    tile, rows = {2q, 2q+1, 2q+8, 2q+9}, q = t%4 (expert_exl3.zig:379-398).
//
// The 32 codewords 32a..32a+31 of a tile ("chunk a") are exactly columns a and
// a+8 over all 16 rows, and for an integer rate K they occupy the K dwords
// K*a..K*a+K-1, plus 16-K history bits from the previous chunk's last dword.
// One lane therefore decodes one chunk with compile-time bit windows and no
// exchange inside the tile beyond that one history dword.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exl3_kernels.h"

namespace exl3 {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16v_t __attribute__((ext_vector_type(16)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

// 1/sqrt(128) as the reference's kernels write it (expert_exl3_kernels.zig:930).
constexpr float HAD_SCALE = 0.08838834764831845f;

// The SwiGLU clamp (turboexl3_ds41/src/exl3/kernels/exl3/
// q3_exl3_prep_gu_epi.metal:47-52): gate to <= limit, up to [-limit, limit];
// a NaN passes through unchanged (a plain min would turn it into a bound).
__device__ __forceinline__ void swiglu_clamp(float &g, float &u, float limit) {
  g = (g != g || g < limit) ? g : limit;
  u = (u != u || u > -limit) ? u : -limit;
  u = (u != u || u < limit) ? u : limit;
}
// mul1: x = cw * 0x83DCD12D; w = f16((1024 + bytesum(x)) * f16(0x1EEE) + f16(0xC931))
// (expert_exl3.zig:275-284; turboexl3_ds41/src/exl3/kernels.zig:966-975).
constexpr uint32_t MUL1_MULT = 0x83DCD12Du;
constexpr uint16_t MUL1_INV = 0x1EEEu;
constexpr uint16_t MUL1_BIAS = 0xC931u;
// mcg: p = 0x3B603B60 ^ ((cw * 0xCBAC1FED) & 0x8FFF8FFF); w = f16(half(p.lo) + half(p.hi))
// (expert_exl3.zig:267-273).
constexpr uint32_t MCG_MULT = 0xCBAC1FEDu;

// Kernel codebook forms: mul1, mcg, the hash-mask codebooks (spec1, std1:
// one multiply, a mask keeping two tiny f16 halves, their sum times 4096;
// expert_exl3.zig:288-295) and pair1 (a pair of weights from the odd
// weight's codeword; expert_exl3.zig:297-301).
enum Codebook { CB_MUL1 = CB_FORM_MUL1, CB_MCG = CB_FORM_MCG, CB_HASH = CB_FORM_HASH, CB_PAIR1 = CB_FORM_PAIR1 };

enum OutType { OUT_F16 = 0, OUT_BF16 = 1, OUT_F32 = 2 };

template <typename T, typename F>
__device__ __forceinline__ T bits(F f) {
  return __builtin_bit_cast(T, f);
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)bits<_Float16>(h); }

// v of lane (this lane ^ m), m in {1, 2, 4, 8, 16, 32}, without the LDS
// crossbar (a __shfl_xor is a ds_bpermute: an LDS round trip per exchange):
// DPP quad permutes for 1 and 2, two DPP mirrors for 4 (half-row mirror =
// lane ^ 7, then quad lane ^ 3) and 8 (row mirror = lane ^ 15, then lane ^ 7),
// the gfx950 permlane swaps for 16 and 32 (each returns the two halves
// exchanged; a lane keeps the one holding its partner).  All 64 lanes must be
// active.  m must fold to a constant (a call inside an unrolled loop).
__device__ __forceinline__ float xor_lanes(float v, int m) {
  const int b = bits<int>(v);
  if (m == 1) return bits<float>(__builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false));
  if (m == 2) return bits<float>(__builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false));
  if (m == 4) {
    const int h = __builtin_amdgcn_mov_dpp(b, 0x141, 0xF, 0xF, false);
    return bits<float>(__builtin_amdgcn_mov_dpp(h, 0x1B, 0xF, 0xF, false));
  }
  if (m == 8) {
    const int r = __builtin_amdgcn_mov_dpp(b, 0x140, 0xF, 0xF, false);
    return bits<float>(__builtin_amdgcn_mov_dpp(r, 0x141, 0xF, 0xF, false));
  }
  const int lane = (int)(threadIdx.x & 63);
  if (m == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)b, (unsigned)b, false, false);
    return bits<float>((lane & 16) ? r[0] : r[1]);
  }
  const auto r = __builtin_amdgcn_permlane32_swap((unsigned)b, (unsigned)b, false, false);
  return bits<float>((lane & 32) ? r[0] : r[1]);
}

// One Hadamard butterfly step with the partner's value p: the lower lane of
// the pair (sg = +1) forms v + p, the upper (sg = -1) p - v.  sg * v is exact,
// so the fused form rounds once, exactly as the add or the subtraction does.
__device__ __forceinline__ float butterfly(float sg, float v, float p) {
  return __builtin_fmaf(sg, v, p);
}
// Materialises an f32 value in a VGPR so the operation that produced it is
// not merged into a following conversion.  The backend otherwise turns
// f16(a * b) into one v_fma_mixlo_f16, which rounds the exact product once;
// the reference rounds the f32 product first and then converts, and the two
// differ whenever the f32 product is an exact f16 tie.
__device__ __forceinline__ float f32_value(float f) {
  asm volatile("" : "+v"(f));
  return f;
}
// f32 -> f16, round to nearest even (v_cvt_f16_f32 under the default mode),
// of the f32 value as rounded (see f32_value).
__device__ __forceinline__ uint16_t f2h(float f) { return bits<uint16_t>((_Float16)f32_value(f)); }
__device__ __forceinline__ float bf2f(uint16_t b) { return bits<float>((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = bits<uint32_t>(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Reads element i of an activation array of type `dt` as f32.
__device__ __forceinline__ float load_act(const void *p, size_t i, int dt) {
  if (dt == OUT_F16) return h2f(((const uint16_t *)p)[i]);
  if (dt == OUT_BF16) return bf2f(((const uint16_t *)p)[i]);
  return ((const float *)p)[i];
}

// Stores a finished f16 value in the output dtype ("then the output dtype",
// turboexl3_qwen38/overlay/mlx_serve/abi/quant.zig:52-55).
__device__ __forceinline__ void store_out(void *p, size_t i, uint16_t y16, int dt) {
  if (dt == OUT_F16)
    ((uint16_t *)p)[i] = y16;
  else if (dt == OUT_BF16)
    ((uint16_t *)p)[i] = f2bf(h2f(y16));
  else
    ((float *)p)[i] = h2f(y16);
}

// ------------------------------------------------------------ codebooks

// Two codewords (low 16 bits of v0, v1 after the window mask) to a packed f16
// pair [w1 | w0].  mul1: v_sad_u8 sums x's bytes onto 0x6400 (f16 1024.0) and
// v_sad_hi_u8 puts the second sum in the high half, so h = f16 pair (1024+s1,
// 1024+s0) exactly; one packed f16 FMA then rounds once, as the reference's
// single RNE does (kernels.zig:966-975).
// The hash-mask codebooks' step after the masks: half sums of a = [w1 lo |
// w0 lo] and b = [w1 hi | w0 hi] halves, then times 4096, as f16 pairs
// (halfSumScaled, expert_exl3.zig:292-295).  One v_pk_add_f16 rounds the
// exact sum as the reference's f32 add then f16 round does (24 >= 2 * 11 + 2
// bits), and the power-of-two scale is exact (the masked halves are below
// 2^-10, so nothing overflows).
__device__ __forceinline__ uint32_t half_sums_scaled(uint32_t lo, uint32_t hi) {
  const h2_t scale = {(_Float16)4096.0f, (_Float16)4096.0f};
  return bits<uint32_t>((bits<h2_t>(lo) + bits<h2_t>(hi)) * scale);
}

// decode_pair on codewords already masked to the window and zero-extended
// (c0: the even weight's, c1: the odd weight's).
template <int CB>
__device__ __forceinline__ uint32_t decode_masked_pair(uint32_t c0, uint32_t c1, const CbRow &d) {
  if constexpr (CB == CB_MUL1) {
    uint32_t h = __builtin_amdgcn_sad_u8(c0 * MUL1_MULT, 0u, 0x64006400u);
    h = __builtin_amdgcn_sad_hi_u8(c1 * MUL1_MULT, 0u, h);
    const h2_t inv = {bits<_Float16>(MUL1_INV), bits<_Float16>(MUL1_INV)};
    const h2_t bias = {bits<_Float16>(MUL1_BIAS), bits<_Float16>(MUL1_BIAS)};
    return bits<uint32_t>(__builtin_elementwise_fma(bits<h2_t>(h), inv, bias));
  } else if constexpr (CB == CB_MCG) {
    const uint32_t p0 = 0x3B603B60u ^ ((c0 * MCG_MULT) & 0x8FFF8FFFu);
    const uint32_t p1 = 0x3B603B60u ^ ((c1 * MCG_MULT) & 0x8FFF8FFFu);
    const uint32_t lo = __builtin_amdgcn_perm(p1, p0, 0x05040100u);  // [p1.lo | p0.lo]
    const uint32_t hi = __builtin_amdgcn_perm(p1, p0, 0x07060302u);  // [p1.hi | p0.hi]
    return bits<uint32_t>(bits<h2_t>(lo) + bits<h2_t>(hi));
  } else if constexpr (CB == CB_HASH) {
    const uint32_t p0 = (c0 * d.mult) & d.mask0;
    const uint32_t p1 = (c1 * d.mult) & d.mask0;
    return half_sums_scaled(__builtin_amdgcn_perm(p1, p0, 0x05040100u),
                            __builtin_amdgcn_perm(p1, p0, 0x07060302u));
  } else {
    // pair1: w0 from p & mask0, w1 from rotl(p, rot) & mask1, p = c1 * mult
    const uint32_t p = c1 * d.mult;
    const uint32_t a = p & d.mask0;
    const uint32_t b = __builtin_amdgcn_alignbit(p, p, d.rsh) & d.mask1;
    (void)c0;
    return half_sums_scaled(__builtin_amdgcn_perm(b, a, 0x05040100u),
                            __builtin_amdgcn_perm(b, a, 0x07060302u));
  }
}

template <int CB>
__device__ __forceinline__ uint32_t decode_pair(uint32_t v0, uint32_t v1, const CbRow &d) {
  return decode_masked_pair<CB>(v0 & d.mask, v1 & d.mask, d);
}

// ---------------------------------------------------- integer-rate chunks

// Codeword i (0..31) of a chunk held as w[0] = history dword (the previous
// chunk's last dword, circularly), w[1..K] = the chunk's K dwords.  In this
// (K+1)-dword buffer codeword i ends at bit E = 32 + (i+1)K; its LSB is bit
// 31 - (E-1)%32 of dword (E-1)/32, and a 16-bit window spans at most two
// dwords, so one v_alignbit_b32 extracts it (bits above 16 are left over).
template <int K, int I>
__device__ __forceinline__ uint32_t chunk_window(const uint32_t (&w)[K + 1]) {
  constexpr int E = 32 + (I + 1) * K;
  constexpr int J1 = (E - 1) >> 5;
  constexpr int SH = 31 - ((E - 1) & 31);
  static_assert(J1 >= 1 && J1 <= K, "window outside the chunk buffer");
  return __builtin_amdgcn_alignbit(w[J1 - 1], w[J1], SH);
}

// Row and column-half of codeword i of a chunk (expert_exl3.zig:379-398):
// i = 8q + j -> row {2q, 2q+1, 2q+8, 2q+9}[j%4], column a (j<4) or a+8.
__host__ __device__ constexpr int chunk_row(int i) {
  return ((i & 3) == 0)   ? 2 * (i >> 3)
         : ((i & 3) == 1) ? 2 * (i >> 3) + 1
         : ((i & 3) == 2) ? 2 * (i >> 3) + 8
                          : 2 * (i >> 3) + 9;
}
__host__ __device__ constexpr int chunk_colhalf(int i) { return (i & 7) >= 4 ? 1 : 0; }

// Decodes pair p (codewords 2p, 2p+1: rows r, r+1 of one column) of a chunk.
template <int K, int CB, int P>
__device__ __forceinline__ uint32_t chunk_pair(const uint32_t (&w)[K + 1], const CbRow &d) {
  return decode_pair<CB>(chunk_window<K, 2 * P>(w), chunk_window<K, 2 * P + 1>(w), d);
}

// Number of a chunk's codewords whose window straddles dwords J and J+1.
__host__ __device__ constexpr int chunk_crossings(int K, int J) {
  int n = 0;
  for (int i = 0; i < 32; ++i) {
    const int e = 32 + (i + 1) * K, s = e - 16;
    if ((s >> 5) == J && ((e - 1) >> 5) == J + 1) ++n;
  }
  return n;
}

// Codeword I of a chunk as a zero-extended 16-bit value, with the cheapest
// extraction its window allows.  (Stream bit b is bit 31 - b%32 of its dword:
// a window starting at bit o of a dword, o <= 16, is bits 31-o .. 16-o.)
//  * inside one dword: one v_bfe_u32 (a shift or an and at o = 0, 16);
//  * straddling dwords J, J+1 where several windows do: the middle dword
//    T = v_alignbit(w[J], w[J+1], 16) (stream bits 32J+16 .. 32J+47) holds
//    every such window whole, so each is one v_bfe_u32 of T, and T is
//    computed once per boundary;
//  * the only straddling window of its boundary: v_perm_b32 when it starts
//    on a byte boundary, else v_alignbit_b32 and a mask.
template <int K, int I>
__device__ __forceinline__ uint32_t chunk_cw(const uint32_t (&w)[K + 1]) {
  constexpr int E = 32 + (I + 1) * K;
  constexpr int S = E - 16;
  constexpr int J0 = S >> 5, J1 = (E - 1) >> 5;
  static_assert(J0 >= 0 && J1 <= K && J1 - J0 <= 1, "window outside the chunk buffer");
  if constexpr (J0 == J1) {
    return __builtin_amdgcn_ubfe(w[J0], 16 - (S & 31), 16);
  } else if constexpr (chunk_crossings(K, J0) > 1) {
    constexpr int o = (S & 31) - 16;  // 1..15: start of the window in T
    const uint32_t T = __builtin_amdgcn_alignbit(w[J0], w[J1], 16);
    return __builtin_amdgcn_ubfe(T, 16 - o, 16);
  } else if constexpr ((S & 31) == 24) {
    // the last byte of dword J0, then the first (most significant) of J1
    return __builtin_amdgcn_perm(w[J0], w[J1], 0x0C0C0403u);
  } else {
    return __builtin_amdgcn_alignbit(w[J0], w[J1], 31 - ((E - 1) & 31)) & 0xFFFFu;
  }
}

// decode_pair on zero-extended codewords; MASKED applies a window below 16.
template <int CB, bool MASKED>
__device__ __forceinline__ uint32_t decode_pair_cw(uint32_t c0, uint32_t c1, const CbRow &d) {
  if constexpr (MASKED) {
    c0 &= d.mask;
    c1 &= d.mask;
  }
  return decode_masked_pair<CB>(c0, c1, d);
}

// (pair1 reads only the odd codeword: the even one's extraction is dead code.)
template <int K, int CB, bool MASKED, int P>
__device__ __forceinline__ uint32_t chunk_pair_cw(const uint32_t (&w)[K + 1], const CbRow &d) {
  return decode_pair_cw<CB, MASKED>(chunk_cw<K, 2 * P>(w), chunk_cw<K, 2 * P + 1>(w), d);
}

// mul1 before its affine step: the f16 pair h = (1024 + s1, 1024 + s0), exact
// integers, with w = f16(h * f16(0x1EEE) + f16(0xC931)).  A dot product over
// these feeds the affine step afterwards:  sum x (h a + b) = a sum x h +
// b sum x  (MUL1_A, MUL1_B below).
template <bool MASKED, int K, int P>
__device__ __forceinline__ uint32_t chunk_pair_mul1_h(const uint32_t (&w)[K + 1], uint32_t mask) {
  uint32_t c0 = chunk_cw<K, 2 * P>(w), c1 = chunk_cw<K, 2 * P + 1>(w);
  if constexpr (MASKED) {
    c0 &= mask;
    c1 &= mask;
  }
  const uint32_t h = __builtin_amdgcn_sad_u8(c0 * MUL1_MULT, 0u, 0x64006400u);
  return __builtin_amdgcn_sad_hi_u8(c1 * MUL1_MULT, 0u, h);
}
// f16(0x1EEE) and f16(0xC931) as f32 (exact).
constexpr float MUL1_A = 0.00676727294921875f;
constexpr float MUL1_B = -10.3828125f;

// ------------------------------------------------------------ generic rate

// Codeword t (0..255) of a tile of n halfwords whose n/2 dwords are in `tw`
// (any even n in 16..128, fractional rates included): ends at bit
// floor((t+1) n / 16), window circular over the tile's 16n bits.
__device__ __forceinline__ uint32_t tile_window(const uint32_t *tw, uint32_t n, uint32_t t) {
  const uint32_t nw = n >> 1;
  const uint32_t e = ((t + 1u) * n) >> 4;  // 1 .. 16n
  const uint32_t j1 = (e - 1u) >> 5;
  const uint32_t j0 = j1 == 0u ? nw - 1u : j1 - 1u;
  const uint32_t sh = 31u - ((e - 1u) & 31u);
  return __builtin_amdgcn_alignbit(tw[j0], tw[j1], sh);
}

// ----------------------------------------------------------- Hadamard-128

// Butterfly stage of the 128-point Walsh-Hadamard transform in the order of
// the reference's prepare/finish kernels (expert_exl3_kernels.zig:902-970):
// stages on index bits 0..6 in turn, each (lo + hi, lo - hi) with lo the
// element whose bit is clear.  Every element sees the same f32 operations in
// the same order, so results are bit-identical to that order.
// In-LDS form over `rows` blocks of 128 floats, executed by `nthreads` threads.
__device__ __forceinline__ void had128_lds(float *v, int rows, int tid, int nthreads) {
  for (int bit = 0; bit < 7; ++bit) {
    const int m = 1 << bit;
    for (int p = tid; p < rows * 64; p += nthreads) {
      const int r = p >> 6, q = p & 63;
      const int lo = ((q >> bit) << (bit + 1)) | (q & (m - 1));
      float *b = v + r * 128;
      const float a = b[lo], c = b[lo + m];
      b[lo] = a + c;
      b[lo + m] = a - c;
    }
    __syncthreads();
  }
}

// The prepare of the 128-block that 16 consecutive lanes hold, 8 elements
// each (lane j of the group: elements 8j .. 8j + 7, given as f16 pairs xo):
// f16(x) * suh in f32, Hadamard-128 with stages on index bits 0-2 in
// register and 3-6 across the 16 lanes, each (lo + hi, lo - hi) as
// had128_pair forms them, * 1/sqrt(128), f16 pairs.  The GEMV prologue's
// rows form and prepare8_kernel run the same operations in the same order.
// All 64 lanes of the wave take part (xor_lanes).
__device__ __forceinline__ uint4 prep_block8(const uint32_t (&xo)[4], uint4 su, int j) {
  const uint32_t ss[4] = {su.x, su.y, su.z, su.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = h2f((uint16_t)(xo[i] & 0xFFFFu)) * h2f((uint16_t)(ss[i] & 0xFFFFu));
    v[2 * i + 1] = h2f((uint16_t)(xo[i] >> 16)) * h2f((uint16_t)(ss[i] >> 16));
  }
#pragma unroll
  for (int b = 1; b < 8; b <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if ((i & b) == 0) {
        const float lo = v[i], hi = v[i + b];
        v[i] = lo + hi;
        v[i + b] = lo - hi;
      }
#pragma unroll
  for (int bit = 1; bit <= 8; bit <<= 1) {
    const float sg = (j & bit) == 0 ? 1.0f : -1.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = butterfly(sg, v[i], xor_lanes(v[i], bit));
  }
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = (uint32_t)f2h(v[2 * i] * HAD_SCALE) | ((uint32_t)f2h(v[2 * i + 1] * HAD_SCALE) << 16);
  return make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace exl3
