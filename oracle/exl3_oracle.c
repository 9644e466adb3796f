/*
 * exl3_oracle.c -- CPU restatement of the reference's EXL3 decode and
 * projection.  TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg as the checker; the product never links it.
 *
 * Built with -ffp-contract=off so every f32 multiply and add rounds on its own,
 * as the reference's Zig (strict float mode) and Metal code do.
 * Citations are relative to /root/reference/plugins/ (prefixes in the header).
 */
#include "exl3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define TILE 16
#define TILE_VALUES 256
#define HAD 128
/* sx/expert_exl3.zig:6 (HAD_SCALE), the f32 nearest to 1/sqrt(128). */
static const float HAD_SCALE = 0.08838834764831845f;
/* sx/expert_exl3.zig:9-11 */
static const uint32_t MCG_MULT = 0xCBAC1FEDu;
static const uint32_t MUL1_MULT = 0x83DCD12Du;

static int g_threads = 0;

void exl3o_set_threads(int n) { g_threads = n; }
int exl3o_get_threads(void) {
#ifdef _OPENMP
  return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---------------------------------------------------------------- binary16 */

float exl3o_h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
  if (e == 0) {
    float v = ldexpf((float)m, -24);
    return sign ? -v : v;
  }
  if (e == 31)
    bits = sign | 0x7F800000u | (m << 13);
  else
    bits = sign | ((e - 15u + 127u) << 23) | (m << 13);
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t exl3o_d2h(double d) {
  uint64_t x;
  memcpy(&x, &d, 8);
  uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
  uint64_t ax = x & 0x7FFFFFFFFFFFFFFFull;
  if (ax > 0x7FF0000000000000ull) return sign | 0x7E00u;
  double a = fabs(d);
  if (a >= 65520.0) return sign | 0x7C00u;
  if (a < 6.103515625e-05) {
    /* subnormal: the integer multiple of 2^-24, nearest-even (the scaling is exact) */
    double q = nearbyint(a * 16777216.0);
    return sign | (uint16_t)q;
  }
  int e = (int)((ax >> 52) & 0x7FF) - 1023 + 15;
  uint64_t m = ax & 0xFFFFFFFFFFFFFull;
  uint32_t h = ((uint32_t)e << 10) | (uint32_t)(m >> 42);
  uint64_t rem = m & ((1ull << 42) - 1), halfway = 1ull << 41;
  if (rem > halfway || (rem == halfway && (h & 1u))) h++;
  return sign | (uint16_t)h;
}

/* f32 -> f16 is exact through f64 then one rounding. */
uint16_t exl3o_f2h(float f) { return exl3o_d2h((double)f); }

static inline float rnd16(float f) { return exl3o_h2f(exl3o_f2h(f)); }

/* ------------------------------------------------------------------ format */

uint32_t exl3o_bit_end(uint32_t n, uint32_t t) { return ((t + 1u) * n) >> 4; }

/* sx/expert_exl3.zig:275-284: f16(h * f16(0x1EEE) + f16(0xC931)) as one f32 FMA,
 * h = f16 bits 0x6400 + byte sum of cw * 0x83DCD12D. */
uint16_t exl3o_decode_mul1(uint16_t cw) {
  uint32_t mixed = (uint32_t)cw * MUL1_MULT;
  uint32_t s = (mixed & 0xFFu) + ((mixed >> 8) & 0xFFu) + ((mixed >> 16) & 0xFFu) + (mixed >> 24);
  float h = exl3o_h2f((uint16_t)(0x6400u + s));
  float inv = exl3o_h2f(0x1EEEu), bias = exl3o_h2f(0xC931u);
  return exl3o_f2h(fmaf(h, inv, bias));
}

/* sx/expert_exl3.zig:267-273 */
uint16_t exl3o_decode_mcg(uint16_t cw) {
  uint32_t mixed = (uint32_t)cw * MCG_MULT;
  uint32_t pair = 0x3B603B60u ^ (mixed & 0x8FFF8FFFu);
  float lo = exl3o_h2f((uint16_t)(pair & 0xFFFFu));
  float hi = exl3o_h2f((uint16_t)(pair >> 16));
  return exl3o_f2h(lo + hi);
}

/* ------------------------------------------------------ table codebooks */

/* Rows of the pack contract's codebook tables, one per even rate n from the
 * table's n_lo: {mult, mask} for the hash-mask codebooks (spec1, std1),
 * {mult, rot, mask0, mask1} for pair1.  Data as sx/codebook_tables.zig:
 * 99-203 (names, digests, ranges) and sx/expert_exl3.zig:23-46 (the pair1
 * rows) hold them. */
static const uint32_t PAIR1_ROWS[21][4] = {
    {0x58F41BF3u, 3, 0x8ED78C13u, 0x8EEE8C03u},  {0x58F41BF3u, 3, 0x8ED78C13u, 0x8EEE8C03u},
    {0x7AA2BE15u, 3, 0x8ED78C13u, 0x8ECE8C03u},  {0x7B229E11u, 3, 0x8ED78C13u, 0x8ECE8C03u},
    {0x3B22BE15u, 3, 0x8ED78C13u, 0x8ECE8C03u},  {0x46C63E17u, 19, 0x8F9A8E6Eu, 0x8E258FFEu},
    {0x46C63E17u, 19, 0x8F9A8E6Eu, 0x8E258FFEu}, {0x46C63E17u, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0x46C63E17u, 19, 0x8F9A8E6Eu, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0x82439F67u, 19, 0x8E6E8F9Au, 0x8E258FAEu}, {0xE2C7FC0Du, 19, 0x8F408FB0u, 0x8F918F89u},
    {0xE2C7FC0Du, 19, 0x8F408FA0u, 0x8F118FC9u}, {0xE2C7FC0Du, 19, 0x8F408FA0u, 0x8F118FC9u},
    {0xE2C7FC0Du, 19, 0x8F408FA0u, 0x8F118FC9u},
};
static const uint32_t SPEC1_W15[57][2] = {
    {0x84d1cf89u, 0x8fe08947u}, {0x84c1cf49u, 0x8fe48a47u}, {0x84d1cfe9u, 0x8fe08a47u},
    {0x84d1cfc9u, 0x8ff08b67u}, {0x84c1cf49u, 0x8fe08b47u}, {0x84c1cf99u, 0x8fa08b66u},
    {0x862c1d37u, 0x8ff28c50u}, {0x84641fb7u, 0x8fa08c40u}, {0x846c1fa7u, 0x8fe08c80u},
    {0x844c1fd7u, 0x8ffe8c98u}, {0x846c1fa7u, 0x8ffe8d10u}, {0x845c1f77u, 0x8ffa8e10u},
    {0x843c1fa7u, 0x8ffe8e40u}, {0x843c1fa7u, 0x8ffe8e40u}, {0x842c1fc7u, 0x8fff8f00u},
    {0x843c1fb7u, 0x8ffe8f10u}, {0x84181fb5u, 0x8fe08f80u}, {0x84081f75u, 0x8ffa8f72u},
    {0x84081f75u, 0x8fd68fd0u}, {0x84241f27u, 0x8ffc8fc0u}, {0x84081f73u, 0x8fe08f80u},
    {0x84081f75u, 0x8fbe8ff0u}, {0x3fed4cefu, 0x8fe08fe0u}, {0x3fed4cefu, 0x8fc18ff2u},
    {0x3fed4cefu, 0x8ff08ff0u}, {0x3fed4cefu, 0x8fe28ff0u}, {0x3fed4cefu, 0x8fe08fe0u},
    {0x80081b7bu, 0x8ff08fc8u}, {0x80081b7bu, 0x8ff48fc0u}, {0x400036cbu, 0x8f448fffu},
    {0x400036cbu, 0x8fe48fffu}, {0x400036cbu, 0x8f448ff9u}, {0x8000387bu, 0x8fe08ff7u},
    {0x8000387bu, 0x8fc08feeu}, {0x80003779u, 0x8fe88ffeu}, {0x80003779u, 0x8fc88ffcu},
    {0x80003779u, 0x8fca8ffcu}, {0x80003779u, 0x8fcc8ffeu}, {0x80003879u, 0x8ffc8fefu},
    {0x50003851u, 0x8ff98fffu}, {0xd0003751u, 0x8ff98fffu}, {0x50003851u, 0x8ff98ff6u},
    {0xd0003931u, 0x8ff98fffu}, {0xd0003931u, 0x8ff98ffau}, {0xd0003931u, 0x8ff48ffau},
    {0x300031b1u, 0x8ffb8ffcu}, {0x300031b1u, 0x8ffa8ffeu}, {0x300031b1u, 0x8ffb8ffcu},
    {0xc00031f1u, 0x8ffe8ffau}, {0x400031f1u, 0x8ffe8ffeu}, {0x400031f1u, 0x8ffe8ffeu},
    {0x40003931u, 0x8ffc8ffcu}, {0x40003931u, 0x8ffc8ffcu}, {0x40003931u, 0x8ff88ffeu},
    {0x40003931u, 0x8ff88ffcu}, {0x80003811u, 0x8ffc8ffcu}, {0x80003811u, 0x8ffc8ffcu},
};
static const uint32_t SPEC1_W16[21][2] = {
    {0x862d1c19u, 0x8fee8c30u}, {0x862d1d37u, 0x8fee8c30u}, {0x862d1d37u, 0x8ffe8c10u},
    {0x842f1f37u, 0x8ffc8d10u}, {0x840f1f67u, 0x8ffc8d10u}, {0x844f1f77u, 0x8ffe8d40u},
    {0x840d1f37u, 0x8ffe8e10u}, {0x84091f33u, 0x8fe88e00u}, {0x844d1f77u, 0x8fe08e00u},
    {0x843c1fa7u, 0x8ffe8e40u}, {0x844c1f7fu, 0x8ffc8f02u}, {0x841c1fb9u, 0x8fe88f04u},
    {0x842c1fc7u, 0x8ffe8fd0u}, {0x83fc1fa3u, 0x8ffe8fd0u}, {0x83fc1fa3u, 0x8ffe8fc1u},
    {0x83fc1fa3u, 0x8ffe8fd0u}, {0x83fc1fa3u, 0x8fee8fc0u}, {0x84061f77u, 0x8fd08f80u},
    {0x84081f6fu, 0x8ffe8fc0u}, {0x84081f25u, 0x8ffe8fe0u}, {0x83f81f6fu, 0x8ff48fc0u},
};
/* sx/codebook_tables.zig:206: std1's one pair, at n = 24..64. */
static const uint32_t STD1_PAIR[2] = {0x840C1F37u, 0x8FFE8FD0u};

int exl3o_table_info(int table, uint32_t *n_lo, uint32_t *rows, uint32_t *fields) {
  switch (table) {
    case EXL3O_TAB_PAIR1_W16_V1: *n_lo = 24; *rows = 21; *fields = 4; return 1;
    case EXL3O_TAB_SPEC1_W15: *n_lo = 16; *rows = 57; *fields = 2; return 1;
    case EXL3O_TAB_SPEC1_W16: *n_lo = 24; *rows = 21; *fields = 2; return 1;
    case EXL3O_TAB_STD1: *n_lo = 24; *rows = 21; *fields = 2; return 1;
    default: return 0;
  }
}

/* sx/codebook_tables.zig:48-52 (Table.row): row (n - n_lo) / 2 for an even n
 * in range, else none (0).  row[] = {mult, mask} or {mult, rot, mask0, mask1}. */
int exl3o_table_row(int table, uint32_t n, uint32_t row[4]) {
  uint32_t n_lo, rows, fields;
  if (!exl3o_table_info(table, &n_lo, &rows, &fields)) return 0;
  if (n % 2u != 0u || n < n_lo || (n - n_lo) / 2u >= rows) return 0;
  const uint32_t i = (n - n_lo) / 2u;
  row[2] = row[3] = 0;
  switch (table) {
    case EXL3O_TAB_PAIR1_W16_V1: memcpy(row, PAIR1_ROWS[i], 16); break;
    case EXL3O_TAB_SPEC1_W15: row[0] = SPEC1_W15[i][0]; row[1] = SPEC1_W15[i][1]; break;
    case EXL3O_TAB_SPEC1_W16: row[0] = SPEC1_W16[i][0]; row[1] = SPEC1_W16[i][1]; break;
    default: row[0] = STD1_PAIR[0]; row[1] = STD1_PAIR[1]; break;
  }
  return 1;
}

/* sx/expert_exl3.zig:292-295 (halfSumScaled): the f16 halves summed in f32 and
 * rounded, then times scale in f32 and rounded. */
static uint16_t half_sum_scaled(uint32_t halves, uint32_t scale) {
  const uint16_t sum = exl3o_f2h(exl3o_h2f((uint16_t)(halves & 0xFFFFu)) +
                                 exl3o_h2f((uint16_t)(halves >> 16)));
  return exl3o_f2h(exl3o_h2f(sum) * (float)scale);
}

/* sx/expert_exl3.zig:288-290 (decodeHashMask), scale 4096 (:17). */
uint16_t exl3o_decode_hash_mask(uint16_t cw, uint32_t mult, uint32_t mask) {
  return half_sum_scaled(((uint32_t)cw * mult) & mask, 4096u);
}

/* sx/expert_exl3.zig:297-301 (decodePair): both weights of a pair from one
 * codeword, w0 from p & mask0, w1 from rotl(p, rot) & mask1, p = cw * mult. */
void exl3o_decode_pair1(uint16_t cw, const uint32_t row[4], uint16_t out[2]) {
  const uint32_t p = (uint32_t)cw * row[0];
  const uint32_t rot = row[1] & 31u;
  const uint32_t r = rot == 0u ? p : (p << rot) | (p >> (32u - rot));
  out[0] = half_sum_scaled(p & row[2], 4096u);
  out[1] = half_sum_scaled(r & row[3], 4096u);
}

/* The decode a `codebook` argument names: the codebook in its low byte
 * (EXL3O_CB_*), for spec1 the table + 1 in the next byte (std1 and pair1 have
 * one table each).  Fills row for the table codebooks; aborts on a rate
 * the table has no row for (a test's mistake). */
static int decode_row(int codebook, uint32_t n, uint32_t row[4]) {
  const int cb = codebook & 0xFF;
  int table = -1;
  if (cb == EXL3O_CB_PAIR1) table = EXL3O_TAB_PAIR1_W16_V1;
  if (cb == EXL3O_CB_STD1) table = EXL3O_TAB_STD1;
  if (cb == EXL3O_CB_SPEC1) table = ((codebook >> 8) & 0xFF) - 1;
  if (table >= 0 && !exl3o_table_row(table, n, row)) abort();
  if (cb == EXL3O_CB_SPEC1 && table < 0) abort();
  return cb;
}

void exl3o_mul1_table(uint16_t out[65536]) {
  for (uint32_t s = 0; s < 65536u; ++s) out[s] = exl3o_decode_mul1((uint16_t)s);
}

/* sx/expert_exl3.zig:313-315: u32 word m = hw[2m] | hw[2m+1] << 16. */
static inline uint32_t word_u32(const uint16_t *w, size_t i) {
  return (uint32_t)w[2 * i] | ((uint32_t)w[2 * i + 1] << 16);
}

/* sx/expert_exl3.zig:317-336: two codewords per step from a 64-bit funnel of the
 * words holding the pair's windows, tail-biting (one lap up, mod the tile). */
void exl3o_unpack_tile(const uint16_t *words, uint32_t n, uint16_t out[256]) {
  const uint32_t word_count = n / 2, total = 16u * n;
  for (uint32_t th = 0; th < 128u; ++th) {
    uint32_t e0 = exl3o_bit_end(n, th * 2), e1 = exl3o_bit_end(n, th * 2 + 1);
    uint32_t bit0 = e0 + total - 16u, bit2 = e1 + total;
    uint32_t i0 = bit0 / 32u, i1 = (bit2 - 1u) / 32u;
    uint32_t shift = (i1 + 1u) * 32u - bit2;
    uint64_t merged = ((uint64_t)word_u32(words, i0 % word_count) << 32) |
                      (uint64_t)word_u32(words, i1 % word_count);
    uint32_t funnel = (uint32_t)(merged >> shift);
    uint32_t fresh = e1 - e0;
    out[th * 2] = (uint16_t)((funnel >> fresh) & 0xFFFFu);
    out[th * 2 + 1] = (uint16_t)(funnel & 0xFFFFu);
  }
}

/* sx/expert_exl3.zig:1062-1069: stream bit `at` is bit 15 - at%16 of halfword
 * 2*(at/32) + 1 - (at%32)/16; codeword = the 16 bits ending at bitEnd, MSB first. */
void exl3o_unpack_tile_bitwise(const uint16_t *words, uint32_t n, uint16_t out[256]) {
  for (uint32_t slot = 0; slot < 256u; ++slot) {
    uint32_t cw = 0;
    for (uint32_t bit = 0; bit < 16u; ++bit) {
      uint32_t at = ((slot + 1u) * n / 16u + 16u * n - 16u + bit) % (16u * n);
      uint32_t v = (words[2 * (at / 32u) + (1u - (at % 32u) / 16u)] >> (15u - at % 16u)) & 1u;
      cw = (cw << 1) | v;
    }
    out[slot] = (uint16_t)cw;
  }
}

/* sx/expert_exl3.zig:379-398 */
void exl3o_tile_perm(uint16_t out[256]) {
  for (uint32_t th = 0; th < 32u; ++th) {
    uint32_t r0 = (th % 4u) * 2u, c0 = th / 4u;
    uint32_t rows[4] = {r0, r0 + 1u, r0 + 8u, r0 + 9u};
    for (uint32_t j = 0; j < 8u; ++j)
      out[th * 8u + j] = (uint16_t)(rows[j % 4u] * 16u + c0 + (j < 4u ? 0u : 8u));
  }
}

/* sx/expert_exl3.zig:338-357 (window mask sx/expert_exl3.zig:124-126): pair1
 * decodes weights 2j and 2j+1 from codeword 2j+1; the others each codeword
 * on its own, the hash-mask codebooks with their table's row for n. */
void exl3o_decode_tile(const uint16_t *words, uint32_t n, int codebook, uint32_t window,
                       uint16_t out[256]) {
  uint16_t cws[256], perm[256];
  uint32_t row[4] = {0, 0, 0, 0};
  const int cb = decode_row(codebook, n, row);
  exl3o_unpack_tile(words, n, cws);
  exl3o_tile_perm(perm);
  uint16_t mask = (uint16_t)((1u << window) - 1u);
  if (cb == EXL3O_CB_PAIR1) {
    for (uint32_t j = 0; j < 128u; ++j) {
      uint16_t w[2];
      exl3o_decode_pair1(cws[2 * j + 1] & mask, row, w);
      out[perm[2 * j]] = w[0];
      out[perm[2 * j + 1]] = w[1];
    }
    return;
  }
  for (uint32_t i = 0; i < 256u; ++i) {
    uint16_t cw = cws[i] & mask;
    out[perm[i]] = cb == EXL3O_CB_MCG                               ? exl3o_decode_mcg(cw)
                   : (cb == EXL3O_CB_SPEC1 || cb == EXL3O_CB_STD1) ? exl3o_decode_hash_mask(cw, row[0], row[1])
                                                                    : exl3o_decode_mul1(cw);
  }
}

/* sx/expert_exl3.zig:416-438 */
void exl3o_reconstruct_inner(const uint16_t *trellis, size_t in_f, size_t out_f, uint32_t n,
                             int codebook, uint32_t window, uint16_t *out) {
  const size_t in_tiles = in_f / TILE, out_tiles = out_f / TILE;
  long long total = (long long)(in_tiles * out_tiles);
#pragma omp parallel for schedule(static) num_threads(exl3o_get_threads())
  for (long long it = 0; it < total; ++it) {
    size_t tk = (size_t)it / out_tiles, tn = (size_t)it % out_tiles;
    uint16_t tile[256];
    exl3o_decode_tile(trellis + (tk * out_tiles + tn) * n, n, codebook, window, tile);
    for (size_t r = 0; r < TILE; ++r)
      memcpy(out + (tk * TILE + r) * out_f + tn * TILE, tile + r * TILE, TILE * sizeof(uint16_t));
  }
}

/* sx/expert_exl3.zig:400-414: acc += (+-HAD_SCALE) * v[k] in k order. */
void exl3o_hadamard128_dense(float v[128]) {
  float tmp[HAD];
  for (int r = 0; r < HAD; ++r) {
    float acc = 0.0f;
    for (int k = 0; k < HAD; ++k) {
      float e = (__builtin_popcount((unsigned)(r & k)) & 1) ? -HAD_SCALE : HAD_SCALE;
      float p = e * v[k];
      acc = acc + p;
    }
    tmp[r] = acc;
  }
  memcpy(v, tmp, sizeof(tmp));
}

/* sx/expert_exl3_kernels.zig:902-936: element i sits in lane i%32, component i/32.
 * Five lane-xor stages (bits 0..4: lower = v + partner, upper = partner - v), then
 * the component stages s0 = x+y, s1 = x-y, s2 = z+w, s3 = z-w and outputs
 * (s0+s2, s1+s3, s0-s2, s1-s3).  Unscaled: callers multiply by HAD_SCALE. */
void exl3o_hadamard128_butterfly(float v[128]) {
  for (int bit = 1; bit <= 16; bit <<= 1) {
    for (int c = 0; c < 4; ++c) {
      float *p = v + 32 * c;
      for (int l = 0; l < 32; ++l) {
        if (l & bit) continue;
        float lo = p[l], up = p[l | bit];
        p[l] = lo + up;
        p[l | bit] = lo - up;
      }
    }
  }
  for (int l = 0; l < 32; ++l) {
    float x = v[l], y = v[l + 32], z = v[l + 64], w = v[l + 96];
    float s0 = x + y, s1 = x - y, s2 = z + w, s3 = z - w;
    v[l] = s0 + s2;
    v[l + 32] = s1 + s3;
    v[l + 64] = s0 - s2;
    v[l + 96] = s1 - s3;
  }
}

void exl3o_prepare(const float *x, const uint16_t *suh, size_t rows, size_t in_f, int dense,
                   uint16_t *xp) {
  for (size_t r = 0; r < rows; ++r) {
    const float *xr = x + r * in_f;
    for (size_t b = 0; b < in_f; b += HAD) {
      float v[HAD];
      for (int i = 0; i < HAD; ++i) v[i] = rnd16(xr[b + i]) * exl3o_h2f(suh[b + i]);
      if (dense) {
        exl3o_hadamard128_dense(v);
        for (int i = 0; i < HAD; ++i) xp[r * in_f + b + i] = exl3o_f2h(v[i]);
      } else {
        exl3o_hadamard128_butterfly(v);
        for (int i = 0; i < HAD; ++i) xp[r * in_f + b + i] = exl3o_f2h(v[i] * HAD_SCALE);
      }
    }
  }
}

/* sx/expert_exl3.zig:503-532, rows at once; each output column sums in k order. */
void exl3o_inner(const uint16_t *trellis, const uint16_t *xp, size_t rows, size_t in_f,
                 size_t out_f, uint32_t n, int codebook, uint32_t window, uint16_t *z) {
  const size_t in_tiles = in_f / TILE, out_tiles = out_f / TILE;
  float *xf = (float *)malloc(rows * in_f * sizeof(float));
  for (size_t i = 0; i < rows * in_f; ++i) xf[i] = exl3o_h2f(xp[i]);
#pragma omp parallel for schedule(static) num_threads(exl3o_get_threads())
  for (long long tnl = 0; tnl < (long long)out_tiles; ++tnl) {
    size_t tn = (size_t)tnl;
    float *acc = (float *)calloc(rows * TILE, sizeof(float));
    uint16_t tile[256];
    float w[256];
    for (size_t tk = 0; tk < in_tiles; ++tk) {
      exl3o_decode_tile(trellis + (tk * out_tiles + tn) * n, n, codebook, window, tile);
      for (int i = 0; i < 256; ++i) w[i] = exl3o_h2f(tile[i]);
      for (size_t row = 0; row < rows; ++row) {
        const float *xr = xf + row * in_f + tk * TILE;
        float *ar = acc + row * TILE;
        for (int r = 0; r < TILE; ++r) {
          float xv = xr[r];
          for (int c = 0; c < TILE; ++c) ar[c] = ar[c] + xv * w[r * TILE + c];
        }
      }
    }
    for (size_t row = 0; row < rows; ++row)
      for (int c = 0; c < TILE; ++c) z[row * out_f + tn * TILE + c] = exl3o_f2h(acc[row * TILE + c]);
    free(acc);
  }
  free(xf);
}

void exl3o_finish(const uint16_t *z, const uint16_t *svh, size_t rows, size_t out_f, int dense,
                  uint16_t *y) {
  for (size_t r = 0; r < rows; ++r) {
    for (size_t b = 0; b < out_f; b += HAD) {
      float v[HAD];
      for (int i = 0; i < HAD; ++i) v[i] = exl3o_h2f(z[r * out_f + b + i]);
      if (dense) {
        exl3o_hadamard128_dense(v);
        for (int i = 0; i < HAD; ++i) y[r * out_f + b + i] = exl3o_f2h(v[i] * exl3o_h2f(svh[b + i]));
      } else {
        exl3o_hadamard128_butterfly(v);
        for (int i = 0; i < HAD; ++i) {
          float s = v[i] * HAD_SCALE;
          y[r * out_f + b + i] = exl3o_f2h(s * exl3o_h2f(svh[b + i]));
        }
      }
    }
  }
}

void exl3o_project(const float *x, const uint16_t *trellis, const uint16_t *suh,
                   const uint16_t *svh, size_t rows, size_t in_f, size_t out_f, uint32_t n,
                   int codebook, uint32_t window, int dense, uint16_t *y) {
  uint16_t *xp = (uint16_t *)malloc(rows * in_f * 2);
  uint16_t *z = (uint16_t *)malloc(rows * out_f * 2);
  exl3o_prepare(x, suh, rows, in_f, dense, xp);
  exl3o_inner(trellis, xp, rows, in_f, out_f, n, codebook, window, z);
  exl3o_finish(z, svh, rows, out_f, dense, y);
  free(xp);
  free(z);
}

/* reconstructPublic, sx/expert_exl3.zig:440-488 (dense H, f32 throughout, one f16 store). */
void exl3o_reconstruct_public(const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
                              size_t in_f, size_t out_f, uint32_t n, int codebook,
                              uint32_t window, uint16_t *out) {
  size_t total = in_f * out_f;
  uint16_t *inner = (uint16_t *)malloc(total * 2);
  float *w = (float *)malloc(total * sizeof(float));
  exl3o_reconstruct_inner(trellis, in_f, out_f, n, codebook, window, inner);
  for (size_t i = 0; i < total; ++i) w[i] = exl3o_h2f(inner[i]);
  for (size_t rb = 0; rb < in_f; rb += HAD) {
#pragma omp parallel for schedule(static) num_threads(exl3o_get_threads())
    for (long long col = 0; col < (long long)out_f; ++col) {
      float v[HAD];
      for (int r = 0; r < HAD; ++r) v[r] = w[(rb + r) * out_f + col];
      exl3o_hadamard128_dense(v);
      for (int r = 0; r < HAD; ++r) w[(rb + r) * out_f + col] = v[r];
    }
  }
  for (size_t r = 0; r < in_f; ++r) {
    float s = exl3o_h2f(suh[r]);
    for (size_t c = 0; c < out_f; ++c) w[r * out_f + c] = w[r * out_f + c] * s;
  }
  for (size_t cb = 0; cb < out_f; cb += HAD) {
#pragma omp parallel for schedule(static) num_threads(exl3o_get_threads())
    for (long long r = 0; r < (long long)in_f; ++r) {
      float v[HAD];
      for (int c = 0; c < HAD; ++c) v[c] = w[r * out_f + cb + c];
      exl3o_hadamard128_dense(v);
      for (int c = 0; c < HAD; ++c) w[r * out_f + cb + c] = v[c];
    }
  }
  for (size_t c = 0; c < out_f; ++c) {
    float s = exl3o_h2f(svh[c]);
    for (size_t r = 0; r < in_f; ++r) w[r * out_f + c] = w[r * out_f + c] * s;
  }
  for (size_t i = 0; i < total; ++i) out[i] = exl3o_f2h(w[i]);
  free(inner);
  free(w);
}

/* ------------------------------------------------------------------- MoE */

/* q38/src/direct/moe.zig:84-89 (top-k of the softmax, renormalised); ties keep
 * the lower expert index first. */
void exl3o_route_topk(const float *logits, size_t rows, size_t experts, size_t k,
                      int32_t *inds, float *scores) {
  float *p = (float *)malloc(experts * sizeof(float));
  for (size_t r = 0; r < rows; ++r) {
    const float *l = logits + r * experts;
    float mx = l[0];
    for (size_t e = 1; e < experts; ++e) mx = l[e] > mx ? l[e] : mx;
    double sum = 0.0;
    for (size_t e = 0; e < experts; ++e) {
      p[e] = expf(l[e] - mx);
      sum += p[e];
    }
    for (size_t e = 0; e < experts; ++e) p[e] = (float)(p[e] / sum);
    double kept = 0.0;
    for (size_t j = 0; j < k; ++j) {
      size_t best = 0;
      float bv = -1.0f;
      for (size_t e = 0; e < experts; ++e)
        if (p[e] > bv) {
          bv = p[e];
          best = e;
        }
      inds[r * k + j] = (int32_t)best;
      scores[r * k + j] = bv;
      kept += bv;
      p[best] = -2.0f;
    }
    for (size_t j = 0; j < k; ++j) scores[r * k + j] = (float)(scores[r * k + j] / kept);
  }
  free(p);
}

/* sx/expert_exl3_kernels.zig:3151-3206: for each routed slot, gate and up
 * projections of x, h = silu(g) * u in f32, the down projection of h, and
 * y += score * down.  limit > 0 clamps as mtl/q3_exl3_prep_gu_epi.metal:47-56
 * (gate <= limit, up in [-limit, limit], NaN kept). */
void exl3o_moe_swiglu(const float *x, size_t rows, const uint16_t *gate_t, const uint16_t *gate_suh,
                      const uint16_t *gate_svh, const uint16_t *up_t, const uint16_t *up_suh,
                      const uint16_t *up_svh, const uint16_t *down_t, const uint16_t *down_suh,
                      const uint16_t *down_svh, const int32_t *inds, const float *scores,
                      size_t topk, size_t hidden, size_t inter, uint32_t n, int codebook,
                      uint32_t window, float limit, float *y) {
  const size_t stride_gu = (hidden / TILE) * (inter / TILE) * n;
  const size_t stride_d = (inter / TILE) * (hidden / TILE) * n;
  uint16_t *gy = (uint16_t *)malloc(inter * 2), *uy = (uint16_t *)malloc(inter * 2);
  uint16_t *dy = (uint16_t *)malloc(hidden * 2);
  float *h = (float *)malloc(inter * sizeof(float));
  for (size_t r = 0; r < rows; ++r) {
    float *yr = y + r * hidden;
    for (size_t i = 0; i < hidden; ++i) yr[i] = 0.0f;
    for (size_t k = 0; k < topk; ++k) {
      size_t e = (size_t)inds[r * topk + k];
      exl3o_project(x + r * hidden, gate_t + e * stride_gu, gate_suh + e * hidden,
                    gate_svh + e * inter, 1, hidden, inter, n, codebook, window, 0, gy);
      exl3o_project(x + r * hidden, up_t + e * stride_gu, up_suh + e * hidden, up_svh + e * inter,
                    1, hidden, inter, n, codebook, window, 0, uy);
      for (size_t i = 0; i < inter; ++i) {
        float g = exl3o_h2f(gy[i]), u = exl3o_h2f(uy[i]);
        if (limit > 0.0f) { /* mtl/q3_exl3_prep_gu_epi.metal:47-52: a NaN passes through */
          g = (isnan(g) || g < limit) ? g : limit;
          u = (isnan(u) || u > -limit) ? u : -limit;
          u = (isnan(u) || u < limit) ? u : limit;
        }
        h[i] = (g / (1.0f + expf(-g))) * u;
      }
      exl3o_project(h, down_t + e * stride_d, down_suh + e * inter, down_svh + e * hidden, 1, inter,
                    hidden, n, codebook, window, 0, dy);
      float w = scores[r * topk + k];
      for (size_t i = 0; i < hidden; ++i) yr[i] = yr[i] + w * exl3o_h2f(dy[i]);
    }
  }
  free(gy);
  free(uy);
  free(dy);
  free(h);
}

/* ------------------------------------------------------------- fixtures */

/* ds41/src/exl3/kernels.zig:1026-1032 */
uint64_t exl3o_splitmix64(uint64_t *state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* ds41/src/exl3/kernels.zig:1034-1045: little-endian int16 view of the outputs. */
void exl3o_synth_plane(uint64_t seed, size_t count, uint16_t *out) {
  uint64_t s = seed;
  for (size_t i = 0; i < count; i += 4) {
    uint64_t z = exl3o_splitmix64(&s);
    for (size_t j = 0; j < 4 && i + j < count; ++j) out[i + j] = (uint16_t)(z >> (16 * j));
  }
}
