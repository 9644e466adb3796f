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

/* sx/expert_exl3.zig:338-357 (scalar codebooks; window mask sx/expert_exl3.zig:124-126). */
void exl3o_decode_tile(const uint16_t *words, uint32_t n, int codebook, uint32_t window,
                       uint16_t out[256]) {
  uint16_t cws[256], perm[256];
  exl3o_unpack_tile(words, n, cws);
  exl3o_tile_perm(perm);
  uint16_t mask = (uint16_t)((1u << window) - 1u);
  for (uint32_t i = 0; i < 256u; ++i) {
    uint16_t cw = cws[i] & mask;
    out[perm[i]] = codebook == EXL3O_CB_MCG ? exl3o_decode_mcg(cw) : exl3o_decode_mul1(cw);
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
 * y += score * down.  limit > 0 clamps as mtl/q3_exl3_prep_gu_epi.metal:47-56. */
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
        if (limit > 0.0f) {
          g = g < limit ? g : limit;
          u = u > -limit ? u : -limit;
          u = u < limit ? u : limit;
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
