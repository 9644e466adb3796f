/*
 * exl3_oracle.h -- CPU restatement of the reference's EXL3 arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP path
 * against.  The product (plugins_amd/, libexl3_mi355x.so) never links, loads
 * or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * /root/reference/plugins/):
 *   sx/   = sushi_ds41/src/sushi/exl3/
 *   ds41/ = turboexl3_ds41/
 *   ovl/  = turboexl3_qwen38/overlay/mlx_serve/
 *   mtl/  = turboexl3_ds41/src/exl3/kernels/exl3/
 *
 * Half-precision values travel as their IEEE binary16 bit patterns (uint16_t).
 */
#ifndef EXL3_ORACLE_H
#define EXL3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Codebooks as sx/expert_exl3.zig:54-60 numbers them.  A `codebook` argument
 * carries the codebook in its low byte and, for spec1, its table + 1 in the
 * next byte (std1 and pair1 each have one table). */
enum { EXL3O_CB_MUL1 = 0, EXL3O_CB_MCG = 1, EXL3O_CB_SPEC1 = 2, EXL3O_CB_PAIR1 = 3, EXL3O_CB_STD1 = 4 };
/* The shipped codebook tables (sx/codebook_tables.zig:99-104). */
enum {
  EXL3O_TAB_PAIR1_W16_V1 = 0,
  EXL3O_TAB_SPEC1_W15 = 1,
  EXL3O_TAB_SPEC1_W16 = 2,
  EXL3O_TAB_STD1 = 3
};

/* binary16 <-> binary32, round-to-nearest-even (sx/expert_exl3.zig:259-265). */
float exl3o_h2f(uint16_t h);
uint16_t exl3o_f2h(float f);
/* binary64 -> binary16 with one RNE rounding (ds41/src/exl3/kernels.zig:966-975). */
uint16_t exl3o_d2h(double d);

/* Rate: one past the last stream bit of codeword t, floor((t+1) n / 16)
 * (sx/expert_exl3.zig:202-205). */
uint32_t exl3o_bit_end(uint32_t n, uint32_t t);

/* Codebooks (sx/expert_exl3.zig:267-284; ds41/src/exl3/kernels.zig:966-975). */
uint16_t exl3o_decode_mul1(uint16_t cw);
uint16_t exl3o_decode_mcg(uint16_t cw);
void exl3o_mul1_table(uint16_t out[65536]);
/* Table codebooks: a table's first rate, row count and fields per row, and
 * its row for rate n (0: none) (sx/codebook_tables.zig:35-52). */
int exl3o_table_info(int table, uint32_t *n_lo, uint32_t *rows, uint32_t *fields);
int exl3o_table_row(int table, uint32_t n, uint32_t row[4]);
/* spec1 / std1: one weight from its codeword and the row's {mult, mask}
 * (sx/expert_exl3.zig:288-295). */
uint16_t exl3o_decode_hash_mask(uint16_t cw, uint32_t mult, uint32_t mask);
/* pair1: both weights of a pair from the odd weight's codeword and the row
 * {mult, rot, mask0, mask1} (sx/expert_exl3.zig:297-301). */
void exl3o_decode_pair1(uint16_t cw, const uint32_t row[4], uint16_t out[2]);

/* The 256 codewords of a tile, code order (sx/expert_exl3.zig:317-336). */
void exl3o_unpack_tile(const uint16_t *words, uint32_t n, uint16_t out[256]);
/* Same thing by the bit-by-bit definition (sx/expert_exl3.zig:1062-1069). */
void exl3o_unpack_tile_bitwise(const uint16_t *words, uint32_t n, uint16_t out[256]);
/* Code position -> row-major tile slot (sx/expert_exl3.zig:379-398). */
void exl3o_tile_perm(uint16_t out[256]);
/* A tile's 16x16 f16 weights, row-major [k][n] (sx/expert_exl3.zig:338-357). */
void exl3o_decode_tile(const uint16_t *words, uint32_t n, int codebook, uint32_t window,
                       uint16_t out[256]);

/* W_inner f16 [in, out] from trellis [in/16][out/16][n] (sx/expert_exl3.zig:416-438). */
void exl3o_reconstruct_inner(const uint16_t *trellis, size_t in_f, size_t out_f, uint32_t n,
                             int codebook, uint32_t window, uint16_t *out);
/* Effective f16 W^T [in, out] = diag(suh) H W H diag(svh) (sx/expert_exl3.zig:440-488). */
void exl3o_reconstruct_public(const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
                              size_t in_f, size_t out_f, uint32_t n, int codebook,
                              uint32_t window, uint16_t *out);

/* Hadamard-128, dense Sylvester form of the CPU reference (sx/expert_exl3.zig:400-414). */
void exl3o_hadamard128_dense(float v[128]);
/* Hadamard-128, the butterfly order of the reference's prepare/finish kernels
 * (sx/expert_exl3_kernels.zig:902-970), unscaled. */
void exl3o_hadamard128_butterfly(float v[128]);

/* prepare: xp = f16(H(f16(x) * suh) / sqrt(128)) per 128-block, rows x in
 * (contract ovl/abi/quant.zig:52-55; sx/expert_exl3.zig:490-501; butterfly
 * order sx/expert_exl3_kernels.zig:902-936).  dense != 0 selects the CPU
 * reference's dense H instead. */
void exl3o_prepare(const float *x, const uint16_t *suh, size_t rows, size_t in_f, int dense,
                   uint16_t *xp);
/* inner: z = f16(sum_k xp[k] W[k, n]) with f32 accumulation in k order
 * (sx/expert_exl3.zig:503-532). */
void exl3o_inner(const uint16_t *trellis, const uint16_t *xp, size_t rows, size_t in_f,
                 size_t out_f, uint32_t n, int codebook, uint32_t window, uint16_t *z);
/* finish: y = f16(H(f16(z)) / sqrt(128) * svh) (ovl/abi/quant.zig:52-55;
 * sx/expert_exl3.zig:534-544; butterfly order sx/expert_exl3_kernels.zig:938-970). */
void exl3o_finish(const uint16_t *z, const uint16_t *svh, size_t rows, size_t out_f, int dense,
                  uint16_t *y);
/* project = prepare + inner + finish (sx/expert_exl3.zig:546-566). */
void exl3o_project(const float *x, const uint16_t *trellis, const uint16_t *suh,
                   const uint16_t *svh, size_t rows, size_t in_f, size_t out_f, uint32_t n,
                   int codebook, uint32_t window, int dense, uint16_t *y);

/* Routing: softmax over E logits, top-k, renormalise (q38/src/direct/moe.zig:84-89). */
void exl3o_route_topk(const float *logits, size_t rows, size_t experts, size_t k,
                      int32_t *inds, float *scores);
/* Routed SwiGLU experts (sx/expert_exl3_kernels.zig:3151-3206), limit > 0: clamped
 * gate min(g, L), up clamp(u, -L, L) (mtl/q3_exl3_prep_gu_epi.metal:47-56).
 * Banks are [E][in/16][out/16][n]; suh/svh [E][dim]; y f32 [rows, hidden]. */
void exl3o_moe_swiglu(const float *x, size_t rows, const uint16_t *gate_t, const uint16_t *gate_suh,
                      const uint16_t *gate_svh, const uint16_t *up_t, const uint16_t *up_suh,
                      const uint16_t *up_svh, const uint16_t *down_t, const uint16_t *down_suh,
                      const uint16_t *down_svh, const int32_t *inds, const float *scores,
                      size_t topk, size_t hidden, size_t inter, uint32_t n, int codebook,
                      uint32_t window, float limit, float *y);

/* splitmix64 and the golden planes' seeded code (ds41/src/exl3/kernels.zig:1026-1045). */
uint64_t exl3o_splitmix64(uint64_t *state);
void exl3o_synth_plane(uint64_t seed, size_t count, uint16_t *out);

/* Threads the oracle's parallel loops use (OpenMP); 0 = library default. */
void exl3o_set_threads(int n);
int exl3o_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
