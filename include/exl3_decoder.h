/* exl3_decoder.h -- the non-EXL3 operations of a Qwen3-8B-shaped decode step,
 * exported by libexl3_mi355x.so for the decode tok/s harness.
 *
 * These are not part of the reference's quant-plugin table: they stand in for
 * the caller of that table (the reference's model plugin, whose ops run on
 * MLX: turboexl3_qwen38/src/direct/linear.zig:65-85 for RMSNorm and SiLU,
 * attn.zig:133-141 and attn_core.zig for q/k norm, RoPE, the KV append and
 * attention; paths relative to /root/reference/plugins/).  Device pointers,
 * f16 as uint16_t bits, streams as hipStream_t; every entry returns 0 or a
 * HIP error code and launches nothing when its shape checks fail.
 */
#ifndef EXL3_DECODER_H
#define EXL3_DECODER_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "exl3_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Head dimension the attention kernels are built for (Qwen3-8B: 128). */
#define EXL3D_HEAD_DIM 128

/* h[b][:] = f32(table[ids[b]][:]); table f16 [vocab][H], h f32 [B][H]; with
 * ssq (H a multiple of 128) also ssq[b][g] = sum of h^2 over columns 128 g ..
 * 128 g + 127 (the input of exl3d_linears' RMSNorm). */
int exl3d_embed(const int32_t *ids, int B, const uint16_t *table, int H, float *h, float *ssq,
                hipStream_t s);

/* h += add (f16 [B][H], may be NULL); out = f16(h * rsqrt(mean(h^2) + eps) * w). */
int exl3d_add_rmsnorm(float *h, const uint16_t *add, const uint16_t *w, uint16_t *out, int B,
                      int H, float eps, hipStream_t s);

/* q [B][nq*D], k, v [B][nkv*D] (projections, f16); per head RMSNorm with qn / kn
 * (D), rotate-half RoPE at position pos[b] (angle pos * theta^(-2i/D)); q to
 * qout [B][nq*D]; k, v into kcache / vcache [B][nkv][Tmax][D] at row pos[b]. */
int exl3d_qk_norm_rope(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *qn,
                       const uint16_t *kn, const int32_t *pos, int B, int nq, int nkv, float eps,
                       float theta, uint16_t *qout, uint16_t *kcache, uint16_t *vcache, int Tmax,
                       hipStream_t s);

/* Scratch bytes exl3d_attn_decode(_rope) needs for these sizes: the split
 * slots (each split's softmax state), which the call's combine launch reads.
 * Calls that share a scratch must be ordered on one stream. */
size_t exl3d_attn_scratch_bytes(int B, int nq, int nkv, int Tmax);

/* The key splits exl3d_attn_decode(_rope) uses for these sizes (0 for sizes
 * it refuses), and the query heads per kv head it serves (4). */
int exl3d_attn_splits(int B, int nkv, int Tmax);
int exl3d_attn_heads_per_kv(void);

/* Decode attention, grouped-query (nq = 4 nkv): out [B][nq*D] f16 =
 * softmax(q k^T * scale) v over keys 0 .. pos[b] of row b's cache, split
 * over the keys (one workgroup per split and kv head), then a second launch
 * combines the splits.  out NULL: no combine; the split slots stay in
 * scratch as [B][nkv][exl3d_attn_splits()][4][D + 2] f32 (a split's
 * unnormalised o values, then its running max m and sum l), for a consumer
 * that combines them (exl3d_attn_o). */
int exl3d_attn_decode(const uint16_t *q, const uint16_t *kcache, const uint16_t *vcache,
                      const int32_t *pos, int B, int nq, int nkv, int Tmax, float scale,
                      uint16_t *out, float *scratch, size_t scratch_bytes, hipStream_t s);

/* exl3d_qk_norm_rope followed by exl3d_attn_decode, in one launch: q, k, v
 * are the raw projections; q's heads are normalized and rotated inside the
 * attention, k (normalized, rotated) and v are appended at row pos[b] of the
 * caches before the attention reads them. */
int exl3d_attn_decode_rope(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                           const uint16_t *qn, const uint16_t *kn, const int32_t *pos, int B,
                           int nq, int nkv, float eps, float theta, uint16_t *kcache,
                           uint16_t *vcache, int Tmax, float scale, uint16_t *out, float *scratch,
                           size_t scratch_bytes, hipStream_t s);

/* The decode step's EXL3 linears with their neighbours fused in, B <= 16
 * rows: outs[i] = x @ W_i^T (f16) for the count weights (as
 * exl3_matmul_shared), where x is
 *  - with norm_w: the RMSNorm of the f32 residual h = x [B][in],
 *    f16(h * rsqrt(sum_g nssq[b][g] / in + eps) * norm_w), nssq [B][in/128]
 *    its sums of squares per 128 columns (in <= 8192; rows that fit one
 *    prepare batch, e.g. B = 1 at in = 4096);
 *  - with up (f16 [B][in]): f16(silu(x) * up), x the gate (f16);
 *  - else x itself (f16);
 * and, with res (count 1): res [B][out] += f32(y) instead of storing
 * outs[0] (outs may be NULL), and res_ssq [B][out/128] = the new res's sums
 * of squares per 128 columns.  Returns 0, a HIP error, or -1 when the
 * weights or shapes are refused. */
int exl3d_linears(const exl3_weight *const *ws, int count, const void *x, int B,
                  const uint16_t *norm_w, const float *nssq, float eps, const uint16_t *up,
                  float *res, float *res_ssq, uint16_t *const *outs, hipStream_t s);

/* The decode step's attention and o projection: exl3d_attn_decode_rope,
 * then res [B][out] += f32(att @ o^T) with res_ssq [B][out/128] the new
 * res's sums of squares per 128 columns (exl3d_linears with res).  Rows
 * that fit one prepare batch of o's GEMV (B = 1 at Qwen3-8B's shapes) skip
 * the combine launch: o's prepare combines the split slots itself, with
 * the combine's arithmetic, so att is not written; other rows combine into
 * att (f16 [B][nq*D]) first, written as o's prepared rows (the attention
 * output rotated with o's suh, which o's GEMV then takes as they are).
 * Results are equal either way.  Returns 0, a
 * HIP error, or -1 when the weight or shapes are refused. */
int exl3d_attn_o(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *qn,
                 const uint16_t *kn, const int32_t *pos, int B, int nq, int nkv, float eps,
                 float theta, uint16_t *kcache, uint16_t *vcache, int Tmax, float scale,
                 const exl3_weight *o, float *res, float *res_ssq, uint16_t *att, float *scratch,
                 size_t scratch_bytes, hipStream_t s);

/* out = f16(silu(g) * u), n elements. */
int exl3d_silu_mul(const uint16_t *g, const uint16_t *u, uint16_t *out, size_t n, hipStream_t s);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_DECODER_H */
