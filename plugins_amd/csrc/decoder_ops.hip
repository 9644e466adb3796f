// decoder_ops.hip -- the non-EXL3 operations of a Qwen3-8B-shaped decode step
// on MI355X (gfx950, wave64): the harness that BASELINE's decode tok/s config
// runs around the EXL3 linears.  Roles in the reference's model plugin (paths
// relative to /root/reference/plugins/turboexl3_qwen38/src/direct/):
//  * residual add + RMSNorm: linear.zig:65-69 (mlx_fast_rms_norm);
//  * q/k RMSNorm + RoPE and the KV append: attn.zig:133-141, attn_core.zig;
//  * SiLU(gate) * up: linear.zig:71-85;
//  * decode attention: attn_core.zig (MLX's scaled-dot-product attention).
// The arithmetic is the usual fp32-accumulated form of each op; the decode
// step is checked against a float32 PyTorch restatement of the whole step.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/exl3_decoder.h"
#include "exl3_device.h"
#include "exl3_kernels.h"

namespace {

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// h[b] = f32(table[ids[b]])
__global__ __launch_bounds__(256) void embed_kernel(const int32_t *__restrict__ ids,
                                                    const uint16_t *__restrict__ table, int H,
                                                    float *__restrict__ h) {
  const int b = blockIdx.y;
  const size_t row = (size_t)ids[b];
  for (int i = blockIdx.x * 256 + threadIdx.x; i < H; i += gridDim.x * 256)
    h[(size_t)b * H + i] = h2f(table[row * H + i]);
}

// h[b] = f32(table[ids[b]]) with the row's sums of squares per 128 columns
// (the RMSNorm prologue's input): one wave per (row, 128 columns), lane l
// columns 2 l, 2 l + 1, the pair's squares summed over the lanes pairwise.
__global__ __launch_bounds__(64) void embed_ssq_kernel(const int32_t *__restrict__ ids,
                                                       const uint16_t *__restrict__ table, int H,
                                                       float *__restrict__ h,
                                                       float *__restrict__ ssq) {
  const int blk = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const size_t row = (size_t)ids[b];
  const int i = blk * 128 + 2 * lane;
  const uint32_t t2 = *reinterpret_cast<const uint32_t *>(table + row * H + i);
  float2 v;
  v.x = h2f((uint16_t)(t2 & 0xFFFFu));
  v.y = h2f((uint16_t)(t2 >> 16));
  *reinterpret_cast<float2 *>(h + (size_t)b * H + i) = v;
  float ss = v.x * v.x + v.y * v.y;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) ss += __shfl_xor(ss, m, 64);
  if (lane == 0) ssq[(size_t)b * (H / 128) + blk] = ss;
}

// h += add (f16, optional); out = f16(h * rsqrt(mean(h^2) + eps) * w).
// One workgroup of 512 threads per row; each thread loads its 8-element
// pieces (two float4 of h, 16 bytes of add and of w) before any arithmetic,
// so a row costs one memory round trip and one reduction.
constexpr int RN_THREADS = 512;
constexpr int RN_PER = 2;  // 8-element pieces per thread: rows up to 8192

// Consumers of the normalized rows (PREP): each gets the rows prepared with
// its suh, set c of xp at c * rows * H.
struct PrepTo {
  const uint16_t *suh[4];
  uint16_t *xp;
  int count;
};

template <bool PREP>
__global__ __launch_bounds__(RN_THREADS) void add_rmsnorm_kernel(float *__restrict__ h,
                                                                 const uint16_t *__restrict__ add,
                                                                 const uint16_t *__restrict__ w,
                                                                 uint16_t *__restrict__ out, int H,
                                                                 float eps, PrepTo pt) {
  __shared__ float part[RN_THREADS / 64];
  float *hr = h + (size_t)blockIdx.x * H;
  const uint16_t *ar = add ? add + (size_t)blockIdx.x * H : nullptr;
  float v[RN_PER][8];
  uint4 wr[RN_PER];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < RN_PER; ++j) {
    const int i = (threadIdx.x + j * RN_THREADS) * 8;
    if (i < H) {
      const float4 h0 = *reinterpret_cast<const float4 *>(hr + i);
      const float4 h1 = *reinterpret_cast<const float4 *>(hr + i + 4);
      v[j][0] = h0.x, v[j][1] = h0.y, v[j][2] = h0.z, v[j][3] = h0.w;
      v[j][4] = h1.x, v[j][5] = h1.y, v[j][6] = h1.z, v[j][7] = h1.w;
      wr[j] = *reinterpret_cast<const uint4 *>(w + i);
      if (ar) {
        const uint4 a4 = *reinterpret_cast<const uint4 *>(ar + i);
        const uint32_t aw[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[j][2 * e] += h2f((uint16_t)(aw[e] & 0xFFFFu));
          v[j][2 * e + 1] += h2f((uint16_t)(aw[e] >> 16));
        }
        *reinterpret_cast<float4 *>(hr + i) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
        *reinterpret_cast<float4 *>(hr + i + 4) = make_float4(v[j][4], v[j][5], v[j][6], v[j][7]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[j][e] * v[j][e];
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < RN_THREADS / 64; ++i) tot += part[i];
  const float r = rsqrtf(tot / (float)H + eps);
  uint16_t *orow = out + (size_t)blockIdx.x * H;
#pragma unroll
  for (int j = 0; j < RN_PER; ++j) {
    const int i = (threadIdx.x + j * RN_THREADS) * 8;
    if (i < H) {
      const uint32_t ww[4] = {wr[j].x, wr[j].y, wr[j].z, wr[j].w};
      uint32_t o4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o4[e] = (uint32_t)f2h(v[j][2 * e] * r * h2f((uint16_t)(ww[e] & 0xFFFFu))) |
                ((uint32_t)f2h(v[j][2 * e + 1] * r * h2f((uint16_t)(ww[e] >> 16))) << 16);
      if constexpr (PREP) {
        // H a multiple of 512: a wave's 64 lanes are all in range here, and
        // 16 consecutive lanes hold one 128-block
        for (int c = 0; c < pt.count; ++c) {
          const uint4 su = *reinterpret_cast<const uint4 *>(pt.suh[c] + i);
          const uint4 pv = exl3::prep_block8(o4, su, (int)(threadIdx.x & 15));
          *reinterpret_cast<uint4 *>(pt.xp + ((size_t)c * gridDim.x + blockIdx.x) * H + i) = pv;
        }
      } else {
        *reinterpret_cast<uint4 *>(orow + i) = make_uint4(o4[0], o4[1], o4[2], o4[3]);
      }
    }
  }
}

// One wave per (head, row): lane holds dims lane and lane + D/2 (the
// rotate-half pairs).  q heads: RMSNorm (qn), RoPE, to qout; k heads: RMSNorm
// (kn), RoPE, to kcache at position pos[b]; v heads: copied to vcache.
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const uint16_t *__restrict__ qn, const uint16_t *__restrict__ kn,
    const int32_t *__restrict__ pos, int nq, int nkv, float eps, float theta,
    uint16_t *__restrict__ qout, uint16_t *__restrict__ kcache, uint16_t *__restrict__ vcache,
    int Tmax) {
  constexpr int D = EXL3D_HEAD_DIM, HALF = D / 2;
  const int lane = threadIdx.x, hd = blockIdx.x, b = blockIdx.y;
  const int p = pos[b];
  if (hd >= nq + nkv) {  // v head: copy into the cache
    const int vh = hd - nq - nkv;
    const uint16_t *src = v + ((size_t)b * nkv + vh) * D;
    uint16_t *dst = vcache + (((size_t)b * nkv + vh) * Tmax + p) * D;
    dst[lane] = src[lane];
    dst[lane + HALF] = src[lane + HALF];
    return;
  }
  const bool isq = hd < nq;
  const uint16_t *src = isq ? q + ((size_t)b * nq + hd) * D : k + ((size_t)b * nkv + (hd - nq)) * D;
  const uint16_t *nw = isq ? qn : kn;
  float x0 = h2f(src[lane]), x1 = h2f(src[lane + HALF]);
  const float r = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / (float)D + eps);
  x0 = h2f(f2h(x0 * r * h2f(nw[lane])));
  x1 = h2f(f2h(x1 * r * h2f(nw[lane + HALF])));
  // angle = pos * theta^(-2 lane / D)
  const float inv = powf(theta, -2.0f * (float)lane / (float)D);
  float sn, cs;
  sincosf((float)p * inv, &sn, &cs);
  const float y0 = x0 * cs - x1 * sn, y1 = x1 * cs + x0 * sn;
  uint16_t *dst = isq ? qout + ((size_t)b * nq + hd) * D
                      : kcache + (((size_t)b * nkv + (hd - nq)) * Tmax + p) * D;
  dst[lane] = f2h(y0);
  dst[lane + HALF] = f2h(y1);
}

// The q/k norm + RoPE of one head's dims 8 li .. 8 li + 7 held by the 16
// lanes of a key group (lane li): RMSNorm with weight nw (sum of squares over
// the 16 lanes), f16, then rotate-half RoPE with the pair partner in lane
// li ^ 8 (dims d and d + 64), f16.  sn / cs: the lane's 8 angles.
__device__ __forceinline__ void norm_rope8(float (&x)[8], const uint4 nw, const float (&sn)[8],
                                           const float (&cs)[8], int li, float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  const float r = rsqrtf(ss / (float)EXL3D_HEAD_DIM + eps);
  const uint32_t w4[4] = {nw.x, nw.y, nw.z, nw.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float wv = h2f((uint16_t)(e & 1 ? w4[e >> 1] >> 16 : w4[e >> 1] & 0xFFFFu));
    x[e] = h2f(f2h(x[e] * r * wv));
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float pr = __shfl_xor(x[e], 8, 64);
    x[e] = li < 8 ? x[e] * cs[e] - pr * sn[e] : x[e] * cs[e] + pr * sn[e];
    x[e] = h2f(f2h(x[e]));
  }
}

// Sum over the 16 lanes of a DPP row (a key group), in every lane of it:
// quad permutations for lanes i ^ 1 and i ^ 2, then the half-row mirror
// (i with 7 - i) and the row mirror (i with 15 - i).  VALU data movement, no
// LDS; every lane adds the same pairs, so all 16 hold the same value.
__device__ __forceinline__ float row16_sum(float v) {
  auto dpp = [](float x, auto CTRL) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), decltype(CTRL)::value, 0xF,
                                        0xF, false));
  };
  v += dpp(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1, 0, 3, 2]
  v += dpp(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2, 3, 0, 1]
  v += dpp(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
  v += dpp(v, std::integral_constant<int, 0x140>{});  // row_mirror
  return v;
}

__device__ __forceinline__ void unpack8(const uint4 raw, float (&x)[8]) {
  const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = h2f((uint16_t)(w4[e] & 0xFFFFu));
    x[2 * e + 1] = h2f((uint16_t)(w4[e] >> 16));
  }
}
__device__ __forceinline__ uint4 pack8(const float (&x)[8]) {
  uint32_t w4[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) w4[e] = (uint32_t)f2h(x[2 * e]) | ((uint32_t)f2h(x[2 * e + 1]) << 16);
  return make_uint4(w4[0], w4[1], w4[2], w4[3]);
}

// The raw projections and norm weights of the q/k norm + RoPE that the
// attention kernel applies itself (ROPE).
struct RopeArgs {
  const uint16_t *k, *v;    // [B][nkv * D]
  const uint16_t *qn, *kn;  // [D]
  float eps, theta;
};

// Split-T decode attention, grouped-query: a workgroup (4 waves) takes one
// (row b, kv head) and keys [s TS, min((s + 1) TS, L)), L = pos[b] + 1, for
// the G = nq / nkv query heads that share the kv head.  Lane l of a wave:
// key group l / 16 (four keys per wave per iteration), dims 8 (l % 16) ..
// +7.  Online softmax per (key group, head) in f32; the 16 partial states of
// the workgroup merge in LDS into (m, l, o[D]) per head, stored in the
// split's slot; attn_combine_kernel, its own launch, combines the slots.
// (The kernel boundary is the hand-off: having the last-arriving split
// combine behind an agent-scope ticket measured ~1 us a layer slower at
// batch 1, its atomic and coherent loads each a round trip.)
// ROPE: q arrives raw; every workgroup applies the q norm and RoPE to its
// heads, and the workgroup of the split holding key pos[b] also normalizes,
// rotates and appends that key (and copies the value) into the caches first.
constexpr int AT_G = 4;  // query heads per kv head (Qwen3-8B: 32 / 8)
constexpr int AC_MAXS = 256;  // splits
constexpr int AT_KD = 4;  // key rows in flight per key group

template <bool ROPE>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const uint16_t *__restrict__ q, uint16_t *__restrict__ kcache, uint16_t *__restrict__ vcache,
    const int32_t *__restrict__ pos, int nq, int nkv, int Tmax, int TS, float scale, RopeArgs ra,
    float *__restrict__ part) {
  constexpr int D = EXL3D_HEAD_DIM;
  __shared__ float sm[16][AT_G][D + 2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int p = pos[b];
  const int L = p + 1;
  const int t0 = s * TS, t1 = min(t0 + TS, L);
  const int nsplit = gridDim.x;
  float qr[AT_G][8];
#pragma unroll
  for (int h = 0; h < AT_G; ++h)
    unpack8(*reinterpret_cast<const uint4 *>(q + ((size_t)b * nq + kvh * AT_G + h) * D + 8 * li),
            qr[h]);
  const size_t kvbase = ((size_t)b * nkv + kvh) * Tmax;
  auto ld = [&](const uint16_t *c, int t) {
    return *reinterpret_cast<const uint4 *>(c + (kvbase + t) * D + 8 * li);
  };
  // The key group's keys t, t + 16, ...: AT_KD of them in flight (a split of
  // 64 keys is loaded at once), each reloaded AT_KD keys ahead once used;
  // keys past the split's end reload its last key (in bounds, unused).  The
  // first ones go out at once, bounded by the cache's rows rather than by
  // pos[b] (so they need not wait for it; rows past the split's end are
  // loaded and not used), before the q/k prologue.
  const int tg = t0 + 4 * wave + g;
  uint4 kr[AT_KD], vr[AT_KD];
#pragma unroll
  for (int j = 0; j < AT_KD; ++j) {
    kr[j] = ld(kcache, min(tg + 16 * j, Tmax - 1));
    vr[j] = ld(vcache, min(tg + 16 * j, Tmax - 1));
  }
  if constexpr (ROPE) {
    // the norm weights, and the new key and value the split holding key
    // pos[b] appends, loaded with the keys (before any wait)
    const uint4 qn = *reinterpret_cast<const uint4 *>(ra.qn + 8 * li);
    const uint4 kn = *reinterpret_cast<const uint4 *>(ra.kn + 8 * li);
    const bool appends = s == p / TS;
    const size_t kvrow = ((size_t)b * nkv + kvh) * D + 8 * li;
    uint4 kraw = make_uint4(0, 0, 0, 0), vnew = make_uint4(0, 0, 0, 0);
    if (appends) {
      kraw = *reinterpret_cast<const uint4 *>(ra.k + kvrow);
      vnew = *reinterpret_cast<const uint4 *>(ra.v + kvrow);
    }
    // angle of dim d: pos * theta^(-2 (d mod 64) / D), the 64 angles once
    // per workgroup (the argument reaches thousands of radians, where a sine
    // costs a long reduction)
    __shared__ float sc_sn[D / 2], sc_cs[D / 2];
    if (threadIdx.x < D / 2) {
      const float inv = powf(ra.theta, -2.0f * (float)threadIdx.x / (float)D);
      sincosf((float)p * inv, &sc_sn[threadIdx.x], &sc_cs[threadIdx.x]);
    }
    __syncthreads();
    float sn[8], cs[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = (8 * li + e) & (D / 2 - 1);
      sn[e] = sc_sn[i];
      cs[e] = sc_cs[i];
    }
#pragma unroll
    for (int h = 0; h < AT_G; ++h) norm_rope8(qr[h], qn, sn, cs, li, ra.eps);
    if (appends) {
      float kx[8];
      unpack8(kraw, kx);
      norm_rope8(kx, kn, sn, cs, li, ra.eps);
      const uint4 knew = pack8(kx);
      if (wave == 0 && g == 0) {
        *reinterpret_cast<uint4 *>(kcache + (kvbase + p) * D + 8 * li) = knew;
        *reinterpret_cast<uint4 *>(vcache + (kvbase + p) * D + 8 * li) = vnew;
      }
      // row p in the ring was loaded before it was written: take it from
      // registers; later reloads read it from the cache (after the barrier)
#pragma unroll
      for (int j = 0; j < AT_KD; ++j) {
        if (tg + 16 * j == p) {
          kr[j] = knew;
          vr[j] = vnew;
        }
      }
      __syncthreads();
    }
  }
  // q is f16-exact here (the raw f16 rows, or norm_rope8's f16 rounding):
  // packed in pairs for v_dot2_f32_f16 against the keys' packed halves; the
  // scale multiplies the summed score
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  h2_t qh[AT_G][4];
#pragma unroll
  for (int h = 0; h < AT_G; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      qh[h][i] = __builtin_bit_cast(h2_t, (uint32_t)f2h(qr[h][2 * i]) |
                                              ((uint32_t)f2h(qr[h][2 * i + 1]) << 16));
  float m[AT_G], l[AT_G], o[AT_G][8];
#pragma unroll
  for (int h = 0; h < AT_G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
  }
  if (t0 < t1) {
    // AT_KD keys of the key group at a time: their AT_KD x AT_G scores are
    // independent (formed side by side), then one online-softmax update per
    // head takes all of them (keys past the split's end score -inf and weigh
    // 0; the first key of a block is always in range, so the new maximum is
    // finite).  Products of f16 halves summed in f32 (v_dot2_f32_f16); the
    // weights rounded to f16 for the value sums (pairs of keys per dot2),
    // and the same rounded weights summed into l.
    static_assert(AT_KD % 2 == 0, "value sums take keys in pairs");
    for (int tb = tg; tb < t1; tb += 16 * AT_KD) {
      float sc[AT_KD][AT_G];
      h2_t vp[AT_KD / 2][8];
#pragma unroll
      for (int j = 0; j < AT_KD; ++j) {
        const int t = tb + 16 * j;
        const uint32_t kw[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
        if (j & 1) {
          // dims 2i / 2i + 1 of keys j - 1 and j in one pair each
          const uint32_t a[4] = {vr[j - 1].x, vr[j - 1].y, vr[j - 1].z, vr[j - 1].w};
          const uint32_t b[4] = {vr[j].x, vr[j].y, vr[j].z, vr[j].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            vp[j >> 1][2 * i] =
                __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(b[i], a[i], 0x05040100u));
            vp[j >> 1][2 * i + 1] =
                __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(b[i], a[i], 0x07060302u));
          }
        }
        const int tn = min(t + 16 * AT_KD, t1 - 1);
        kr[j] = ld(kcache, tn);
        if (j & 1) {
          vr[j - 1] = ld(vcache, min(t - 16 + 16 * AT_KD, t1 - 1));
          vr[j] = ld(vcache, tn);
        }
#pragma unroll
        for (int h = 0; h < AT_G; ++h) {
          float d = 0.0f;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            d = __builtin_amdgcn_fdot2(qh[h][i], __builtin_bit_cast(h2_t, kw[i]), d, false);
          sc[j][h] = row16_sum(d) * scale;
          if (t >= t1) sc[j][h] = -INFINITY;
        }
      }
#pragma unroll
      for (int h = 0; h < AT_G; ++h) {
        float mn = m[h];
#pragma unroll
        for (int j = 0; j < AT_KD; ++j) mn = fmaxf(mn, sc[j][h]);
        const float c = __expf(m[h] - mn);
        uint32_t pb[AT_KD];
        float ps = 0.0f;
#pragma unroll
        for (int j = 0; j < AT_KD; ++j) {
          pb[j] = f2h(__expf(sc[j][h] - mn));
          ps += h2f((uint16_t)pb[j]);
        }
        l[h] = fmaf(l[h], c, ps);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float a = o[h][e] * c;
#pragma unroll
          for (int jp = 0; jp < AT_KD / 2; ++jp)
            a = __builtin_amdgcn_fdot2(
                __builtin_bit_cast(h2_t, pb[2 * jp] | (pb[2 * jp + 1] << 16)), vp[jp][e], a, false);
          o[h][e] = a;
        }
        m[h] = mn;
      }
    }
  }
  // merge the 16 states (4 waves x 4 key groups) per head
  const int st = wave * 4 + g;
#pragma unroll
  for (int h = 0; h < AT_G; ++h) {
#pragma unroll
    for (int e = 0; e < 8; ++e) sm[st][h][8 * li + e] = o[h][e];
    if (li == 0) {
      sm[st][h][D] = m[h];
      sm[st][h][D + 1] = l[h];
    }
  }
  __syncthreads();
  // thread t: head t / 64, dims 2 (t % 64), +1
  const int h = threadIdx.x >> 6, d = 2 * (threadIdx.x & 63);
  float M = -INFINITY;
  for (int i = 0; i < 16; ++i) M = fmaxf(M, sm[i][h][D]);
  float Ls = 0.0f, a0 = 0.0f, a1 = 0.0f;
  if (M != -INFINITY) {
    for (int i = 0; i < 16; ++i) {
      const float f = __expf(sm[i][h][D] - M);
      Ls += sm[i][h][D + 1] * f;
      a0 += sm[i][h][d] * f;
      a1 += sm[i][h][d + 1] * f;
    }
  }
  const size_t sstride = (size_t)AT_G * (D + 2);
  float *slots = part + ((size_t)b * nkv + kvh) * nsplit * sstride;
  float *dst = slots + s * sstride + h * (D + 2);
  dst[d] = a0;
  dst[d + 1] = a1;
  if (d == 0) {
    dst[D] = M;
    dst[D + 1] = Ls;
  }
}

// The split combine, its own launch: out[b][head][d] = sum_s o_s e^(m_s - M)
// / sum_s l_s e^(m_s - M), f16.  One workgroup per (row, kv head): the
// splits' m and l go through LDS, each thread's o values of 32 splits at a
// time are in flight together, and every sum runs in split order.
// suh set: out gets the combined rows prepared for the consumer linear
// (its suh over the nq * D inputs; the GEMV reads them as prepared rows):
// each head is one 128-block, prepared by wave 0 (16 lanes a head).
__global__ __launch_bounds__(AT_G * EXL3D_HEAD_DIM) void attn_combine_kernel(
    const float *__restrict__ part, int nq, int nkv, int nsplit, uint16_t *__restrict__ out,
    const uint16_t *__restrict__ suh) {
  constexpr int D = EXL3D_HEAD_DIM;
  constexpr int CH = 32;  // splits whose o values a thread has in flight at once
  __shared__ float msh[AT_G][AC_MAXS], lsh[AT_G][AC_MAXS];
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int h = threadIdx.x / D, d = threadIdx.x % D;
  const float *base = part + ((size_t)b * nkv + kvh) * nsplit * AT_G * (D + 2);
  const size_t sstride = (size_t)AT_G * (D + 2);
  // one round of loads: the first CH splits' o values of this thread, and
  // every split's (m, l) of every head (spread over the threads)
  float ov[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) ov[j] = base[(size_t)min(j, nsplit - 1) * sstride + h * (D + 2) + d];
  for (int i = threadIdx.x; i < AT_G * nsplit; i += AT_G * D) {
    const int hh = i % AT_G, s = i / AT_G;
    const float *ml = base + s * sstride + hh * (D + 2) + D;
    msh[hh][s] = ml[0];
    lsh[hh][s] = ml[1];
  }
  __syncthreads();
  // out = sum_s o_s f_s / sum_s l_s f_s, f_s = e^(m_s - M), in split order
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, msh[h][s]);
  float Ls = 0.0f, acc = 0.0f;
  for (int s0 = 0; s0 < nsplit; s0 += CH) {
    if (s0 > 0) {
#pragma unroll
      for (int j = 0; j < CH; ++j)
        ov[j] = base[(size_t)min(s0 + j, nsplit - 1) * sstride + h * (D + 2) + d];
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (s0 + j < nsplit) {
        const float ms = msh[h][s0 + j];
        const float f = ms == -INFINITY ? 0.0f : __expf(ms - M);
        Ls += lsh[h][s0 + j] * f;
        acc += ov[j] * f;
      }
    }
  }
  const uint16_t y = f2h(acc / Ls);
  if (suh == nullptr) {
    out[((size_t)b * nq + kvh * AT_G + h) * D + d] = y;
    return;
  }
  static_assert(AT_G * 16 == 64, "one wave prepares the workgroup's heads");
  __shared__ __attribute__((aligned(16))) uint16_t ob[AT_G][D];
  ob[h][d] = y;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int hh = threadIdx.x >> 4, j = threadIdx.x & 15;
    const uint4 xv = *reinterpret_cast<const uint4 *>(&ob[hh][8 * j]);
    const uint32_t xo[4] = {xv.x, xv.y, xv.z, xv.w};
    const size_t col = (size_t)(kvh * AT_G + hh) * D + 8 * j;
    const uint4 su = *reinterpret_cast<const uint4 *>(suh + col);
    *reinterpret_cast<uint4 *>(out + (size_t)b * nq * D + col) = exl3::prep_block8(xo, su, j);
  }
}


__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ g,
                                                       const uint16_t *__restrict__ u,
                                                       uint16_t *__restrict__ out, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const float gv = h2f(g[i]);
    out[i] = f2h(gv / (1.0f + __expf(-gv)) * h2f(u[i]));
  }
}

// The device's compute units (256 on MI355X), read once per device.
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Workgroups of the attention kernel resident at once on the device (its
// registers allow 3 a CU on gfx950), read once per device.
int attn_resident_wgs() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return device_cus();
  if (cached[dev] == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void *>(&attn_decode_kernel<true>), 256, 0) != hipSuccess ||
        n <= 0)
      n = 1;
    cached[dev] = n * device_cus();
  }
  return cached[dev];
}

int attn_split(int Tmax, int B, int nkv, int *TS) {
  // keys per split: a power of two >= 128 (each key group's 4 keys in
  // flight twice), at most ~2048 workgroups overall (each is bound by its
  // own memory round trips, so many in flight), at most AC_MAXS splits.
  // Fewer splits leave fewer slots for the o projection's prologue to
  // combine (each of its column groups reads its heads' slots): at batch 1,
  // context 2048, 16 splits of 128 keys took 2.27 ms a step against 2.31
  // with 32 of 64 and 2.35 with 8 of 256.
  int ts = 128;
  while (((long)((Tmax + ts - 1) / ts) * B * nkv > 2048 || (Tmax + ts - 1) / ts > AC_MAXS))
    ts *= 2;
  // then whole rounds of resident workgroups: the few workgroups past a
  // round would finish last (at batch 1, context 2048: 33 x 8 = 264
  // workgroups ran ~4 us behind on 8 CUs); the splits grow so the grid is
  // the round count below it times the resident workgroups (at batch 16,
  // context 2048: 6 splits, 768 workgroups, 4.08 ms a step against 4.16
  // with 8 splits, 1024 workgroups, counted in rounds of the 256 CUs)
  const long per = (long)B * nkv;
  const int cus = attn_resident_wgs();
  const long wgs = (long)((Tmax + ts - 1) / ts) * per;
  const long rounds = wgs / cus;
  if (rounds >= 1) {
    const long ns = rounds * cus / per;
    if (ns >= 1 && ns < (Tmax + ts - 1) / ts) ts = (int)((Tmax + ns - 1) / ns);
  }
  *TS = ts;
  return (Tmax + ts - 1) / ts;
}


size_t attn_slot_floats(int B, int nkv, int ns) {
  return (size_t)B * nkv * ns * AT_G * (EXL3D_HEAD_DIM + 2);
}

int attn_launch(bool rope, const uint16_t *q, const RopeArgs &ra, uint16_t *kcache,
                uint16_t *vcache, const int32_t *pos, int B, int nq, int nkv, int Tmax, float scale,
                uint16_t *out, float *scratch, size_t scratch_bytes, hipStream_t s) {
  if (B <= 0 || nkv <= 0 || nq != AT_G * nkv || B > 65535 || nkv > 65535 || Tmax <= 0)
    return hipErrorInvalidValue;
  if (scratch_bytes < exl3d_attn_scratch_bytes(B, nq, nkv, Tmax)) return hipErrorInvalidValue;
  int ts;
  const int ns = attn_split(Tmax, B, nkv, &ts);
  const dim3 grid(ns, nkv, B);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, q, kcache, vcache, pos, nq, nkv, Tmax, ts,
                       scale, ra, scratch);
  };
  if (rope)
    go(attn_decode_kernel<true>);
  else
    go(attn_decode_kernel<false>);
  // out NULL: the slots stay for a consumer that combines them itself (the
  // o projection's attention prologue)
  if (out != nullptr)
    hipLaunchKernelGGL(attn_combine_kernel, dim3(nkv, B), dim3(AT_G * EXL3D_HEAD_DIM), 0, s,
                       scratch, nq, nkv, ns, out, (const uint16_t *)nullptr);
  return hipGetLastError();
}

}  // namespace

extern "C" {

int exl3d_embed(const int32_t *ids, int B, const uint16_t *table, int H, float *h, float *ssq,
                hipStream_t s) {
  if (B <= 0 || H <= 0 || B > 65535) return hipErrorInvalidValue;
  if (ssq != nullptr) {
    if (H % 128 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_ssq_kernel, dim3(H / 128, B), dim3(64), 0, s, ids, table, H, h, ssq);
  } else {
    hipLaunchKernelGGL(embed_kernel, dim3((H + 255) / 256, B), dim3(256), 0, s, ids, table, H, h);
  }
  return hipGetLastError();
}

int exl3d_add_rmsnorm(float *h, const uint16_t *add, const uint16_t *w, uint16_t *out, int B,
                      int H, float eps, hipStream_t s) {
  if (B <= 0 || H <= 0 || H % 8 != 0 || H > RN_THREADS * RN_PER * 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(add_rmsnorm_kernel<false>, dim3(B), dim3(RN_THREADS), 0, s, h, add, w, out, H,
                     eps, PrepTo{});
  return hipGetLastError();
}

int exl3d_qk_norm_rope(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *qn,
                       const uint16_t *kn, const int32_t *pos, int B, int nq, int nkv, float eps,
                       float theta, uint16_t *qout, uint16_t *kcache, uint16_t *vcache,
                       int Tmax, hipStream_t s) {
  if (B <= 0 || nq <= 0 || nkv <= 0 || B > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(nq + 2 * nkv, B), dim3(64), 0, s, q, k, v, qn, kn,
                     pos, nq, nkv, eps, theta, qout, kcache, vcache, Tmax);
  return hipGetLastError();
}

int exl3d_attn_splits(int B, int nkv, int Tmax) {
  if (B <= 0 || nkv <= 0 || Tmax <= 0) return 0;
  int ts;
  return attn_split(Tmax, B, nkv, &ts);
}

int exl3d_attn_heads_per_kv(void) { return AT_G; }

size_t exl3d_attn_scratch_bytes(int B, int nq, int nkv, int Tmax) {
  int ts;
  const int ns = attn_split(Tmax, B, nkv, &ts);
  return attn_slot_floats(B, nkv, ns) * sizeof(float);
}

int exl3d_attn_decode(const uint16_t *q, const uint16_t *kcache, const uint16_t *vcache,
                      const int32_t *pos, int B, int nq, int nkv, int Tmax, float scale,
                      uint16_t *out, float *scratch, size_t scratch_bytes, hipStream_t s) {
  // the caches are only read without ROPE
  return attn_launch(false, q, RopeArgs{}, const_cast<uint16_t *>(kcache),
                     const_cast<uint16_t *>(vcache), pos, B, nq, nkv, Tmax, scale, out, scratch,
                     scratch_bytes, s);
}

int exl3d_attn_decode_rope(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                           const uint16_t *qn, const uint16_t *kn, const int32_t *pos, int B,
                           int nq, int nkv, float eps, float theta, uint16_t *kcache,
                           uint16_t *vcache, int Tmax, float scale, uint16_t *out, float *scratch,
                           size_t scratch_bytes, hipStream_t s) {
  const RopeArgs ra{k, v, qn, kn, eps, theta};
  return attn_launch(true, q, ra, kcache, vcache, pos, B, nq, nkv, Tmax, scale, out, scratch,
                     scratch_bytes, s);
}

int exl3d_silu_mul(const uint16_t *g, const uint16_t *u, uint16_t *out, size_t n, hipStream_t s) {
  if (n == 0) return hipErrorInvalidValue;
  const size_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256),
                     0, s, g, u, out, n);
  return hipGetLastError();
}

}  // extern "C"

namespace exl3 {

hipError_t launch_attn_combine_prepare(const float *part, int B, int nq, int nkv, int Tmax,
                                       const uint16_t *suh, uint16_t *xp, hipStream_t s) {
  if (B <= 0 || B > 65535 || nkv <= 0 || nq != AT_G * nkv || suh == nullptr || xp == nullptr)
    return hipErrorInvalidValue;
  int ts;
  const int ns = attn_split(Tmax, B, nkv, &ts);
  hipLaunchKernelGGL(attn_combine_kernel, dim3(nkv, B), dim3(AT_G * EXL3D_HEAD_DIM), 0, s, part,
                     nq, nkv, ns, xp, suh);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_prepare(const float *h, const uint16_t *w, int B, int H, float eps,
                                  const uint16_t *const *suh, int count, uint16_t *xp,
                                  hipStream_t s) {
  if (B <= 0 || B > 65535 || H <= 0 || H % 512 != 0 || H > RN_THREADS * RN_PER * 8 ||
      count < 1 || count > 4 || xp == nullptr)
    return hipErrorInvalidValue;
  PrepTo pt{};
  for (int c = 0; c < count; ++c) {
    if (suh[c] == nullptr) return hipErrorInvalidValue;
    pt.suh[c] = suh[c];
  }
  pt.xp = xp;
  pt.count = count;
  hipLaunchKernelGGL(add_rmsnorm_kernel<true>, dim3(B), dim3(RN_THREADS), 0, s,
                     const_cast<float *>(h), nullptr, w, nullptr, H, eps, pt);
  return hipGetLastError();
}

}  // namespace exl3
