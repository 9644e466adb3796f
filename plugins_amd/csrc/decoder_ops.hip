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

#include "../../include/exl3_decoder.h"

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

// h += add (f16, optional); out = f16(h * rsqrt(mean(h^2) + eps) * w).
// One workgroup of 512 threads per row; each thread loads its 8-element
// pieces (two float4 of h, 16 bytes of add and of w) before any arithmetic,
// so a row costs one memory round trip and one reduction.
constexpr int RN_THREADS = 512;
constexpr int RN_PER = 2;  // 8-element pieces per thread: rows up to 8192

__global__ __launch_bounds__(RN_THREADS) void add_rmsnorm_kernel(float *__restrict__ h,
                                                                 const uint16_t *__restrict__ add,
                                                                 const uint16_t *__restrict__ w,
                                                                 uint16_t *__restrict__ out, int H,
                                                                 float eps) {
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
      *reinterpret_cast<uint4 *>(orow + i) = make_uint4(o4[0], o4[1], o4[2], o4[3]);
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

// Split-T decode attention, grouped-query: a workgroup (4 waves) takes one
// (row b, kv head) and keys [s TS, min((s + 1) TS, L)), L = pos[b] + 1, for
// the G = nq / nkv query heads that share the kv head.  Lane l of a wave:
// key group l / 16 (four keys per wave per iteration), dims 8 (l % 16) ..
// +7.  Online softmax per (key group, head) in f32; the 16 partial states of
// the workgroup merge in LDS and go out as (m, l, o[D]) per head.
constexpr int AT_G = 4;  // query heads per kv head (Qwen3-8B: 32 / 8)

__global__ __launch_bounds__(256) void attn_decode_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ kcache,
    const uint16_t *__restrict__ vcache, const int32_t *__restrict__ pos, int nq, int nkv,
    int Tmax, int TS, float scale, float *__restrict__ part) {
  constexpr int D = EXL3D_HEAD_DIM;
  __shared__ float sm[16][AT_G][D + 2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int L = pos[b] + 1;
  const int t0 = s * TS, t1 = min(t0 + TS, L);
  const int nsplit = gridDim.x;
  float qr[AT_G][8];
#pragma unroll
  for (int h = 0; h < AT_G; ++h) {
    const uint4 raw =
        *reinterpret_cast<const uint4 *>(q + ((size_t)b * nq + kvh * AT_G + h) * D + 8 * li);
    const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qr[h][2 * e] = h2f((uint16_t)(w4[e] & 0xFFFFu)) * scale;
      qr[h][2 * e + 1] = h2f((uint16_t)(w4[e] >> 16)) * scale;
    }
  }
  float m[AT_G], l[AT_G], o[AT_G][8];
#pragma unroll
  for (int h = 0; h < AT_G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
  }
  const size_t kvbase = ((size_t)b * nkv + kvh) * Tmax;
  auto ld = [&](const uint16_t *c, int t) {
    return *reinterpret_cast<const uint4 *>(c + (kvbase + t) * D + 8 * li);
  };
  int t = t0 + 4 * wave + g;
  if (t0 < t1) {
    // the next key's rows are loaded before this one is processed (clamped
    // to the split's last key: in bounds, unused past the end)
    uint4 kr = ld(kcache, min(t, t1 - 1)), vr = ld(vcache, min(t, t1 - 1));
    for (; t < t1; t += 16) {
      const int tn = min(t + 16, t1 - 1);
      const uint4 krn = ld(kcache, tn), vrn = ld(vcache, tn);
      const uint32_t kw[4] = {kr.x, kr.y, kr.z, kr.w};
      const uint32_t vw[4] = {vr.x, vr.y, vr.z, vr.w};
      float kf[8], vf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kf[2 * e] = h2f((uint16_t)(kw[e] & 0xFFFFu));
        kf[2 * e + 1] = h2f((uint16_t)(kw[e] >> 16));
        vf[2 * e] = h2f((uint16_t)(vw[e] & 0xFFFFu));
        vf[2 * e + 1] = h2f((uint16_t)(vw[e] >> 16));
      }
#pragma unroll
      for (int h = 0; h < AT_G; ++h) {
        float sc = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sc += qr[h][e] * kf[e];
#pragma unroll
        for (int mk = 8; mk >= 1; mk >>= 1) sc += __shfl_xor(sc, mk, 64);  // over the 16 lanes
        const float mn = fmaxf(m[h], sc);
        const float c = __expf(m[h] - mn), pr = __expf(sc - mn);
        l[h] = l[h] * c + pr;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = o[h][e] * c + pr * vf[e];
        m[h] = mn;
      }
      kr = krn;
      vr = vrn;
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
  float *dst = part + ((((size_t)b * nkv + kvh) * nsplit + s) * AT_G + h) * (D + 2);
  dst[d] = a0;
  dst[d + 1] = a1;
  if (d == 0) {
    dst[D] = M;
    dst[D + 1] = Ls;
  }
}

// out[b][head][d] = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M), f16.  One
// workgroup per (row, kv head): the splits' m and l go through LDS (loaded in
// parallel), then thread (head, d) sums its o over the splits, the loads
// unrolled so that several are in flight.
constexpr int AC_MAXS = 256;  // splits the combine takes

__global__ __launch_bounds__(AT_G * EXL3D_HEAD_DIM) void attn_combine_kernel(
    const float *__restrict__ part, int nq, int nkv, int nsplit, uint16_t *__restrict__ out) {
  constexpr int D = EXL3D_HEAD_DIM;
  __shared__ float wsh[AT_G][AC_MAXS];
  __shared__ float lsum[AT_G];
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int h = threadIdx.x / D, d = threadIdx.x % D;
  const float *base = part + ((size_t)b * nkv + kvh) * nsplit * AT_G * (D + 2);
  const size_t sstride = (size_t)AT_G * (D + 2);
  for (int i = threadIdx.x; i < AT_G * nsplit; i += AT_G * D) {
    const int hh = i % AT_G, s = i / AT_G;
    wsh[hh][s] = base[s * sstride + hh * (D + 2) + D];
  }
  __syncthreads();
  if (d == 0) {
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, wsh[h][s]);
    float Ls = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
      const float ms = wsh[h][s];
      const float f = ms == -INFINITY ? 0.0f : __expf(ms - M);
      Ls += base[s * sstride + h * (D + 2) + D + 1] * f;
      wsh[h][s] = f;
    }
    lsum[h] = Ls;
  }
  __syncthreads();
  float acc = 0.0f;
#pragma unroll 8
  for (int s = 0; s < nsplit; ++s) acc += base[s * sstride + h * (D + 2) + d] * wsh[h][s];
  out[((size_t)b * nq + kvh * AT_G + h) * D + d] = f2h(acc / lsum[h]);
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ g,
                                                       const uint16_t *__restrict__ u,
                                                       uint16_t *__restrict__ out, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const float gv = h2f(g[i]);
    out[i] = f2h(gv / (1.0f + __expf(-gv)) * h2f(u[i]));
  }
}

int attn_split(int Tmax, int B, int nkv, int *TS) {
  // keys per split: a power of two >= 64 (four iterations of the
  // workgroup's 16 keys), at most ~2048 workgroups overall (each is bound
  // by its own memory round trips, so many in flight), at most AC_MAXS
  // splits
  int ts = 64;
  while (((long)((Tmax + ts - 1) / ts) * B * nkv > 2048 || (Tmax + ts - 1) / ts > AC_MAXS))
    ts *= 2;
  *TS = ts;
  return (Tmax + ts - 1) / ts;
}

}  // namespace

extern "C" {

int exl3d_embed(const int32_t *ids, int B, const uint16_t *table, int H, float *h,
                hipStream_t s) {
  if (B <= 0 || H <= 0 || B > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_kernel, dim3((H + 255) / 256, B), dim3(256), 0, s, ids, table, H, h);
  return hipGetLastError();
}

int exl3d_add_rmsnorm(float *h, const uint16_t *add, const uint16_t *w, uint16_t *out, int B,
                      int H, float eps, hipStream_t s) {
  if (B <= 0 || H <= 0 || H % 8 != 0 || H > RN_THREADS * RN_PER * 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(B), dim3(RN_THREADS), 0, s, h, add, w, out, H, eps);
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

size_t exl3d_attn_scratch_bytes(int B, int nq, int nkv, int Tmax) {
  int ts;
  const int ns = attn_split(Tmax, B, nkv, &ts);
  return (size_t)B * nkv * ns * AT_G * (EXL3D_HEAD_DIM + 2) * sizeof(float);
}

int exl3d_attn_decode(const uint16_t *q, const uint16_t *kcache, const uint16_t *vcache,
                      const int32_t *pos, int B, int nq, int nkv, int Tmax, float scale,
                      uint16_t *out, float *scratch, size_t scratch_bytes, hipStream_t s) {
  if (B <= 0 || nkv <= 0 || nq != AT_G * nkv || B > 65535 || nkv > 65535)
    return hipErrorInvalidValue;
  if (scratch_bytes < exl3d_attn_scratch_bytes(B, nq, nkv, Tmax)) return hipErrorInvalidValue;
  int ts;
  const int ns = attn_split(Tmax, B, nkv, &ts);
  hipLaunchKernelGGL(attn_decode_kernel, dim3(ns, nkv, B), dim3(256), 0, s, q, kcache, vcache,
                     pos, nq, nkv, Tmax, ts, scale, scratch);
  hipLaunchKernelGGL(attn_combine_kernel, dim3(nkv, B), dim3(AT_G * EXL3D_HEAD_DIM), 0, s, scratch,
                     nq, nkv, ns, out);
  return hipGetLastError();
}

int exl3d_silu_mul(const uint16_t *g, const uint16_t *u, uint16_t *out, size_t n, hipStream_t s) {
  if (n == 0) return hipErrorInvalidValue;
  const size_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256),
                     0, s, g, u, out, n);
  return hipGetLastError();
}

}  // extern "C"
