// exl3_kernels.hip -- HIP kernels for the EXL3 trellis-quantized linear on
// MI355X (gfx950, wave64) and their host launchers.
//
// Kernels (reference roles, paths relative to /root/reference/plugins/):
//  * prepare / finish: the Hadamard-128 rotations around the inner product
//    (sushi_ds41/src/sushi/exl3/expert_exl3_kernels.zig:902-970; contract
//    turboexl3_qwen38/overlay/mlx_serve/abi/quant.zig:52-55);
//  * decode_matrix: whole-matrix decode to f16 (the `q3_exl3_dig_decmat_*`
//    role, turboexl3_ds41/src/exl3/kernels/exl3/q3_exl3_dig_decmat_5120x2304_mul1hk3.metal);
//  * gemv: rows <= 8, weights decoded in registers, split-K over workgroups
//    with the finish fused into the last workgroup of each 128-column group
//    (the decode GEMV role: expert_exl3_kernels.zig:1653-1849,
//    turboexl3_ds41/src/exl3/kernels/exl3/dsv41_exl3_mul1h_k3_2304.metal);
//  * gemm: any rows, weight tiles decoded into LDS as f16 in MFMA operand
//    layout, v_mfma_f32_32x32x16_f16 with f32 accumulation, finish fused
//    (the prefill GEMM role: expert_exl3_kernels.zig:676-750,
//    dsv41_prefill_dig_gemm_5120x2304_gu_xmul1hk3_m128.metal).
//
// Compiled with -ffp-contract=off: every f32 multiply and add rounds on its
// own where the reference's order of operations is reproduced; fused
// multiply-adds are written out where they are meant.
// The rate-templated kernels live in exl3_kern.h; their launchers are
// instantiated once per rate in exl3_rate.hip.
#include <atomic>

#include "exl3_kern.h"

namespace exl3 {

// =================================================================== prepare

// One wave per 128-block of one row, four blocks per workgroup: element i
// of the block lives in lane i/2, register i%2 (had128_pair: the stage on
// index bit 0 in-register, bits 1..6 across lanes; each stage (lo + hi,
// lo - hi) in bit order, as the reference computes it).
// Row r takes suh row r % groups (groups 1: one suh for every row; a grouped
// linear's [rows, G, in] input: group g's suh for its rows).
__global__ __launch_bounds__(256) void prepare_kernel(const void *__restrict__ x, int xdt,
                                                      const uint16_t *__restrict__ suh,
                                                      uint16_t *__restrict__ xp, int in,
                                                      int nblk, int groups) {
  const int lane = threadIdx.x & 63;
  const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= nblk) return;  // whole waves
  const size_t base = (size_t)blockIdx.y * in;
  const int k = blk * 128 + 2 * lane;
  // f16(x) * suh in f32 (expert_exl3.zig:490-493; the kernel's
  // float(x) * float(suh), expert_exl3_kernels.zig:908-912).
  const uint32_t su =
      *reinterpret_cast<const uint32_t *>(suh + (size_t)(blockIdx.y % (unsigned)groups) * in + k);
  float v0 = h2f(f2h(load_act(x, base + k, xdt))) * h2f((uint16_t)(su & 0xFFFFu));
  float v1 = h2f(f2h(load_act(x, base + k + 1, xdt))) * h2f((uint16_t)(su >> 16));
  had128_pair(v0, v1, lane);
  *reinterpret_cast<uint32_t *>(xp + base + k) =
      (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
}

// The same rotation on an f16 [rows, 128-block] of inner products, then
// * svh, rounded to f16, stored in the output dtype
// (expert_exl3_kernels.zig:938-970; expert_exl3.zig:534-544).
__device__ __forceinline__ void finish_row_wave(const uint16_t *z, const uint16_t *svh, void *y,
                                                int ydt, size_t yoff, int lane) {
  float v0 = h2f(z[lane]);
  float v1 = h2f(z[lane + 64]);
#pragma unroll
  for (int bit = 1; bit <= 32; bit <<= 1) {
    const float p0 = xor_lanes(v0, bit), p1 = xor_lanes(v1, bit);
    const float sg = (lane & bit) == 0 ? 1.0f : -1.0f;
    v0 = butterfly(sg, v0, p0);
    v1 = butterfly(sg, v1, p1);
  }
  const float a = v0 + v1, b = v0 - v1;
  const float s0 = a * HAD_SCALE, s1 = b * HAD_SCALE;
  store_out(y, yoff + lane, f2h(s0 * h2f(svh[lane])), ydt);
  store_out(y, yoff + lane + 64, f2h(s1 * h2f(svh[lane + 64])), ydt);
}

__global__ __launch_bounds__(64) void finish_kernel(const uint16_t *__restrict__ z,
                                                    const uint16_t *__restrict__ svh,
                                                    void *__restrict__ y, int ydt, int out) {
  const size_t off = (size_t)blockIdx.y * out + blockIdx.x * 128;
  finish_row_wave(z + off, svh + blockIdx.x * 128, y, ydt, off, threadIdx.x);
}

// prepare_kernel's rotation with 8 elements per lane and 16-byte accesses:
// a 128-block is 16 lanes, element 8 j + i in lane j's register i.  The
// butterflies on element bits 0-2 run in registers, bits 3-6 across the 16
// lanes, in had128_pair's stage order and with its sums (lo + hi, lo - hi),
// so the results are identical.  Block gb of the flattened [rows][in / 128]
// starts at element 128 gb.  x, suh and xp must be 16-byte aligned.
__global__ __launch_bounds__(256) void prepare8_kernel(const void *__restrict__ x, int xdt,
                                                       const uint16_t *__restrict__ suh,
                                                       uint16_t *__restrict__ xp, int nblk,
                                                       uint32_t nblocks, int groups) {
  const int j = threadIdx.x & 15;
  const uint32_t gb0 = blockIdx.x * 16u + (threadIdx.x >> 4);
  const bool valid = gb0 < nblocks;  // a 16-lane group is valid or not as a whole
  const uint32_t gb = valid ? gb0 : nblocks - 1;
  const size_t off = (size_t)gb * 128 + 8 * j;
  const int k = (int)(gb % (uint32_t)nblk) * 128 + 8 * j;
  const size_t ks = (size_t)((gb / (uint32_t)nblk) % (uint32_t)groups) * nblk * 128 + k;
  float v[8];
  if (xdt == OUT_F32) {
    const float4 a = *reinterpret_cast<const float4 *>((const float *)x + off);
    const float4 b = *reinterpret_cast<const float4 *>((const float *)x + off + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4 *>((const uint16_t *)x + off);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = (uint16_t)(ws[i] & 0xFFFFu), hi = (uint16_t)(ws[i] >> 16);
      v[2 * i] = xdt == OUT_F16 ? h2f(lo) : bf2f(lo);
      v[2 * i + 1] = xdt == OUT_F16 ? h2f(hi) : bf2f(hi);
    }
  }
  const uint4 su = *reinterpret_cast<const uint4 *>(suh + ks);
  const uint32_t ss[4] = {su.x, su.y, su.z, su.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = h2f(f2h(v[2 * i])) * h2f((uint16_t)(ss[i] & 0xFFFFu));
    v[2 * i + 1] = h2f(f2h(v[2 * i + 1])) * h2f((uint16_t)(ss[i] >> 16));
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
  if (valid) {
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = (uint32_t)f2h(v[2 * i] * HAD_SCALE) | ((uint32_t)f2h(v[2 * i + 1] * HAD_SCALE) << 16);
    *reinterpret_cast<uint4 *>(xp + off) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

hipError_t launch_prepare(const void *x, int xdt, const uint16_t *suh, uint16_t *xp, int rows,
                          int in, hipStream_t s, int groups) {
  if (rows <= 0 || in <= 0 || in % 128 != 0 || groups <= 0) return hipErrorInvalidValue;
  if (rows > 65535) return hipErrorInvalidValue;
  const int nblk = in / 128;
  const size_t nblocks = (size_t)rows * nblk;
  const bool aligned = (((uintptr_t)x | (uintptr_t)suh | (uintptr_t)xp) & 15) == 0;
  if (aligned && nblocks * 16 < ((size_t)1 << 31)) {
    hipLaunchKernelGGL(prepare8_kernel, dim3((unsigned)((nblocks + 15) / 16)), dim3(256), 0, s, x,
                       xdt, suh, xp, nblk, (uint32_t)nblocks, groups);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(prepare_kernel, dim3((nblk + 3) / 4, rows), dim3(256), 0, s, x, xdt, suh, xp,
                     in, nblk, groups);
  return hipGetLastError();
}

hipError_t launch_finish(const uint16_t *z, const uint16_t *svh, void *y, int ydt, int rows,
                         int out, hipStream_t s) {
  if (rows <= 0 || out <= 0 || out % 128 != 0 || rows > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(finish_kernel, dim3(out / 128, rows), dim3(64), 0, s, z, svh, y, ydt, out);
  return hipGetLastError();
}

// ============================================================ decode matrix

// One wave per (k-tile row tk, 8 consecutive output tiles): lane = 8*tile +
// chunk.  Decoded values are staged in LDS as the 16 x 128 row block and
// written out as contiguous rows of W_inner [in, out].
template <int K, int CB>
__global__ __launch_bounds__(64) void decode_matrix_kernel(const uint32_t *__restrict__ tw,
                                                           uint16_t *__restrict__ w, int out_tiles,
                                                           CbRow d) {
  __shared__ uint32_t blk[16 * 64];  // 16 rows x 128 f16, as dwords
  const int lane = threadIdx.x;
  const int tk = blockIdx.y, cg = blockIdx.x;
  const int tl = lane >> 3, c = lane & 7;
  const size_t tile = (size_t)tk * out_tiles + cg * 8 + tl;
  const uint32_t *tp = tw + tile * (8 * K);
  uint32_t wd[K + 1];
#pragma unroll
  for (int i = 0; i < K; ++i) wd[i + 1] = tp[c * K + i];
  wd[0] = tp[((c + 7) & 7) * K + (K - 1)];
  uint16_t *row16 = reinterpret_cast<uint16_t *>(blk);
  static_for<16>([&](auto P) {
    constexpr int p = decltype(P)::value;
    const uint32_t v = chunk_pair<K, CB, p>(wd, d);
    constexpr int r = chunk_row(2 * p);
    const int col = tl * 16 + c + 8 * chunk_colhalf(2 * p);
    row16[r * 128 + col] = (uint16_t)(v & 0xFFFFu);
    row16[(r + 1) * 128 + col] = (uint16_t)(v >> 16);
  });
  __syncthreads();
  const size_t out = (size_t)out_tiles * 16;
  // 16 rows x 64 dwords: lane writes dword `lane` of every row.
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    uint32_t *dst = reinterpret_cast<uint32_t *>(w + ((size_t)tk * 16 + r) * out + cg * 128);
    dst[lane] = blk[r * 64 + lane];
  }
}

// Any even n: the 8 tiles' dwords are staged in LDS and each lane extracts its
// 32 codewords with run-time windows.
template <int CB>
__global__ __launch_bounds__(64) void decode_matrix_generic_kernel(const uint32_t *__restrict__ tw,
                                                                   uint16_t *__restrict__ w,
                                                                   int out_tiles, int n,
                                                                   CbRow d) {
  __shared__ uint32_t words[8 * 64];
  __shared__ uint32_t blk[16 * 64];
  const int lane = threadIdx.x;
  const int tk = blockIdx.y, cg = blockIdx.x;
  const int nw = n >> 1;
  const uint32_t *src = tw + ((size_t)tk * out_tiles + cg * 8) * nw;
  for (int i = lane; i < 8 * nw; i += 64) words[i] = src[i];
  __syncthreads();
  const int tl = lane >> 3, c = lane & 7;
  const uint32_t *mine = words + tl * nw;
  uint16_t *row16 = reinterpret_cast<uint16_t *>(blk);
  for (int p = 0; p < 16; ++p) {
    const uint32_t t = 32u * c + 2u * p;
    const uint32_t v = decode_pair<CB>(tile_window(mine, n, t), tile_window(mine, n, t + 1u), d);
    const int r = chunk_row(2 * p);
    const int col = tl * 16 + c + 8 * chunk_colhalf(2 * p);
    row16[r * 128 + col] = (uint16_t)(v & 0xFFFFu);
    row16[(r + 1) * 128 + col] = (uint16_t)(v >> 16);
  }
  __syncthreads();
  const size_t out = (size_t)out_tiles * 16;
  for (int r = 0; r < 16; ++r) {
    uint32_t *dst = reinterpret_cast<uint32_t *>(w + ((size_t)tk * 16 + r) * out + cg * 128);
    dst[lane] = blk[r * 64 + lane];
  }
}

template <int CB>
static hipError_t decode_matrix_cb(const uint32_t *tw, const Format &f, int in, int out,
                                   uint16_t *w, hipStream_t s) {
  const dim3 grid(out / 128, in / 16);
  const int ot = out / 16;
  const CbRow m = f.dec();
  switch (f.integer_rate() ? f.n / 16 : 0) {
#define EXL3_DM(KK)                                                                             \
  case KK:                                                                                      \
    hipLaunchKernelGGL((decode_matrix_kernel<KK, CB>), grid, dim3(64), 0, s, tw, w, ot, m); \
    break;
    EXL3_DM(1) EXL3_DM(2) EXL3_DM(3) EXL3_DM(4) EXL3_DM(5) EXL3_DM(6) EXL3_DM(7) EXL3_DM(8)
#undef EXL3_DM
    default:
      hipLaunchKernelGGL((decode_matrix_generic_kernel<CB>), grid, dim3(64), 0, s, tw, w, ot, f.n,
                         m);
  }
  return hipGetLastError();
}

hipError_t launch_decode_matrix(const uint16_t *trellis, const Format &f, int in, int out,
                                uint16_t *w, hipStream_t s) {
  if (in <= 0 || out <= 0 || in % 16 != 0 || out % 128 != 0) return hipErrorInvalidValue;
  if (f.n < 16 || f.n > 128 || (f.n & 1)) return hipErrorInvalidValue;
  if (in / 16 > 65535) return hipErrorInvalidValue;
  const uint32_t *tw = reinterpret_cast<const uint32_t *>(trellis);
  switch (f.codebook) {
    case CB_MCG: return decode_matrix_cb<CB_MCG>(tw, f, in, out, w, s);
    case CB_HASH: return decode_matrix_cb<CB_HASH>(tw, f, in, out, w, s);
    case CB_PAIR1: return decode_matrix_cb<CB_PAIR1>(tw, f, in, out, w, s);
    default: return decode_matrix_cb<CB_MUL1>(tw, f, in, out, w, s);
  }
}

// Every state of a codebook, the table the load-time self-check hashes:
// w[s] = the weight codeword s decodes to (mul1, mcg, the hash-mask tables;
// 65536 f16), through the same device decode the GEMV and GEMM use (pairs of
// codewords, the window's mask applied first).  pair1 decodes a pair of
// weights from one codeword: w[2c], w[2c + 1] for codeword c (131072 f16).
template <int CB>
__global__ __launch_bounds__(256) void decode_states_kernel(uint16_t *__restrict__ w, CbRow d) {
  const uint32_t p = blockIdx.x * 256u + threadIdx.x;  // pair index
  uint32_t v;
  if constexpr (CB == CB_PAIR1)
    v = decode_pair<CB>(0u, p, d);
  else
    v = decode_pair<CB>(2u * p, 2u * p + 1u, d);
  reinterpret_cast<uint32_t *>(w)[p] = v;
}

hipError_t launch_decode_states(const Format &f, uint16_t *w, hipStream_t s) {
  const CbRow d = f.dec();
  switch (f.codebook) {
    case CB_MCG: hipLaunchKernelGGL(decode_states_kernel<CB_MCG>, dim3(128), dim3(256), 0, s, w, d); break;
    case CB_HASH: hipLaunchKernelGGL(decode_states_kernel<CB_HASH>, dim3(128), dim3(256), 0, s, w, d); break;
    case CB_PAIR1: hipLaunchKernelGGL(decode_states_kernel<CB_PAIR1>, dim3(256), dim3(256), 0, s, w, d); break;
    default: hipLaunchKernelGGL(decode_states_kernel<CB_MUL1>, dim3(128), dim3(256), 0, s, w, d);
  }
  return hipGetLastError();
}

// ------------------------------------------------------------ un-rotation

// W_public = diag(suh) H W_inner H diag(svh) / 128 per 128 x 128 block, in
// the reference's order (sushi_ds41/src/sushi/exl3/expert_exl3.zig:440-488,
// `reconstructPublic`): the dense Hadamard over the input index of every
// column (out[r] = sum_k e(r,k) * v[k], e = +-HAD_SCALE by the parity of
// r & k, products and sums in f32 in k order), times suh per row, the dense
// Hadamard over the output index of every row, times svh per column, then
// one rounding to the output type (f16: the reference's value bit for bit).
// e * v is +-(HAD_SCALE * v) exactly and acc + (-p) is acc - p, so each term
// is the scaled value added or subtracted.  A thread keeps 8 sums: rows (or
// columns) o0 + i, i < 8, o0 a multiple of 8, whose sign for k = k8 + j is
// parity(o0 & k8) ^ parity(i & j) -- the second term fixed at compile time.
constexpr int UNROT_THREADS = 256;
constexpr int UNROT_LD = 129;  // padded LDS row (floats)

__device__ __forceinline__ void unrot_eight(const float *hv, int stride, int o0, float (&acc)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int k8 = 0; k8 < 128; k8 += 8) {
    const uint32_t flip = (uint32_t)(__builtin_popcount((unsigned)(o0 & k8)) & 1) << 31;
    static_for<8>([&](auto J) {
      constexpr int j = decltype(J)::value;
      const float p = bits<float>(bits<uint32_t>(hv[(k8 + j) * stride]) ^ flip);
      static_for<8>([&](auto I) {
        constexpr int i = decltype(I)::value;
        if constexpr (__builtin_popcount(i & j) & 1)
          acc[i] = acc[i] - p;
        else
          acc[i] = acc[i] + p;
      });
    });
  }
}

__global__ __launch_bounds__(UNROT_THREADS) void unrotate_kernel(
    const uint16_t *__restrict__ w, const uint16_t *__restrict__ suh,
    const uint16_t *__restrict__ svh, void *__restrict__ dst, int out, int64_t ld, int ydt) {
  __shared__ __attribute__((aligned(16))) float lds[2 * 128 * UNROT_LD];  // 129 KiB
  float *A = lds;                    // HAD_SCALE * W_inner block [k][c]
  float *B = lds + 128 * UNROT_LD;   // HAD_SCALE * (column Hadamard * suh) [r][k]
  const int tid = threadIdx.x;
  const int rb = blockIdx.y * 128, cb = blockIdx.x * 128;
  for (int e = tid; e < 128 * 128; e += UNROT_THREADS) {
    const int r = e >> 7, c = e & 127;
    A[r * UNROT_LD + c] = f32_value(HAD_SCALE * h2f(w[(size_t)(rb + r) * out + cb + c]));
  }
  __syncthreads();
  {
    // input-index Hadamard: column c, rows o0 .. o0 + 7 at a time
    const int c = tid & 127;
    for (int o0 = (tid >> 7) * 8; o0 < 128; o0 += 16) {
      float acc[8];
      unrot_eight(A + c, UNROT_LD, o0, acc);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = f32_value(acc[i] * h2f(suh[rb + o0 + i]));
        B[(o0 + i) * UNROT_LD + c] = f32_value(HAD_SCALE * v);
      }
    }
  }
  __syncthreads();
  {
    // output-index Hadamard: row r, columns o0 .. o0 + 7 at a time
    const int r = tid & 127;
    for (int o0 = (tid >> 7) * 8; o0 < 128; o0 += 16) {
      float acc[8];
      unrot_eight(B + r * UNROT_LD, 1, o0, acc);
      const size_t base = (size_t)(rb + r) * ld + cb + o0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = f32_value(acc[i] * h2f(svh[cb + o0 + i]));
        if (ydt == OUT_F16)
          ((uint16_t *)dst)[base + i] = f2h(v);
        else if (ydt == OUT_BF16)
          ((uint16_t *)dst)[base + i] = f2bf(v);
        else
          ((float *)dst)[base + i] = v;
      }
    }
  }
}

hipError_t launch_unrotate(const uint16_t *w_inner, const uint16_t *suh, const uint16_t *svh,
                           int in, int out, void *dst, int64_t ld, int ydt, hipStream_t s) {
  if (in <= 0 || out <= 0 || in % 128 != 0 || out % 128 != 0 || ld < out) return hipErrorInvalidValue;
  if (in / 128 > 65535 || ydt < OUT_F16 || ydt > OUT_F32) return hipErrorInvalidValue;
  hipLaunchKernelGGL(unrotate_kernel, dim3(out / 128, in / 128), dim3(UNROT_THREADS), 0, s, w_inner,
                     suh, svh, dst, out, ld, ydt);
  return hipGetLastError();
}

static std::atomic<int> g_poll_bound{-1};
int splitk_poll_max() {
  const int v = g_poll_bound.load(std::memory_order_relaxed);
  return v >= 0 ? v : PARTIAL_POLL_MAX;
}
void set_splitk_poll_max(int polls) { g_poll_bound.store(polls, std::memory_order_relaxed); }
static std::atomic<int> g_splitk_drop{0};
int splitk_drop() { return g_splitk_drop.load(std::memory_order_relaxed); }
void set_splitk_drop(int on) { g_splitk_drop.store(on != 0, std::memory_order_relaxed); }

// k-splits of a GEMV: whole input Hadamard blocks per split, at most
// GEMV_KSPLIT_MAX splits and tps_max k-tile rows (GEMV_TPS_MAX; the generic
// rate's launchers clamp to 32 afterwards), GEMV_TPS_ONE_ROW_MAX at one or
// two rows.
// * Up to 4 rows, over at most 1024 workgroups: the split count that
//   balances the launch over the 256 CUs, the least (workgroups on the
//   busiest CU) x (blocks a workgroup), ties to fewer splits (fewer partial
//   sums and hand-offs).  Qwen3-8B at one row: q+k+v 16 splits of 2 blocks
//   (768 workgroups, against 11 of 3: 528, 16 CUs holding a third), o 8 of 4
//   (256), down 8 of 12 (256), gate+up 4 of 8 (768); the pass 1.7 % faster
//   than with ~512 workgroups a launch.
// * Else ~512 workgroups over `groups` column groups; above 4 rows at most
//   256 (one round: q+k+v 5 splits, 240 workgroups, against 6 and 288, 0.3 %
//   faster a decode step at 16 rows), whose split-K partial sums (rows x 128
//   floats per workgroup) would otherwise add half the weight bytes again.
void gemv_plan(int in, int out, int groups, int rows, int *ksplit, int *tps, int tps_max) {
  const int nb = in / 128;
  const int cgs = std::max(1, out / 128) * std::max(1, groups);
  if (rows <= 4) {
    const int cap = (rows <= 2 ? std::max(tps_max, GEMV_TPS_ONE_ROW_MAX) : tps_max) / 8;
    long best = -1;
    int bks = 0;
    for (int ks = 1; ks <= std::min(nb, GEMV_KSPLIT_MAX) && (long)cgs * ks <= 1024; ++ks) {
      const int bps = (nb + ks - 1) / ks;
      if (bps > cap || (nb + bps - 1) / bps != ks) continue;  // not the fewest splits of bps
      const long cost = (long)(((long)cgs * ks + 255) / 256) * bps;
      if (best < 0 || cost < best) {
        best = cost;
        bks = ks;
      }
    }
    if (bks > 0) {
      const int bps = (nb + bks - 1) / bks;
      *tps = 8 * bps;
      *ksplit = bks;
      return;
    }
  }
  const int target = rows > 4 ? 256 : 512;
  int ks = std::min(nb, std::max(1, rows > 4 ? target / cgs : (target + cgs - 1) / cgs));
  int bps = std::min(tps_max / 8, (nb + ks - 1) / ks);  // blocks per split
  bps = std::max(bps, (nb + GEMV_KSPLIT_MAX - 1) / GEMV_KSPLIT_MAX);
  *tps = 8 * bps;
  *ksplit = (nb + bps - 1) / bps;
}

int gemv_ksplit(int in, int out, int groups, int rows) {
  int ks, tps;
  gemv_plan(in, out, groups, rows, &ks, &tps, GEMV_TPS_MAX);
  return ks;
}

void gemv_multi_plan(int in, int total_out, bool generic, int rows, int *ksplit, int *tps) {
  gemv_plan(in, total_out, 1, rows, ksplit, tps, GEMV_TPS_MAX);
  if (generic && *tps > 32) {
    *tps = 32;
    *ksplit = (in / 16 + 31) / 32;
  }
}

// Calls launch(integral_constant<int, K>) for K = kk in 1..8, K = 0 otherwise.
template <typename F>
static void rate_dispatch(int kk, F &&launch) {
  switch (kk) {
    case 1: launch(std::integral_constant<int, 1>{}); break;
    case 2: launch(std::integral_constant<int, 2>{}); break;
    case 3: launch(std::integral_constant<int, 3>{}); break;
    case 4: launch(std::integral_constant<int, 4>{}); break;
    case 5: launch(std::integral_constant<int, 5>{}); break;
    case 6: launch(std::integral_constant<int, 6>{}); break;
    case 7: launch(std::integral_constant<int, 7>{}); break;
    case 8: launch(std::integral_constant<int, 8>{}); break;
    default: launch(std::integral_constant<int, 0>{});
  }
}

static hipError_t gemv_multi(const GemvLinear *ls, int count, const Format &f, const void *x,
                             int xdt, bool prepared, int ydt, int rows, int in, Scratch *sc,
                             const GemvFuse &fz, hipStream_t s) {
  if (count < 1 || count > GEMV_MAXW || rows < 1 || rows > GEMV_ROWS_MAX) return hipErrorInvalidValue;
  if (in <= 0 || in % 128 != 0) return hipErrorInvalidValue;
  if (f.n < 16 || f.n > 128 || (f.n & 1)) return hipErrorInvalidValue;
  const bool generic = !f.integer_rate();
  int maxout = 0, totcg = 0;
  for (int i = 0; i < count; ++i) {
    if (ls[i].out <= 0 || ls[i].out % 128 != 0) return hipErrorInvalidValue;
    if (ls[i].y == nullptr && ls[i].zout == nullptr && fz.res == nullptr) return hipErrorInvalidValue;
    maxout = std::max(maxout, ls[i].out);
    totcg += ls[i].out / 128;
  }
  if ((int64_t)rows * std::max(in, maxout) >= (int64_t)1 << 31) return hipErrorInvalidValue;
  int ksplit, tps;
  gemv_multi_plan(in, 128 * totcg, generic, rows, &ksplit, &tps);
  if (ksplit > GEMV_KSPLIT_MAX || totcg > 65535) return hipErrorInvalidValue;
  if (in / 16 > 65535) return hipErrorInvalidValue;
  GemvArgs a{};
  const uint32_t *tw[GEMV_MAXW] = {nullptr, nullptr, nullptr, nullptr};
  int cgs[GEMV_MAXW] = {0, 0, 0, 0};
  int cg0 = 0;
  for (int i = 0; i < count; ++i) {
    GemvWeight &w = a.w[i];
    tw[i] = reinterpret_cast<const uint32_t *>(ls[i].trellis);
    w.suh = ls[i].suh;
    w.svh = ls[i].svh;
    w.y = ls[i].y;
    w.zout = ls[i].zout;
    w.expert_words = 0;
    cgs[i] = cg0;
    cg0 += ls[i].out / 128;
    if (ksplit > 1) {
      if (sc[i].partial == nullptr || sc[i].partial_floats < (size_t)ksplit * rows * ls[i].out)
        return hipErrorInvalidValue;
    }
    w.partial = sc[i].partial;
  }
  if (ksplit > 1 && sc[0].status == nullptr) return hipErrorInvalidValue;
  // the unused trellis arguments carry suh pointers, which gemv_kernel's
  // workgroups read without waiting for the argument segment
  if (count == 1) {
    tw[1] = reinterpret_cast<const uint32_t *>(ls[0].suh);
  } else if (count == 2) {
    tw[2] = reinterpret_cast<const uint32_t *>(ls[0].suh);
    tw[3] = reinterpret_cast<const uint32_t *>(ls[1].suh);
  } else if (count == 3) {
    tw[3] = reinterpret_cast<const uint32_t *>(ls[0].suh);
  }
  a.c.status = sc[0].status;
  a.c.poll_max = splitk_poll_max();
  a.c.drop_partials = splitk_drop();
  a.c.ydt = ydt;
  a.c.ptotal = (size_t)rows;
  a.c.ksplit = ksplit;
  a.c.dec = f.dec();
  a.c.nw = f.n / 2;
  a.c.x2 = fz.up;
  a.c.limit = fz.limit;
  a.c.nssq = fz.nssq;
  a.c.nw_norm = fz.norm_w;
  a.c.eps = fz.eps;
  a.c.res = fz.res;
  a.c.res_ssq = fz.res_ssq;
  a.c.attn_part = fz.attn_part;
  a.c.attn_nkv = fz.attn_nkv;
  a.c.attn_g = fz.attn_g;
  a.c.attn_nsplit = fz.attn_nsplit;
  GemvGeo geo{};
  geo.cg1 = cgs[1];
  geo.cg2 = cgs[2];
  geo.cg3 = cgs[3];
  geo.cgend = totcg;
  geo.rows = rows;
  geo.xdt = xdt;
  geo.prepared = prepared || fz.stacked ? 1 : 0;
  geo.stacked = fz.stacked ? 1 : 0;
  geo.in_tiles = in / 16;
  geo.tps = tps;
  uint32_t g0, g1, g2;
  if (!gemv_geo_pack(geo, &g0, &g1, &g2)) return hipErrorInvalidValue;
  const size_t lds = gemv_lds_bytes(rows, tps, generic);
  const dim3 grid(totcg, ksplit);
  const int prep = gemv_prep_form(rows, tps);
  const bool oneb = prep == 0;
  if (fz.nssq != nullptr &&
      (!oneb || xdt != OUT_F32 || prepared || fz.norm_w == nullptr || in / 128 > NORM_MAXBLK))
    return hipErrorInvalidValue;
  if (fz.res != nullptr && (count != 1 || fz.res_ssq == nullptr)) return hipErrorInvalidValue;
  if (fz.stacked && (xdt != OUT_F16 || fz.nssq != nullptr || fz.up != nullptr ||
                     fz.attn_part != nullptr))
    return hipErrorInvalidValue;
  if (fz.attn_part != nullptr &&
      (!oneb || count != 1 || xdt != OUT_F16 || prepared || fz.nssq != nullptr ||
       fz.up != nullptr || fz.attn_nkv < 1 || fz.attn_g < 1 || fz.attn_nsplit < 1 ||
       in != fz.attn_nkv * fz.attn_g * 128))
    return hipErrorInvalidValue;
  rate_dispatch(generic ? 0 : f.n / 16, [&](auto KC) {
    gemv_go<decltype(KC)::value>(f, prep, grid, lds, s, tw, x, g0, g1, g2, a);
  });
  return hipGetLastError();
}

hipError_t launch_gemv_multi(const GemvLinear *ls, int count, const Format &f, const void *x,
                             int xdt, bool prepared, int ydt, int rows, int in, Scratch *sc,
                             hipStream_t s) {
  return gemv_multi(ls, count, f, x, xdt, prepared, ydt, rows, in, sc, GemvFuse{}, s);
}

hipError_t launch_gemv_fused(const GemvLinear *ls, int count, const Format &f, const void *x,
                             int xdt, int ydt, int rows, int in, Scratch *sc, const GemvFuse &fz,
                             hipStream_t s) {
  if (fz.up != nullptr && (xdt != OUT_F16 || fz.nssq != nullptr)) return hipErrorInvalidValue;
  return gemv_multi(ls, count, f, x, xdt, false, ydt, rows, in, sc, fz, s);
}

namespace {
// h = f16(silu(g) * u) elementwise (the prologue's arithmetic, swiglu1).
// h = f16(silu(g) * u) and its prepare with suh (the consumer's), in one
// pass: a 16-lane group per 128-block of the flattened [rows][in] (in a
// multiple of 128), 8 elements a lane; the prepared rows equal what the
// GEMV prologue forms from h (prep_block8).  Groups past the last block
// redo the last one (whole waves), storing nothing.
__global__ __launch_bounds__(256) void swiglu_prepare_kernel(const uint16_t *__restrict__ g,
                                                             const uint16_t *__restrict__ u,
                                                             const uint16_t *__restrict__ suh,
                                                             uint16_t *__restrict__ xp, int nblk,
                                                             uint32_t nblocks, float limit) {
  const int j = threadIdx.x & 15;
  const uint32_t gb0 = blockIdx.x * 16u + (threadIdx.x >> 4);
  const bool valid = gb0 < nblocks;
  const uint32_t gb = valid ? gb0 : nblocks - 1;
  const size_t off = (size_t)gb * 128 + 8 * j;
  const int k = (int)(gb % (uint32_t)nblk) * 128 + 8 * j;
  const uint4 gv = *reinterpret_cast<const uint4 *>(g + off);
  const uint4 uv = *reinterpret_cast<const uint4 *>(u + off);
  const uint4 su = *reinterpret_cast<const uint4 *>(suh + k);
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    h[i] = (uint32_t)f2h(swiglu1((uint16_t)(gw[i] & 0xFFFFu), (uint16_t)(uw[i] & 0xFFFFu), limit)) |
           ((uint32_t)f2h(swiglu1((uint16_t)(gw[i] >> 16), (uint16_t)(uw[i] >> 16), limit)) << 16);
  const uint4 o = prep_block8(h, su, j);
  if (valid) *reinterpret_cast<uint4 *>(xp + off) = o;
}

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t *__restrict__ g,
                                                     const uint16_t *__restrict__ u,
                                                     uint16_t *__restrict__ h, size_t n,
                                                     float limit) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    h[i] = f2h(swiglu1(g[i], u[i], limit));
}
}  // namespace

hipError_t launch_gemv_swiglu(const GemvLinear &l, const Format &f, const uint16_t *g,
                              const uint16_t *u, uint16_t *h, float limit, int ydt, int rows,
                              int in, Scratch &sc, hipStream_t s) {
  if (g == nullptr || u == nullptr || !(limit >= 0.0f)) return hipErrorInvalidValue;
  if (rows <= SWIGLU_PROLOGUE_ROWS) {
    GemvFuse fz{};
    fz.up = u;
    fz.limit = limit;
    return gemv_multi(&l, 1, f, g, OUT_F16, false, ydt, rows, in, &sc, fz, s);
  }
  // more rows: every column group would redo the rows' SwiGLU and prepare,
  // so both run once here, into prepared rows
  if (h == nullptr) return hipErrorInvalidValue;
  hipError_t e = launch_swiglu_prepare(g, u, l.suh, h, rows, in, limit, s);
  if (e != hipSuccess) return e;
  GemvFuse fz{};
  fz.stacked = true;
  return gemv_multi(&l, 1, f, h, OUT_F16, false, ydt, rows, in, &sc, fz, s);
}

hipError_t launch_swiglu(const uint16_t *g, const uint16_t *u, uint16_t *h, size_t n, float limit,
                         hipStream_t s) {
  if (n == 0 || !(limit >= 0.0f)) return hipErrorInvalidValue;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g, u, h, n, limit);
  return hipGetLastError();
}

hipError_t launch_swiglu_prepare(const uint16_t *g, const uint16_t *u, const uint16_t *suh,
                                 uint16_t *xp, int rows, int in, float limit, hipStream_t s) {
  if (rows <= 0 || in <= 0 || in % 128 != 0 || !(limit >= 0.0f) || suh == nullptr)
    return hipErrorInvalidValue;
  const int nblk = in / 128;
  const uint32_t nblocks = (uint32_t)rows * (uint32_t)nblk;
  hipLaunchKernelGGL(swiglu_prepare_kernel, dim3((nblocks + 15) / 16), dim3(256), 0, s, g, u, suh,
                     xp, nblk, nblocks, limit);
  return hipGetLastError();
}

bool gemv_one_batch(int in, int total_out, bool generic, int rows) {
  int ks, tps;
  gemv_multi_plan(in, total_out, generic, rows, &ks, &tps);
  return rows * (tps / 8) <= PREP_ITEMS;
}

hipError_t launch_gemv(const uint16_t *trellis, const Format &f, const void *x, int xdt,
                       bool prepared, const uint16_t *suh, const uint16_t *svh, void *y, int ydt,
                       uint16_t *zout, int rows, int in, int out, Scratch &sc, hipStream_t s) {
  GemvLinear l{trellis, suh, svh, y, zout, out};
  return launch_gemv_multi(&l, 1, f, x, xdt, prepared, ydt, rows, in, &sc, s);
}


namespace {
// The end of a split-K GEMM: z = f16(sum of the S planes of kpart, in split
// order), then the finish (Hadamard-128 in the reference's stage order,
// * 1/sqrt(128) * svh, as the GEMV's) or z itself.  One wave per row, lane l
// columns 2 l, 2 l + 1 of the block's 128.
__global__ __launch_bounds__(512) void gemm_splitk_finish_kernel(
    const float *__restrict__ part, int S, int M, int out, const uint16_t *__restrict__ svh,
    void *__restrict__ y, int ydt, uint16_t *__restrict__ zout) {
  const int cg = blockIdx.x, lane = threadIdx.x & 63;
  const int m = blockIdx.y * 8 + (threadIdx.x >> 6);
  if (m >= M) return;
  const size_t plane = (size_t)M * out;
  const float *p = part + (size_t)m * out + cg * 128 + 2 * lane;
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll 8
  for (int k = 0; k < S; ++k) {
    const float2 v = *reinterpret_cast<const float2 *>(p + (size_t)k * plane);
    s0 += v.x;
    s1 += v.y;
  }
  float v0 = h2f(f2h(s0)), v1 = h2f(f2h(s1));
  const size_t o = (size_t)m * out + cg * 128 + 2 * lane;
  if (y == nullptr) {
    zout[o] = f2h(v0);
    zout[o + 1] = f2h(v1);
    return;
  }
  had128_pair(v0, v1, lane);
  const float sv0 = h2f(svh[cg * 128 + 2 * lane]), sv1 = h2f(svh[cg * 128 + 2 * lane + 1]);
  store_out2(y, o, f2h(v0 * HAD_SCALE * sv0), f2h(v1 * HAD_SCALE * sv1), ydt);
}
}  // namespace

// Split-K of a GEMM whose tiles fill at most half the GPU: S splits (an
// even run of stages each), the most that keep tiles x S within one round
// of the 256 CUs (one workgroup a CU: its LDS); their f32 sums take S planes
// of rows x out floats.  A partial second round costs a whole split's time
// (gate+up at 128 rows: 96 tiles, 45.7 us a call in 2 splits against 57.3 in
// 3, 288 workgroups).  Above 128 tiles the planes' traffic costs more than
// the idle CUs (gate+up at 512 rows: 192 tiles, 547 TFLOP/s split in two
// against 629 whole).
GemmSplit gemm_split(int rows, int in, int out) {
  GemmSplit g;
  const int mblocks = (rows + GM_BM - 1) / GM_BM;
  const int tiles = ((out + GM_BN - 1) / GM_BN) * mblocks;
  const int pairs = in / 16 / 4 / 2;  // stage pairs
  int S = tiles > GM_SPLIT_TILES ? 1 : 256 / tiles;
  S = std::max(1, std::min(S, std::min(pairs, GM_SPLIT_MAX)));
  g.splits = S;
  g.tiles = tiles;
  g.part_floats = S > 1 ? (size_t)S * rows * out : 0;
  return g;
}

// The most rows one GEMM launch takes: the kernel addresses a launch's
// activations with 32-bit byte offsets, so a call past that runs as windows
// of whole row tiles, each its own launch (rows are independent: the same
// results).
static int64_t gemm_window_rows(int in) {
  return std::max<int64_t>(GM_BM, (int64_t)(0xFFFFFFFFull / ((uint64_t)in * 2)) / GM_BM * GM_BM);
}

size_t gemm_kpart_floats(int64_t rows, int in, int out) {
  const int64_t wmax = gemm_window_rows(in);
  const int64_t last = rows > wmax ? (rows - 1) % wmax + 1 : rows;
  size_t need = gemm_split((int)std::min(rows, wmax), in, out).part_floats;
  return std::max(need, gemm_split((int)last, in, out).part_floats);
}

hipError_t launch_gemm(const uint16_t *trellis, const Format &f, const uint16_t *xp,
                       const uint16_t *svh, void *y, int ydt, uint16_t *zout, int rows, int in,
                       int out, float *kpart, size_t kpart_floats, hipStream_t s) {
  if (rows < 1 || in <= 0 || out <= 0 || in % 128 != 0 || out % 128 != 0) return hipErrorInvalidValue;
  if (!f.gemm_rate()) return hipErrorInvalidValue;
  if (y == nullptr && zout == nullptr) return hipErrorInvalidValue;
  const int64_t wmax = gemm_window_rows(in);
  if (rows > wmax) {
    const size_t ysz = ydt == OUT_F32 ? 4 : 2;
    for (int64_t r0 = 0; r0 < rows; r0 += wmax) {
      const int r = (int)std::min<int64_t>(wmax, rows - r0);
      const hipError_t e = launch_gemm(
          trellis, f, xp + (size_t)r0 * in, svh, y ? (char *)y + (size_t)r0 * out * ysz : nullptr,
          ydt, zout ? zout + (size_t)r0 * out : nullptr, r, in, out, kpart, kpart_floats, s);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  const int mblocks = (rows + GM_BM - 1) / GM_BM;
  if (mblocks > 65535) return hipErrorInvalidValue;
  const GemmSplit sp = gemm_split(rows, in, out);
  if (sp.splits > 1 && (kpart == nullptr || kpart_floats < sp.part_floats))
    return hipErrorInvalidValue;
  if (sp.splits > 1 && (rows + 7) / 8 > 65535) return hipErrorInvalidValue;
  const dim3 grid((out + GM_BN - 1) / GM_BN, mblocks, sp.splits);
  const uint32_t *tw = reinterpret_cast<const uint32_t *>(trellis);
  const int it = in / 16, ot = out / 16;
  if (f.n == 24)
    gemm_frac_go<3>(f, grid, s, tw, xp, svh, y, ydt, zout, rows, it, ot, kpart);
  else if (f.n == 40)
    gemm_frac_go<5>(f, grid, s, tw, xp, svh, y, ydt, zout, rows, it, ot, kpart);
  else
    rate_dispatch(f.n / 16, [&](auto KC) {
      constexpr int K = decltype(KC)::value;
      if constexpr (K > 0) gemm_go<K>(f, grid, s, tw, xp, svh, y, ydt, zout, rows, it, ot, kpart);
    });
  if (sp.splits > 1)
    hipLaunchKernelGGL(gemm_splitk_finish_kernel, dim3(out / 128, (rows + 7) / 8), dim3(512), 0, s,
                       kpart, sp.splits, rows, out, svh, y, ydt, zout);
  return hipGetLastError();
}

// A grouped linear's prefill: the grouped GEMM over every group's row tiles
// in one launch, items formed from the grid (GemmGroup.groups), each
// group's trellis and svh at its index in the G-bank, the finish fused.
hipError_t launch_gemm_groups(const uint16_t *trellis, const Format &f, const uint16_t *xp,
                              const uint16_t *svh, void *y, int ydt, int rows, int groups,
                              int in, int out, hipStream_t s) {
  if (rows < 1 || groups < 1 || in <= 0 || out <= 0 || in % 128 != 0 || out % 128 != 0)
    return hipErrorInvalidValue;
  if (!f.integer_rate() || y == nullptr) return hipErrorInvalidValue;
  // activation offsets (bytes from xp) are 32-bit in the kernel
  if ((size_t)rows * groups * in * 2 > 0xFFFFFFFFu) return hipErrorInvalidValue;
  const size_t tiles_y = (size_t)groups * ((rows + GM_BM - 1) / GM_BM);
  if (tiles_y > 65535) return hipErrorInvalidValue;
  GemmGroup gg{nullptr, nullptr, nullptr, (size_t)(in / 16) * (out / 16) * (f.n / 2), groups, rows};
  const dim3 grid(out / GM_BN, (unsigned)tiles_y);
  const uint32_t *tw = reinterpret_cast<const uint32_t *>(trellis);
  rate_dispatch(f.n / 16, [&](auto KC) {
    constexpr int K = decltype(KC)::value;
    if constexpr (K > 0) gemm_grouped_go<K>(f, grid, s, tw, xp, svh, y, ydt, in / 16, out / 16, gg);
  });
  return hipGetLastError();
}

// ====================================================================== MoE
//
// Routed SwiGLU experts (sushi_ds41/src/sushi/exl3/expert_exl3_kernels.zig:
// 3151-3206 for the arithmetic; decode chain :2765-3113):
//   1. route: one workgroup counts the (row, k) slots per expert, orders the
//      slots by expert (within an expert in any order: every slot's
//      arithmetic is independent of its position) and emits work items of
//      up to 16 slots of one expert;
//   2. grouped GEMV, gate and up in one launch: each work item is the GEMV
//      workgroup above over its expert's packed weights for its slots, the
//      prepare (x[row] * suh[e]) fused, split-K with the fused finish,
//      giving g and u (f16) per slot;
//   3. mid: h = silu(g) * u in f32 (limit > 0: g <= limit, |u| <= limit,
//      turboexl3_ds41/src/exl3/kernels/exl3/q3_exl3_prep_gu_epi.metal:47-56),
//      then the down projection's prepare with suh_down[e];
//   4. grouped GEMV down on the prepared rows, finished per slot (f16);
//   5. combine: y[row] = sum_k score[row, k] * d[slot(row, k)] in f32, in k
//      order, then the output dtype.


constexpr int MOE_ROUTE_THREADS = 1024;

// Exclusive prefix sum over the 1024 threads of a block; *total gets the sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *tmp,
                                                         uint32_t *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t t = __shfl_up(inc, d, 64);
    if (lane >= d) inc += t;
  }
  if (lane == 63) tmp[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int w = 0; w < MOE_ROUTE_THREADS / 64; ++w) {
      const uint32_t t = tmp[w];
      tmp[w] = run;
      run += t;
    }
    *total = run;
  }
  __syncthreads();
  const uint32_t r = tmp[wave] + inc - v;
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(MOE_ROUTE_THREADS) void moe_route_kernel(
    const uint32_t *__restrict__ inds, int slots, int experts, uint32_t *__restrict__ sorted,
    MoeItem *__restrict__ items, uint32_t *__restrict__ n_items, uint32_t item_rows) {
  __shared__ uint32_t cnt[MOE_ROUTE_THREADS], cur[MOE_ROUTE_THREADS], tmp[MOE_ROUTE_THREADS / 64];
  __shared__ uint32_t total;
  const int t = threadIdx.x;
  cnt[t] = 0;
  __syncthreads();
  for (int s = t; s < slots; s += MOE_ROUTE_THREADS) {
    const uint32_t e = inds ? inds[s] : 0u;
    if (e < (uint32_t)experts) atomicAdd(&cnt[e], 1u);
  }
  __syncthreads();
  const uint32_t c = t < experts ? cnt[t] : 0u;
  const uint32_t off = block_exclusive_scan(c, tmp, &total);
  const uint32_t nit = (c + item_rows - 1) / item_rows;
  const uint32_t ioff = block_exclusive_scan(nit, tmp, &total);
  cur[t] = off;
  __syncthreads();
  for (int s = t; s < slots; s += MOE_ROUTE_THREADS) {
    const uint32_t e = inds ? inds[s] : 0u;
    if (e < (uint32_t)experts) sorted[atomicAdd(&cur[e], 1u)] = (uint32_t)s;
  }
  for (uint32_t r = 0; r < nit; ++r) {
    MoeItem it;
    it.expert = (uint32_t)t;
    it.start = off + r * item_rows;
    it.count = min(item_rows, c - r * item_rows);
    it.pad = 0;
    items[ioff + r] = it;
  }
  if (t == 0) *n_items = total;
}

// The grouped GEMM's gate and up inputs: slot s's row x[s / topk] prepared
// with expert e = inds[s]'s suh of each (as prepare_kernel: f16(x) * suh,
// Hadamard-128, * 1/sqrt(128), f16), one wave per 128-block.
__global__ __launch_bounds__(256) void moe_prep_kernel(const void *__restrict__ x, int xdt,
                                                       const uint32_t *__restrict__ inds,
                                                       int experts, int topk,
                                                       const uint16_t *__restrict__ suh_g,
                                                       const uint16_t *__restrict__ suh_u,
                                                       uint16_t *__restrict__ xg,
                                                       uint16_t *__restrict__ xu, int in,
                                                       int nblk) {
  const int lane = threadIdx.x & 63;
  const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= nblk) return;  // whole waves
  const size_t slot = blockIdx.y;
  const uint32_t e = inds[slot];
  if (e >= (uint32_t)experts) return;
  const int k = blk * 128 + 2 * lane;
  const size_t xrow = (slot / (size_t)topk) * in;
  const float x0 = h2f(f2h(load_act(x, xrow + k, xdt))), x1 = h2f(f2h(load_act(x, xrow + k + 1, xdt)));
  const uint16_t *const su[2] = {suh_g + (size_t)e * in, suh_u + (size_t)e * in};
  uint16_t *const dst[2] = {xg, xu};
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const uint32_t sv = *reinterpret_cast<const uint32_t *>(su[w] + k);
    float v0 = x0 * h2f((uint16_t)(sv & 0xFFFFu)), v1 = x1 * h2f((uint16_t)(sv >> 16));
    had128_pair(v0, v1, lane);
    *reinterpret_cast<uint32_t *>(dst[w] + slot * in + k) =
        (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
  }
}

// The mid step: h = silu(g) * u (clamped when limit > 0), then down's
// prepare with suh_d[e] (the shared expert's, sh_suh_d, for e == shared).
// A down GEMV launch of few workgroups forms the same values, bit for bit,
// in its SwiGLU prologue instead.
__global__ __launch_bounds__(64) void moe_mid_kernel(const uint16_t *__restrict__ g,
                                                     const uint16_t *__restrict__ u,
                                                     const uint32_t *__restrict__ inds, int experts,
                                                     const uint16_t *__restrict__ suh_d,
                                                     uint16_t *__restrict__ xd, int inter,
                                                     float limit, int shared,
                                                     const uint16_t *__restrict__ sh_suh_d) {
  const int lane = threadIdx.x;
  const size_t slot = blockIdx.y;
  const uint32_t e = inds ? inds[slot] : 0u;
  if (e >= (uint32_t)experts) return;
  const uint16_t *sud = (int)e == shared ? sh_suh_d : suh_d + (size_t)e * inter;
  const int i0 = blockIdx.x * 128 + lane;
  float v[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = i0 + 64 * j;
    float gv = h2f(g[slot * inter + i]), uv = h2f(u[slot * inter + i]);
    if (limit > 0.0f) swiglu_clamp(gv, uv, limit);
    const float h = f32_value(gv / (1.0f + expf(-gv))) * uv;
    v[j] = h2f(f2h(h)) * h2f(sud[i]);
  }
#pragma unroll
  for (int bit = 1; bit <= 32; bit <<= 1) {
    const float p0 = xor_lanes(v[0], bit), p1 = xor_lanes(v[1], bit);
    const float sg = (lane & bit) == 0 ? 1.0f : -1.0f;
    v[0] = butterfly(sg, v[0], p0);
    v[1] = butterfly(sg, v[1], p1);
  }
  const float a = v[0] + v[1], b = v[0] - v[1];
  xd[slot * inter + i0] = f2h(a * HAD_SCALE);
  xd[slot * inter + i0 + 64] = f2h(b * HAD_SCALE);
}

// y[row] = sum_k score * d[slot] (f32, k order), in the output dtype.
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t *__restrict__ d,
                                                          const uint32_t *__restrict__ inds,
                                                          const void *__restrict__ scores, int sdt,
                                                          int topk, int experts, int hidden,
                                                          void *__restrict__ y, int ydt) {
  const size_t row = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= hidden) return;
  float acc = 0.0f;
  for (int k = 0; k < topk; ++k) {
    const size_t slot = row * topk + k;
    const uint32_t e = inds ? inds[slot] : 0u;
    if (e >= (uint32_t)experts) continue;
    const float w = scores ? load_act(scores, slot, sdt) : 1.0f;
    acc = acc + f32_value(w * h2f(d[slot * hidden + i]));
  }
  if (ydt == OUT_F16)
    ((uint16_t *)y)[row * hidden + i] = f2h(acc);
  else if (ydt == OUT_BF16)
    ((uint16_t *)y)[row * hidden + i] = f2bf(acc);
  else
    ((float *)y)[row * hidden + i] = acc;
}

// The routes of a swiglu with a shared expert (launch_moe_shared_route): one
// wave per row.  Top k of a softmax: the same order as the logits' (exp is
// monotonic), so the selection runs on the logits, k rounds of a wave argmax
// (ties: the lower index); the kept probabilities exp(l - max) / sum are
// renormalized to sum 1.
constexpr int SHARED_ROUTE_PER_LANE = 16;  // experts per lane: up to 1024

__device__ __forceinline__ float round_act(float v, int dt) {
  if (dt == OUT_F16) return h2f(f2h(v));
  if (dt == OUT_BF16) return bf2f(f2bf(v));
  return v;
}

// The shared expert's gate of row `row` (one wave; every lane returns it):
// sigmoid of the given logit, or of f(x . gate_vec) summed lane-strided
// then across the wave, rounded to the activation dtype xdt.
__device__ __forceinline__ float shared_gate(size_t row, int lane, const void *logit,
                                             const void *gate_vec, const void *x, int xdt,
                                             int hidden) {
  float lg;
  if (logit != nullptr) {
    lg = load_act(logit, row, xdt);
  } else {
    float d = 0.0f;
    for (int i = lane; i < hidden; i += 64)
      d += load_act(x, row * hidden + i, xdt) * load_act(gate_vec, i, xdt);
    for (int m = 32; m >= 1; m >>= 1) d += __shfl_xor(d, m, 64);
    lg = round_act(d, xdt);
  }
  return round_act(1.0f / (1.0f + expf(-lg)), xdt);
}

__global__ __launch_bounds__(64) void moe_shared_route_kernel(
    const uint32_t *__restrict__ inds, const void *__restrict__ scores, int sdt,
    const void *__restrict__ logits, int E, int k, const void *__restrict__ logit,
    const void *__restrict__ gate_vec, const void *__restrict__ x, int xdt, int hidden,
    uint32_t *__restrict__ inds_out, float *__restrict__ scores_out) {
  const size_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const int kk = k + 1;
  if (logits != nullptr) {
    float l[SHARED_ROUTE_PER_LANE];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < SHARED_ROUTE_PER_LANE; ++i) {
      const int e = lane + 64 * i;
      l[i] = e < E ? load_act(logits, row * E + e, xdt) : -INFINITY;
      mx = fmaxf(mx, l[i]);
    }
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < SHARED_ROUTE_PER_LANE; ++i)
      if (lane + 64 * i < E) sum += expf(l[i] - mx);
    for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 64);
    uint32_t taken = 0;
    float kept = 0.0f, pk = 0.0f;
    int ek = 0;
    for (int j = 0; j < k; ++j) {
      float bv = -INFINITY;
      int bi = 0x7FFFFFFF;
#pragma unroll
      for (int i = 0; i < SHARED_ROUTE_PER_LANE; ++i) {
        const int e = lane + 64 * i;
        if (e < E && !(taken & (1u << i)) && (l[i] > bv || (l[i] == bv && e < bi))) {
          bv = l[i];
          bi = e;
        }
      }
      for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(bv, m, 64);
        const int oi = __shfl_xor(bi, m, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
      const float p = expf(bv - mx) / sum;
      kept += p;
      if (lane == j) {
        pk = p;
        ek = bi;
      }
    }
    if (lane < k) {
      inds_out[row * kk + lane] = (uint32_t)ek;
      scores_out[row * kk + lane] = pk / kept;
    }
  } else if (lane < k) {
    inds_out[row * kk + lane] = inds[row * k + lane];
    scores_out[row * kk + lane] = load_act(scores, row * k + lane, sdt);
  }
  const float gate = shared_gate(row, lane, logit, gate_vec, x, xdt, hidden);
  if (lane == 0) {
    inds_out[row * kk + k] = (uint32_t)E;
    scores_out[row * kk + k] = gate;
  }
}

// The combine of a one-row swiglu_shared call whose k routes are given
// (no route launch): y[row] = sum over the routed slots j < k (expert below
// experts) of score_j * d[slot j], then + gate * d[slot k], gate the shared
// expert's sigmoid formed here by one wave as moe_shared_route_kernel forms
// it; the same f32 operations in the same order as moe_combine_kernel over
// that kernel's (k + 1)-wide routes, so results are equal bit for bit.
__global__ __launch_bounds__(256) void moe_combine_shared_kernel(
    const uint16_t *__restrict__ d, const uint32_t *__restrict__ inds,
    const void *__restrict__ scores, int sdt, int k, int experts,
    const void *__restrict__ logit, const void *__restrict__ gate_vec,
    const void *__restrict__ x, int xdt, int hidden, void *__restrict__ y, int ydt) {
  __shared__ float gsh;
  const size_t row = blockIdx.y;
  if (threadIdx.x < 64) {
    const float gate = shared_gate(row, (int)threadIdx.x, logit, gate_vec, x, xdt, hidden);
    if (threadIdx.x == 0) gsh = gate;
  }
  __syncthreads();
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= hidden) return;
  const size_t kk = (size_t)k + 1;
  float acc = 0.0f;
  for (int j = 0; j < k; ++j) {
    const uint32_t e = inds[row * k + j];
    if (e >= (uint32_t)experts) continue;
    const float w = load_act(scores, row * k + j, sdt);
    acc = acc + f32_value(w * h2f(d[(row * kk + j) * hidden + i]));
  }
  acc = acc + f32_value(gsh * h2f(d[(row * kk + k) * hidden + i]));
  if (ydt == OUT_F16)
    ((uint16_t *)y)[row * hidden + i] = f2h(acc);
  else if (ydt == OUT_BF16)
    ((uint16_t *)y)[row * hidden + i] = f2bf(acc);
  else
    ((float *)y)[row * hidden + i] = acc;
}

hipError_t launch_moe_shared_route(const uint32_t *inds, const void *scores, int sdt,
                                   const void *logits, int experts, int k, const void *logit,
                                   const void *gate_vec, const void *x, int xdt, int rows,
                                   int hidden, uint32_t *inds_out, float *scores_out,
                                   hipStream_t s) {
  if (rows <= 0 || k <= 0 || k > 63 || experts <= 0 || experts > 64 * SHARED_ROUTE_PER_LANE ||
      (logits == nullptr && (inds == nullptr || scores == nullptr)) ||
      (logit == nullptr && (gate_vec == nullptr || x == nullptr)))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(moe_shared_route_kernel, dim3(rows), dim3(64), 0, s, inds, scores, sdt,
                     logits, experts, k, logit, gate_vec, x, xdt, hidden, inds_out, scores_out);
  return hipGetLastError();
}

namespace {

struct MoeLayout {
  size_t sorted, items, n_items, g, u, xd, d, xg, xu, total;
  size_t partial_floats;  // slots in the separate slot buffer: gate, up, down
  int slots, max_items, ks_gu, ks_d, tps_gu, tps_d;
  bool gemm;  // prefill-sized expert batches: grouped GEMMs over 256-slot items
  bool direct;  // one row, routes given: every slot its own one-row item
};

// Down GEMV launches of at most this many workgroups take the mid step in
// their prepare (measured on the DeepSeek-V3 shape: 1008 workgroups at
// batch 1 gain ~3 us a call, 8064 at batch 16 lose ~11 us).
constexpr size_t MOE_FUSED_MID_MAX_WG = 2048;

// Grouped GEMMs when the slots average at least this many per expert (and
// every rate is an integer rate); below, the routed GEMV items.
constexpr int MOE_GEMM_SLOTS_PER_EXPERT = 32;

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

bool moe_uses_gemm(const MoeArgs &a, bool gu_generic, bool d_generic) {
  const long slots = (long)a.rows * a.topk;
  return !gu_generic && !d_generic && a.inds != nullptr && !a.verify_rows &&
         slots >= (long)MOE_GEMM_SLOTS_PER_EXPERT * a.experts;
}

namespace {

// A grouped GEMV launch's k-splits: as many as keep the launch within 768
// workgroups (three a CU; the grouped kernel's registers hold two a CU
// resident, and the third starts as the first two end: a further partial
// round and the split-K hand-off cost more than the longer splits;
// DeepSeek-V3's down at one row: 448 workgroups unsplit, 3 % faster a call
// than 896 in two splits), splits of at most MOE_TPS_MAX k-tiles, or
// MOE_DIRECT_TPS_MAX for one-row items (direct: DeepSeek-V3's gate+up at one
// row in 3 splits of 19 blocks, 768 workgroups, ~4 % faster a call than 4
// splits of up to 16 blocks, 1024 workgroups).
constexpr int MOE_RESIDENT_WG = 3 * 256;
void moe_plan(int in, int out, int groups, bool direct, int *ksplit, int *tps) {
  const int nb = in / 128;
  const int cgs = std::max(1, out / 128) * std::max(1, groups);
  const int ks = std::min(nb, std::max(1, MOE_RESIDENT_WG / cgs));
  int bps = std::min((direct ? MOE_DIRECT_TPS_MAX : MOE_TPS_MAX) / 8, (nb + ks - 1) / ks);
  bps = std::max(bps, (nb + GEMV_KSPLIT_MAX - 1) / GEMV_KSPLIT_MAX);
  // splits of even length: the fewest splits of at most bps blocks, then
  // the blocks spread over them (56 blocks at most 32 a split: 28 + 28, not
  // 32 + 24)
  const int nsplit = (nb + bps - 1) / bps;
  bps = (nb + nsplit - 1) / nsplit;
  *tps = 8 * bps;
  *ksplit = (nb + bps - 1) / bps;
}

MoeLayout moe_layout(const MoeArgs &a, bool generic_gu, bool generic_d) {
  MoeLayout L{};
  const int slots = a.rows * a.topk;
  L.slots = slots;
  L.gemm = moe_uses_gemm(a, generic_gu, generic_d);
  // one row with its routes given: every slot its own work item, read from
  // the routes directly (no route launch; a row's routes name distinct
  // experts, and a repeated one would only be read twice)
  L.direct = !L.gemm && a.rows == 1 && a.inds != nullptr;
  const int item_rows = L.gemm ? GM_BM : MOE_ITEM_ROWS;
  L.max_items = std::min(a.experts, slots) + (slots + item_rows - 1) / item_rows;
  const int groups = std::max(1, std::min(a.experts, slots));
  moe_plan(a.hidden, a.inter, 2 * groups, L.direct, &L.ks_gu, &L.tps_gu);
  moe_plan(a.inter, a.hidden, groups, L.direct, &L.ks_d, &L.tps_d);
  if (generic_gu && L.tps_gu > 32) {
    L.tps_gu = 32;
    L.ks_gu = (a.hidden / 16 + 31) / 32;
  }
  if (generic_d && L.tps_d > 32) {
    L.tps_d = 32;
    L.ks_d = (a.inter / 16 + 31) / 32;
  }
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align256(bytes);
    return at;
  };
  L.sorted = take((size_t)slots * 4);
  L.items = take((size_t)L.max_items * sizeof(MoeItem));
  L.n_items = take(4);
  L.g = take((size_t)slots * a.inter * 2);
  L.u = take((size_t)slots * a.inter * 2);
  L.xd = take((size_t)slots * a.inter * 2);
  L.d = take((size_t)slots * a.hidden * 2);
  if (L.gemm) {
    L.xg = take((size_t)slots * a.hidden * 2);
    L.xu = take((size_t)slots * a.hidden * 2);
  }
  L.total = o;
  L.partial_floats = L.gemm ? 1
                            : (size_t)2 * L.ks_gu * slots * a.inter + (size_t)L.ks_d * slots * a.hidden;
  return L;
}

// One grouped GEMV launch over `nweights` banks (gate and up side by side,
// or down); x holds raw rows (slot / topk) or prepared rows (slot); pro
// PRO_SWIGLU: x the slots' gate rows, a.c.x2 their up rows.
struct MoeGemv {
  const uint32_t *tw[2];
  int nweights;
  const void *x;
  int xdt;
  bool prepared;
  int pro;
  int in, out, ksplit, tps;
  GemvArgs a;
};

// The launch's packed geometry; false when a field does not fit.
bool moe_geo(const MoeGemv &m, dim3 grid, uint32_t *g0, uint32_t *g1, uint32_t *g2) {
  GemvGeo geo{};
  geo.cg1 = m.nweights > 1 ? m.out / 128 : 0;
  geo.cgend = (int)grid.x;
  geo.rows = MOE_ITEM_ROWS;
  geo.xdt = m.xdt;
  geo.prepared = m.prepared ? 1 : 0;
  geo.in_tiles = m.in / 16;
  geo.tps = m.tps;
  return gemv_geo_pack(geo, g0, g1, g2);
}

void moe_gemv_launch(const Format &f, dim3 grid, size_t lds, hipStream_t s, const MoeGemv &m,
                     const uint32_t *sorted, const MoeItem *items, const uint32_t *n_items,
                     int topk) {
  uint32_t g0, g1, g2;
  if (!moe_geo(m, grid, &g0, &g1, &g2)) return;  // checked before the first launch
  rate_dispatch(f.integer_rate() ? f.n / 16 : 0, [&](auto KC) {
    moe_gemv_go<decltype(KC)::value>(f, m.pro, grid, lds, s, m.tw[0], m.tw[1], m.x, g0, g1, g2,
                                     topk, sorted, items, n_items, m.a);
  });
}

GemvWeight moe_weight(const MoeBank &b, uint16_t *y, float *partial) {
  GemvWeight w{};
  w.suh = b.suh;
  w.svh = b.svh;
  w.y = y;
  w.zout = nullptr;
  w.partial = partial;
  w.expert_words = (size_t)(b.in / 16) * (b.out / 16) * (b.f.n / 2);
  return w;
}

MoeGemv moe_gemv(const void *x, int xdt, bool prepared, size_t slots, int in, int out,
                 const Format &f, int ksplit, int tps) {
  MoeGemv m{};
  m.x = x;
  m.xdt = xdt;
  m.prepared = prepared;
  m.in = in;
  m.out = out;
  m.ksplit = ksplit;
  m.tps = tps;
  m.a.c.ydt = OUT_F16;
  m.a.c.ptotal = slots;
  m.a.c.ksplit = ksplit;
  m.a.c.dec = f.dec();
  m.a.c.nw = f.n / 2;
  m.a.c.shared_expert = -1;
  return m;
}

}  // namespace

bool moe_shared_direct(const MoeArgs &a, bool gu_generic, bool d_generic) {
  if (a.rows != 1 || a.topk <= 0 || a.experts <= 0 || a.hidden % 128 != 0) return false;
  const MoeLayout L = moe_layout(a, gu_generic, d_generic);
  return !L.gemm &&
         (size_t)(a.hidden / 128) * L.ks_d * L.slots <= MOE_FUSED_MID_MAX_WG;
}

size_t moe_scratch_bytes(const MoeArgs &a, bool gu_generic, bool d_generic,
                         size_t *partial_floats) {
  if (a.rows <= 0 || a.topk <= 0) {
    *partial_floats = 1;
    return 256;
  }
  const MoeLayout L = moe_layout(a, gu_generic, d_generic);
  *partial_floats = L.partial_floats;
  return L.total;
}

hipError_t launch_moe(const MoeArgs &a, const MoeBank &gate, const MoeBank &up,
                      const MoeBank &down, void *scratch, size_t scratch_bytes,
                      const Scratch &slots, hipStream_t s, const MoeShared *shared) {
  if (a.rows <= 0 || a.topk <= 0 || a.experts <= 0 || a.experts > MOE_ROUTE_THREADS)
    return hipErrorInvalidValue;
  if (a.hidden % 128 != 0 || a.inter % 128 != 0) return hipErrorInvalidValue;
  if (a.hidden / 16 > 65535 || a.inter / 16 > 65535) return hipErrorInvalidValue;
  if (gate.f.n != up.f.n || !gate.f.same_decode(up.f) ||
      gate.in != a.hidden || up.in != a.hidden || down.out != a.hidden || gate.out != a.inter ||
      up.out != a.inter || down.in != a.inter)
    return hipErrorInvalidValue;
  const bool gu_generic = !gate.f.integer_rate(), d_generic = !down.f.integer_rate();
  const MoeLayout L = moe_layout(a, gu_generic, d_generic);
  if (shared) {
    auto same = [](const MoeBank &b, const MoeBank &r) {
      return b.trellis && b.suh && b.svh && b.in == r.in && b.out == r.out && b.f.n == r.f.n &&
             b.f.same_decode(r.f);
    };
    if (L.gemm || a.inds == nullptr || !same(shared->gate, gate) || !same(shared->up, up) ||
        !same(shared->down, down))
      return hipErrorInvalidValue;
  }
  const int sh_index = shared ? a.experts - 1 : -1;
  // one row, k routes given: slot k is the shared expert, no route launch
  const int routes_k = shared ? shared->routes_k : 0;
  if (routes_k > 0 && (a.rows != 1 || a.inds == nullptr || a.topk != routes_k + 1 ||
                       (shared->logit == nullptr && shared->gate_vec == nullptr)))
    return hipErrorInvalidValue;
  if (scratch_bytes < L.total || slots.status == nullptr || slots.partial == nullptr ||
      slots.partial_floats < L.partial_floats || L.slots > MOE_SLOTS_MAX ||
      L.max_items > 65535 || (int64_t)L.slots * std::max(a.hidden, a.inter) >= (int64_t)1 << 31)
    return hipErrorInvalidValue;
  float *partial = slots.partial;
  char *base = (char *)scratch;
  uint32_t *sorted = (uint32_t *)(base + L.sorted);
  MoeItem *items = (MoeItem *)(base + L.items);
  uint32_t *n_items = (uint32_t *)(base + L.n_items);
  uint16_t *g = (uint16_t *)(base + L.g), *u = (uint16_t *)(base + L.u);
  uint16_t *xd = (uint16_t *)(base + L.xd), *d = (uint16_t *)(base + L.d);
  float *pgu = partial, *pd = partial + (size_t)2 * L.ks_gu * L.slots * a.inter;

  if (L.gemm) {
    // prefill-sized expert batches: per-slot prepared rows, grouped GEMMs
    // gate and up, the mid step, grouped GEMM down, the weighted sum
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(MOE_ROUTE_THREADS), 0, s, a.inds, L.slots,
                       a.experts, sorted, items, n_items, (uint32_t)GM_BM);
    uint16_t *xg = (uint16_t *)(base + L.xg), *xu = (uint16_t *)(base + L.xu);
    const int nblk = a.hidden / 128;
    hipLaunchKernelGGL(moe_prep_kernel, dim3((nblk + 3) / 4, L.slots), dim3(256), 0, s, a.x,
                       a.xdt, a.inds, a.experts, a.topk, gate.suh, up.suh, xg, xu, a.hidden, nblk);
    auto grouped = [&](const MoeBank &b, const uint16_t *xp, uint16_t *yo) {
      GemmGroup gg{sorted, items, n_items, (size_t)(b.in / 16) * (b.out / 16) * (b.f.n / 2)};
      const dim3 grid(b.out / 128, L.max_items);
      const uint32_t *tw = reinterpret_cast<const uint32_t *>(b.trellis);
      rate_dispatch(b.f.n / 16, [&](auto KC) {
        constexpr int K = decltype(KC)::value;
        if constexpr (K > 0)
          gemm_grouped_go<K>(b.f, grid, s, tw, xp, b.svh, yo, OUT_F16, b.in / 16, b.out / 16, gg);
      });
    };
    grouped(gate, xg, g);
    grouped(up, xu, u);
    hipLaunchKernelGGL(moe_mid_kernel, dim3(a.inter / 128, L.slots), dim3(64), 0, s, g, u, a.inds,
                       a.experts, down.suh, xd, a.inter, a.limit, -1, nullptr);
    grouped(down, xd, d);
    hipLaunchKernelGGL(moe_combine_kernel, dim3((a.hidden + 255) / 256, a.rows), dim3(256), 0, s,
                       d, a.inds, a.scores, a.sdt, a.topk, a.experts, a.hidden, a.y, a.ydt);
    return hipGetLastError();
  }
  const size_t gu_part = (size_t)L.ks_gu * L.slots * a.inter;
  MoeGemv mgu = moe_gemv(a.x, a.xdt, false, L.slots, a.hidden, a.inter, gate.f, L.ks_gu, L.tps_gu);
  mgu.nweights = 2;
  // one-row items (direct) allocate one row of LDS
  const bool direct = L.direct;
  const int nz = direct ? L.slots : L.max_items;
  const dim3 grid_gu(2 * (a.inter / 128), L.ks_gu, nz);
  const dim3 grid_d(a.hidden / 128, L.ks_d, nz);
  // down: in a launch of few workgroups every workgroup forms the mid step
  // (the SwiGLU of its slots' gate and up rows, the down rotation) for its
  // k-slice in its prepare, which costs less than the mid launch; in larger
  // launches the repeats across column groups cost more than the launch
  const bool fused_mid = (size_t)grid_d.x * grid_d.y * grid_d.z <= MOE_FUSED_MID_MAX_WG;
  if (routes_k > 0 && !fused_mid) return hipErrorInvalidValue;
  MoeGemv md = fused_mid ? moe_gemv(g, OUT_F16, false, L.slots, a.inter, a.hidden, down.f, L.ks_d,
                                    L.tps_d)
                         : moe_gemv(xd, OUT_F16, true, L.slots, a.inter, a.hidden, down.f, L.ks_d,
                                    L.tps_d);
  md.nweights = 1;
  if (fused_mid) {
    md.pro = PRO_SWIGLU;
    md.a.c.x2 = u;
    md.a.c.limit = a.limit;
  }
  mgu.a.c.status = md.a.c.status = slots.status;
  mgu.a.c.poll_max = md.a.c.poll_max = splitk_poll_max();
  mgu.a.c.drop_partials = md.a.c.drop_partials = splitk_drop();
  uint32_t gg[3];
  if (!moe_geo(mgu, grid_gu, &gg[0], &gg[1], &gg[2]) || !moe_geo(md, grid_d, &gg[0], &gg[1], &gg[2]))
    return hipErrorInvalidValue;
  if (!direct)
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(MOE_ROUTE_THREADS), 0, s, a.inds, L.slots,
                       a.experts, sorted, items, n_items, (uint32_t)MOE_ITEM_ROWS);
  const uint32_t *isorted = direct ? a.inds : sorted;
  const MoeItem *iitems = direct ? nullptr : items;
  const uint32_t *in_items = direct ? nullptr : n_items;
  mgu.a.c.experts = md.a.c.experts = a.experts;
  mgu.a.c.routes_k = md.a.c.routes_k = routes_k;
  mgu.tw[0] = reinterpret_cast<const uint32_t *>(gate.trellis);
  mgu.tw[1] = reinterpret_cast<const uint32_t *>(up.trellis);
  mgu.a.w[0] = moe_weight(gate, g, pgu);
  mgu.a.w[1] = moe_weight(up, u, pgu + gu_part);
  if (shared) {
    mgu.a.c.shared_expert = md.a.c.shared_expert = sh_index;
    const MoeBank *sb[2] = {&shared->gate, &shared->up};
    for (int i = 0; i < 2; ++i) {
      mgu.a.w[i].sh_tw = reinterpret_cast<const uint32_t *>(sb[i]->trellis);
      mgu.a.w[i].sh_suh = sb[i]->suh;
      mgu.a.w[i].sh_svh = sb[i]->svh;
    }
  }
  const int lds_rows = direct ? 1 : MOE_ITEM_ROWS;
  moe_gemv_launch(gate.f, grid_gu, gemv_lds_bytes(lds_rows, L.tps_gu, gu_generic), s, mgu,
                  isorted, iitems, in_items, a.topk);
  if (!fused_mid)
    hipLaunchKernelGGL(moe_mid_kernel, dim3(a.inter / 128, L.slots), dim3(64), 0, s, g, u, a.inds,
                       a.experts, down.suh, xd, a.inter, a.limit, sh_index,
                       shared ? shared->down.suh : nullptr);
  md.tw[0] = md.tw[1] = reinterpret_cast<const uint32_t *>(down.trellis);
  md.a.w[0] = moe_weight(down, d, pd);
  if (shared) {
    md.a.w[0].sh_tw = reinterpret_cast<const uint32_t *>(shared->down.trellis);
    md.a.w[0].sh_suh = shared->down.suh;
    md.a.w[0].sh_svh = shared->down.svh;
  }
  moe_gemv_launch(down.f, grid_d, gemv_lds_bytes(lds_rows, L.tps_d, d_generic), s, md,
                  isorted, iitems, in_items, fused_mid ? 1 : a.topk);
  if (routes_k > 0)
    hipLaunchKernelGGL(moe_combine_shared_kernel, dim3((a.hidden + 255) / 256, 1), dim3(256), 0,
                       s, d, a.inds, a.scores, a.sdt, routes_k, a.experts, shared->logit,
                       shared->gate_vec, a.x, a.xdt, a.hidden, a.y, a.ydt);
  else
    hipLaunchKernelGGL(moe_combine_kernel, dim3((a.hidden + 255) / 256, a.rows), dim3(256), 0, s,
                       d, a.inds, a.scores, a.sdt, a.topk, a.experts, a.hidden, a.y, a.ydt);
  return hipGetLastError();
}

}  // namespace exl3
