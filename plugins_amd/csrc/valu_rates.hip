// valu_rates.hip -- issue cost of the VALU instructions in the mul1 decode
// on the GPU it runs on (a measurement program, not part of the library).
//
// The decode of a mul1 codeword is a bit-field extract, a 32-bit integer
// multiply (v_mul_lo_u32) and a byte sum (v_sad_u8).  SQ_INSTS_VALU counts
// instructions, not the cycles each holds its SIMD, so the GEMV's VALU
// ceiling needs the multiply's cost beside the full-rate instructions'.
// Three kernels run the same loop, 8 independent codeword chains per lane
// and 8 waves per SIMD, and differ in one instruction per codeword:
//   0: v_mul_lo_u32 (x = cw * 0x83DCD12D, the mul1 hash)
//   1: v_xor_b32    (a full-rate instruction in the same place)
//   2: v_mul_u32_u24
// The time difference per wave-instruction against kernel 1 is the extra
// issue cost of that instruction, in cycles.
//
//   python -m plugins_amd.build --valu-rates && plugins_amd/lib/valu_rates
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

namespace {

constexpr uint32_t MUL1 = 0x83DCD12Du;
constexpr int THREADS = 256, CHAINS = 8;

// clk (block 0, thread 0): the shader-clock and 100 MHz counters at the loop's
// start and end, so the clock the loop ran at is measured with it.
template <int MODE>
__global__ __launch_bounds__(THREADS) void chain_kernel(uint32_t *out, int iters, uint32_t seed,
                                                        unsigned long long *clk) {
  const bool probe = blockIdx.x == 0 && threadIdx.x == 0;
  unsigned long long c0 = 0, r0 = 0;
  if (probe) {
    c0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  uint32_t c[CHAINS], acc[CHAINS];
#pragma unroll
  for (int j = 0; j < CHAINS; ++j) {
    c[j] = (threadIdx.x * CHAINS + j + seed) & 0xFFFFu;
    acc[j] = 0u;
  }
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < CHAINS; ++j) {
      uint32_t x;
      if constexpr (MODE == 0) x = c[j] * MUL1;
      if constexpr (MODE == 1) x = c[j] ^ MUL1;
      if constexpr (MODE == 2) x = __umul24(c[j], 0xD12Du);
      acc[j] = __builtin_amdgcn_sad_u8(x, 0u, acc[j]);
      c[j] = (c[j] + acc[j]) & 0xFFFFu;
    }
  }
  uint32_t s = 0u;
#pragma unroll
  for (int j = 0; j < CHAINS; ++j) s += acc[j];
  out[(size_t)blockIdx.x * THREADS + threadIdx.x] = s;
  if (probe) {
    clk[0] = __builtin_amdgcn_s_memtime() - c0;
    clk[1] = __builtin_amdgcn_s_memrealtime() - r0;
  }
}

#define CHECK(e)                                                             \
  do {                                                                       \
    const hipError_t r_ = (e);                                               \
    if (r_ != hipSuccess) {                                                  \
      std::fprintf(stderr, "%s: %s\n", #e, hipGetErrorString(r_));           \
      std::exit(1);                                                          \
    }                                                                        \
  } while (0)

template <int MODE>
float time_ms(uint32_t *out, unsigned long long *clk, int blocks, int iters, int reps,
              double *ghz) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  chain_kernel<MODE><<<blocks, THREADS>>>(out, iters, 1u, clk);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(a));
  for (int r = 0; r < reps; ++r)
    chain_kernel<MODE><<<blocks, THREADS>>>(out, iters, (uint32_t)r, clk);
  CHECK(hipEventRecord(b));
  CHECK(hipEventSynchronize(b));
  float ms = 0.0f;
  CHECK(hipEventElapsedTime(&ms, a, b));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  unsigned long long h[2];
  CHECK(hipMemcpy(h, clk, sizeof(h), hipMemcpyDeviceToHost));
  *ghz = h[1] ? (double)h[0] / (double)h[1] * 0.1 : 0.0;  // the real-time counter runs at 100 MHz
  return ms / (float)reps;
}

}  // namespace

int main() {
  hipDeviceProp_t p;
  CHECK(hipGetDeviceProperties(&p, 0));
  const int simds = p.multiProcessorCount * 4;
  const int blocks = p.multiProcessorCount * 8;  // 8 waves per SIMD
  const int iters = 2048, reps = 5;
  uint32_t *out = nullptr;
  unsigned long long *clk = nullptr;
  CHECK(hipMalloc(&out, (size_t)blocks * THREADS * sizeof(uint32_t)));
  CHECK(hipMalloc(&clk, 2 * sizeof(unsigned long long)));
  double ghz[3];
  const float t[3] = {time_ms<0>(out, clk, blocks, iters, reps, &ghz[0]),
                      time_ms<1>(out, clk, blocks, iters, reps, &ghz[1]),
                      time_ms<2>(out, clk, blocks, iters, reps, &ghz[2])};
  CHECK(hipFree(out));
  CHECK(hipFree(clk));
  // wave-instructions of the varying kind per SIMD
  const double per_simd = (double)blocks * (THREADS / 64) * iters * CHAINS / simds;
  const char *names[3] = {"v_mul_lo_u32", "v_xor_b32 (full rate)", "v_mul_u32_u24"};
  std::printf("device %s, %d CUs, %d SIMDs; %d blocks x %d threads, %d iterations x %d chains\n",
              p.name, p.multiProcessorCount, simds, blocks, THREADS, iters, CHAINS);
  for (int m = 0; m < 3; ++m) {
    const double extra_ns = (t[m] - t[1]) * 1e6 / per_simd;
    std::printf("%-22s %.3f ms at %.2f GHz; extra per wave-instruction vs v_xor_b32: %.3f ns = "
                "%.2f cycles\n",
                names[m], t[m], ghz[m], extra_ns, extra_ns * ghz[m]);
  }
  return 0;
}
