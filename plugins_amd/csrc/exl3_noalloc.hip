// exl3_noalloc.hip -- the scratch of exl3_matmul_noalloc: a file-scope device
// array instead of allocations, for callers that cannot call hipMalloc (code
// under HIP graph capture, tight serving loops, harnesses that forbid it).
//
// Each GPU the library runs on holds its own copy of the array, at its own
// address, from the moment the library's code object is loaded onto it until
// the process ends.  Host code never uses the array's name as an address: the
// set-up below asks HIP for the array's device address on each device (with
// that device current) and every launch gets that pointer.
//
// Layout (NOALLOC_* in exl3_kernels.h):
//   [0, NOALLOC_SLOT_BYTES)            a slot buffer: the status word's header,
//                                      then GEMV split-K partial-sum slots,
//                                      which hold the empty mark between calls
//   [NOALLOC_SLOT_BYTES, NOALLOC_BYTES) staging: the GEMM's prepared rows,
//                                      then its split-K planes
// Every call leaves the slots empty and the status word as it found it (zero
// unless a split-K wait gave up: exl3_stream_status reads the word, and after
// a give-up refills the slots and clears it), and overwrites the staging it
// uses, so the array needs no clearing between calls; calls that overlap on
// one GPU (two streams at once) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "exl3_kernels.h"

namespace exl3 {

static __device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void *g_ptr[MAX_DEVICES] = {};

}  // namespace

hipError_t noalloc_scratch(int device, hipStream_t s, void **base) {
  if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(g_mu);
  if (g_ptr[device] == nullptr) {
    // set-up, once per device, with that device current (the caller's
    // hipSetDevice): the array's address on this device, then the slots'
    // empty mark (the array starts zeroed), done before the first use
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return hipErrorStreamCaptureUnsupported;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    e = hipMemsetAsync(p, 0, SLOT_HEADER_BYTES, s);
    if (e == hipSuccess)
      e = hipMemsetAsync((char *)p + SLOT_HEADER_BYTES, 0xFF,
                         NOALLOC_SLOT_BYTES - SLOT_HEADER_BYTES, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return e;
    g_ptr[device] = p;
  }
  *base = g_ptr[device];
  return hipSuccess;
}

hipError_t noalloc_status(int device, bool *gave_up) {
  if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(g_mu);
  if (g_ptr[device] == nullptr) return hipSuccess;  // never set up: no call ran
  uint32_t st = 0;
  hipError_t e = hipMemcpy(&st, g_ptr[device], 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess || st == 0) return e;
  *gave_up = true;
  // the caller has synchronized the stream of the calls: every late store
  // has landed, so the slots can take the empty mark again
  e = hipMemset((char *)g_ptr[device] + SLOT_HEADER_BYTES, 0xFF,
                NOALLOC_SLOT_BYTES - SLOT_HEADER_BYTES);
  if (e == hipSuccess) e = hipMemset(g_ptr[device], 0, 4);
  return e;
}

}  // namespace exl3
