// exl3_rate.hip -- one rate's instantiation of the EXL3 GEMV / GEMM / grouped
// MoE GEMV kernels.  The build compiles this file once per K (0..8) with
// -DEXL3_INST_K=K: K = 1..8 are the integer rates n = 16K with compile-time
// bit windows, K = 0 the run-time window form for any even n (GEMV) and the
// half-integer rates' GEMM (n = 24, 40).
#include "exl3_kern.h"

#ifndef EXL3_INST_K
#error "exl3_rate.hip is built with -DEXL3_INST_K=<rate>"
#endif

namespace exl3 {

template EXL3_GEMV_GO(EXL3_INST_K);
template EXL3_MOE_GEMV_GO(EXL3_INST_K);
#if EXL3_INST_K > 0
template EXL3_GEMM_GO(EXL3_INST_K);
template EXL3_GEMM_GROUPED_GO(EXL3_INST_K);
#else
// the half-integer rates' prefill GEMM (n = 24, 40)
template EXL3_GEMM_FRAC_GO(3);
template EXL3_GEMM_FRAC_GO(5);
#endif

}  // namespace exl3

