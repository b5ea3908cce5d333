// One (epilogue, output dtype) instantiation of the INT8 GEMM launchers.
// The build compiles this file once per pair with -DW8A8_INST_EPI=<e>
// -DW8A8_INST_OUT=<o> (e: 0 int32, 1 row, 2 column; o: 1 f16, 2 bf16,
// 3 f32, 4 i32), so the seven variants compile in parallel.
#include "gemm_kernels.h"

#ifndef W8A8_INST_EPI
#error "compile gemm_inst.hip with -DW8A8_INST_EPI and -DW8A8_INST_OUT"
#endif

namespace w8a8 {

template int launch_gemm<W8A8_INST_EPI, W8A8_INST_OUT>(const GemmParams&, hipStream_t);

#if W8A8_INST_EPI != 0
template void launch_dequant<W8A8_INST_EPI, W8A8_INST_OUT>(const GemmParams&, const int32_t*, int64_t,
                                                           hipStream_t);
#else
int launch_gemm_partials(const GemmParams& p, const GemmPlan& plan, int dev, hipStream_t s) {
  return launch_persistent_nb<kEpiInt32, kI32, 0>(p, plan, dev, s);
}

// K split and workspace bytes of an m x n x k GEMM. M <= 64 takes the
// weight-streaming kernel's split (stream_ksplit); above, the persistent
// kernel's plan (gemm_plan).
int gemm_ksplit(int64_t m, int64_t n, int64_t k, int dev, int64_t* workspace_bytes) {
  *workspace_bytes = 0;
  if (m <= kSkinnyMaxM) {   // the weight-streaming kernel's own split
    if (!stream_applies(m, n, k, device_cus(dev))) return 1;
    const int ks = stream_ksplit(n, k, device_cus(dev));
    if (ks > 1) *workspace_bytes = (int64_t)ks * m * n * 4;
    return ks;
  }
  if (k % kSK != 0) return 1;
  if ((m - 1) * k + k >= (1ll << 32) || (n - 1) * k + k >= (1ll << 32)) return 1;
  const GemmPlan plan = gemm_plan(m, n, k, device_cus(dev));
  *workspace_bytes = split_partials_bytes(m, n, plan.ksplit);
  return plan.ksplit;
}
#endif

}  // namespace w8a8
