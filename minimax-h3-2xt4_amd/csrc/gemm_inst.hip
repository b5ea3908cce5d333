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
#endif

}  // namespace w8a8
