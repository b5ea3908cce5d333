// Host-visible pieces of the INT8 GEMM: the kernel parameter block and the
// per-(epilogue, output dtype) launchers. The launchers are defined in
// gemm_kernels.h and instantiated one pair per object file by gemm_inst.hip;
// gemm_api.hip (the C ABI) only calls them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "w8a8_host.h"

namespace w8a8 {

struct GemmParams {
  const int8_t* a;
  const int8_t* b;
  int64_t lda, ldb;
  int m, n, k;
  const float* row_scale;
  const float* col_scale;
  int col_stride;
  int cs_vec;       // col_scale has stride 1 and a 16-byte aligned base (float4 loads)
  int bias_dtype;   // 0 none, kF16, kF32
  const void* bias;
  const uint16_t* residual;
  int64_t ldr;
  void* out;
  int64_t ldc;
  int vec_out;  // out rows allow 4-element vector stores (16-byte base, ldc % 4 == 0)
  int vec16;    // out (and residual) rows are 16-byte aligned: staged full-row stores
};

// EPI: kEpiInt32 / kEpiRow / kEpiColumn; OUT: kI32 / kF16 / kBF16 / kF32.
template <int EPI, int OUT>
int launch_gemm(const GemmParams& p, hipStream_t s);

template <int EPI, int OUT>
void launch_dequant(const GemmParams& p, const int32_t* acc, int64_t ldacc, hipStream_t s);

}  // namespace w8a8
