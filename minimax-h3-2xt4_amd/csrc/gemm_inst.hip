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
int launch_gemm_partials(const GemmParams& p, int dev, hipStream_t s) {
  const int64_t tiles = (int64_t)((p.m + kBM - 1) / kBM) * ((p.n + kBN - 1) / kBN);
  return launch_persistent<kEpiInt32, kI32, 0>(p, tiles, dev, s);
}

// K split and workspace bytes of an m x n x k GEMM. M <= 64 takes the
// weight-streaming kernel's split (stream_ksplit). Above, split K when the
// output tiles leave CUs idle. Cost model in units of one K = 128 stage of a
// 256x256 tile (about 1 us on the power-limited clock): rounds of work items
// times stages per item, plus the partial sums' write-and-read traffic at
// about 6.5 TB/s.
int gemm_ksplit(int64_t m, int64_t n, int64_t k, int dev, int64_t* workspace_bytes) {
  *workspace_bytes = 0;
  if (m <= kSkinnyMaxM) {   // the weight-streaming kernel's own split
    if (!stream_applies(m, k)) return 1;
    const int ks = stream_ksplit(n, k, device_cus(dev));
    if (ks > 1) *workspace_bytes = (int64_t)ks * m * n * 4;
    return ks;
  }
  if (k % kSK != 0) return 1;
  if ((m - 1) * k + k >= (1ll << 32) || (n - 1) * k + k >= (1ll << 32)) return 1;
  const int64_t tiles = ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN);
  const int64_t kstages = k / kSK, cus = device_cus(dev);
  if (tiles >= cus) return 1;
  int best = 1;
  double best_t = (double)kstages;
  for (int ks = 2; ks <= 8; ks *= 2) {
    if (kstages / ks < 2) break;
    const int64_t rounds = (tiles * ks + cus - 1) / cus;
    const double t = (double)(rounds * ((kstages + ks - 1) / ks)) + (double)ks * m * n * 8 / 6.5e12 * 1e6;
    if (t < 0.9 * best_t) {
      best = ks;
      best_t = t;
    }
  }
  if (best > 1) *workspace_bytes = (int64_t)best * m * n * 4;
  return best;
}
#endif

}  // namespace w8a8
