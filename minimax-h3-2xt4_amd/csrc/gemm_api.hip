// C ABI of the INT8 GEMM and the standalone epilogue: argument checks, then
// dispatch to the (epilogue, output dtype) launcher instantiated in
// gemm_inst.hip.
#include <mutex>

#include "gemm_launch.h"
#include "w8a8_device.h"

namespace w8a8 {

static int check_epilogue(int epi, int out_dtype, int bias_dtype, const void* bias, const void* residual,
                          int64_t ldr, const float* gate, const int32_t* labels, int64_t ldg, int64_t n,
                          const float* row_scale, const float* col_scale, int64_t col_stride, const void* out,
                          int64_t ldc) {
  W8A8_REQUIRE(out != nullptr, "null output");
  const int es = out_dtype == W8A8_F16 || out_dtype == W8A8_BF16 ? 2 : 4;
  W8A8_REQUIRE(((uintptr_t)out % es) == 0 && ldc >= n, "out must be element-aligned with ldc >= n");
  if (epi == W8A8_EPI_INT32) {
    W8A8_REQUIRE(out_dtype == W8A8_I32, "EPI_INT32 requires out_dtype I32");
    W8A8_REQUIRE(bias == nullptr && residual == nullptr && gate == nullptr,
                 "EPI_INT32 takes no bias, residual or gate");
    return W8A8_OK;
  }
  W8A8_REQUIRE(epi == W8A8_EPI_ROW || epi == W8A8_EPI_COLUMN, "unknown epilogue %d", epi);
  W8A8_REQUIRE(out_dtype == W8A8_F16 || out_dtype == W8A8_BF16 || out_dtype == W8A8_F32,
               "dequantized out_dtype must be F16, BF16 or F32");
  W8A8_REQUIRE(row_scale && col_scale, "row_scale and col_scale required");
  W8A8_REQUIRE(col_stride == 0 || col_stride == 1, "col_scale_stride must be 0 (scalar) or 1");
  W8A8_REQUIRE(bias == nullptr || bias_dtype == W8A8_F16 || bias_dtype == W8A8_F32,
               "bias_dtype must be F16 or F32");
  if (residual) {
    W8A8_REQUIRE(out_dtype == W8A8_F16, "residual requires F16 output");
    W8A8_REQUIRE(((uintptr_t)residual & 1u) == 0 && ldr >= n, "residual must be 2-byte aligned with ldr >= n");
  }
  if (gate) {
    W8A8_REQUIRE(residual != nullptr, "gate requires a residual");
    W8A8_REQUIRE(labels != nullptr && ldg >= n && ((uintptr_t)gate & 3u) == 0,
                 "gate requires gate_labels, a 4-byte aligned table and ldg >= n");
  }
  return W8A8_OK;
}

template <int EPI>
static int launch_gemm_out(int out, const GemmParams& p, hipStream_t s) {
  switch (out) {
    case kF16: return launch_gemm<EPI, kF16>(p, s);
    case kBF16: return launch_gemm<EPI, kBF16>(p, s);
    default: return launch_gemm<EPI, kF32>(p, s);
  }
}

template <int EPI>
static void launch_dequant_out(int out, const GemmParams& p, const int32_t* acc, int64_t ldacc, hipStream_t s) {
  switch (out) {
    case kF16: launch_dequant<EPI, kF16>(p, acc, ldacc, s); break;
    case kBF16: launch_dequant<EPI, kBF16>(p, acc, ldacc, s); break;
    default: launch_dequant<EPI, kF32>(p, acc, ldacc, s); break;
  }
}

// Shared epilogue fields of W8A8GemmArgs / W8A8DequantArgs.
template <typename Args>
static void fill_epilogue(GemmParams& p, const Args* a) {
  p.m = (int)a->m;
  p.n = (int)a->n;
  p.row_scale = a->row_scale;
  p.col_scale = a->col_scale;
  p.col_stride = (int)a->col_scale_stride;
  p.cs_vec = a->col_scale_stride == 1 && aligned16(a->col_scale);
  p.bias_dtype = a->bias ? a->bias_dtype : 0;
  p.bias = a->bias;
  p.residual = reinterpret_cast<const uint16_t*>(a->residual);
  p.ldr = a->ldr;
  p.gate = a->gate;
  p.labels = a->gate_labels;
  p.ldg = a->ldg;
  p.gvec = a->gate != nullptr && aligned16(a->gate) && a->ldg % 4 == 0;
  p.out = a->out;
  p.ldc = a->ldc;
  p.vec_out = aligned16(a->out) && a->ldc % 4 == 0;
}

}  // namespace w8a8

namespace w8a8 {

// Checks and dispatch shared by w8a8_gemm (the caller's workspace) and
// w8a8_gemm_noalloc (the file-scope scratch array).
static int gemm_entry(const W8A8GemmArgs* a, void* workspace, int64_t workspace_bytes) {
  W8A8_REQUIRE(a->m >= 0 && a->n >= 0 && a->k >= 0, "w8a8_gemm: negative shape");
  W8A8_REQUIRE(a->m < (1LL << 31) && a->n < (1LL << 31) && a->k < (1LL << 31), "w8a8_gemm: shape too large");
  W8A8_REQUIRE(a->k * 128 * 128 < (1LL << 31), "w8a8_gemm: k=%lld could overflow int32 accumulation",
               (long long)a->k);
  W8A8_REQUIRE(a->k % 16 == 0, "w8a8_gemm: k %lld not a multiple of 16", (long long)a->k);
  if (a->m == 0 || a->n == 0) return W8A8_OK;
  int rc = check_epilogue(a->epilogue, a->out_dtype, a->bias_dtype, a->bias, a->residual, a->ldr, a->gate,
                          a->gate_labels, a->ldg, a->n, a->row_scale, a->col_scale, a->col_scale_stride, a->out,
                          a->ldc);
  if (rc != W8A8_OK) return rc;
  W8A8_REQUIRE(a->k == 0 || (a->a && a->b), "w8a8_gemm: null operand");
  W8A8_REQUIRE(aligned16(a->a) && aligned16(a->b) && a->lda % 16 == 0 && a->ldb % 16 == 0 && a->lda >= a->k &&
                   a->ldb >= a->k,
               "w8a8_gemm: operands must be 16-byte aligned with lda, ldb %% 16 == 0 and >= k");
  const int64_t tiles = ((a->m + 255) / 256) * ((a->n + 255) / 256);
  W8A8_REQUIRE(tiles < (1LL << 31), "w8a8_gemm: too many tiles");
  GemmParams p{};
  fill_epilogue(p, a);
  p.a = a->a; p.b = a->b; p.lda = a->lda; p.ldb = a->ldb;
  p.k = (int)a->k;
  p.ksplit = 1;
  W8A8_REQUIRE(workspace_bytes >= 0 && (workspace == nullptr || aligned16(workspace)),
               "w8a8_gemm: workspace must be 16-byte aligned with workspace_bytes >= 0");
  p.ws = workspace_bytes > 0 ? workspace : nullptr;
  p.ws_bytes = workspace_bytes;
  {
    const int es = (a->out_dtype == W8A8_F16 || a->out_dtype == W8A8_BF16) ? 2 : 4;
    p.vec16 = aligned16(a->out) && (a->ldc * es) % 16 == 0 &&
              (a->residual == nullptr || (aligned16(a->residual) && a->ldr % 8 == 0));
  }
  if (a->rope) {
    const W8A8RopeEpilogue* r = a->rope;
    W8A8_REQUIRE(r->heads > 0 && 2 * (int64_t)r->heads * 128 <= a->n,
                 "w8a8_gemm: rope needs heads > 0 and n >= 2 * heads * 128");
    W8A8_REQUIRE(r->rot_dim > 0 && r->rot_dim <= 128 && r->rot_dim % 2 == 0, "w8a8_gemm: rope rot_dim %d invalid",
                 r->rot_dim);
    W8A8_REQUIRE(r->freq_dtype == W8A8_F16 || r->freq_dtype == W8A8_F32, "w8a8_gemm: rope freq_dtype not F16/F32");
    W8A8_REQUIRE(r->freq_layout == W8A8_ROPE_MATRICES || r->freq_layout == W8A8_ROPE_PAIRS,
                 "w8a8_gemm: rope freq_layout %d unknown", r->freq_layout);
    W8A8_REQUIRE(r->freqs && r->q_gain && r->k_gain && aligned16(r->freqs) && aligned16(r->q_gain) &&
                     aligned16(r->k_gain),
                 "w8a8_gemm: rope freqs and gains must be non-null and 16-byte aligned");
    if (a->epilogue == W8A8_EPI_INT32 || a->out_dtype != W8A8_F16 || a->bias || a->residual || a->gate ||
        (r->rot_dim / 2) % 8 != 0 || a->m <= 64 || a->k % 128 != 0 || !p.vec16 ||
        (a->m - 1) * a->lda + a->k >= (1LL << 32) || (a->n - 1) * a->ldb + a->k >= (1LL << 32)) {
      set_error("w8a8_gemm: the rope epilogue needs F16 output without bias/residual/gate, (rot_dim/2) %% 8 == 0, "
                "m > 64, k %% 128 == 0, 16-byte aligned output rows and operands under 4 GB");
      return W8A8_ERR_UNSUPPORTED;
    }
    p.rope_heads = r->heads;
    p.rope_rot = r->rot_dim;
    p.rope_half = r->rot_dim / 2;
    p.rope_f32 = r->freq_dtype == W8A8_F32;
    p.rope_pairs = r->freq_layout == W8A8_ROPE_PAIRS;
    p.rope_eps = r->eps;
    p.rope_freqs = r->freqs;
    p.rope_q_gain = r->q_gain;
    p.rope_k_gain = r->k_gain;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  int rc2;
  switch (a->epilogue) {
    case W8A8_EPI_INT32: rc2 = launch_gemm<kEpiInt32, kI32>(p, s); break;
    case W8A8_EPI_ROW: rc2 = launch_gemm_out<kEpiRow>(a->out_dtype, p, s); break;
    default: rc2 = launch_gemm_out<kEpiColumn>(a->out_dtype, p, s); break;
  }
  if (rc2 != W8A8_OK) return rc2;
  return launch_status("w8a8_gemm");
}

// No-allocation variant: the split-K partials of w8a8_gemm_noalloc live in
// this file-scope array, one instance per GPU, held until the process ends.
// Host code never passes `scratch` itself (its host-side name is not a device
// address): the entry point looks up each device's address once with
// hipGetSymbolAddress and passes that pointer to the kernels.
constexpr int64_t kScratchBytes = W8A8_GEMM_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[kScratchDevices];

// The current device's scratch address (looked up on the first call on that
// device, with the device current).
static int scratch_of_current_device(void** out, int* device) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    set_error("w8a8_gemm_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return W8A8_ERR_LAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("w8a8_gemm_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return W8A8_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  *device = dev;
  return W8A8_OK;
}

}  // namespace w8a8

extern "C" int w8a8_gemm(const W8A8GemmArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_gemm: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8GemmArgs), "w8a8_gemm: struct_size %u != %zu", a->struct_size,
               sizeof(W8A8GemmArgs));
  return gemm_entry(a, a->workspace, a->workspace_bytes);
}

extern "C" int w8a8_gemm_noalloc(const W8A8GemmArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_gemm_noalloc: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8GemmArgs), "w8a8_gemm_noalloc: struct_size %u != %zu",
               a->struct_size, sizeof(W8A8GemmArgs));
  W8A8_REQUIRE(a->workspace == nullptr && a->workspace_bytes == 0,
               "w8a8_gemm_noalloc: the static scratch replaces the workspace (pass NULL and 0)");
  void* ws = nullptr;
  int dev = 0;
  int rc = scratch_of_current_device(&ws, &dev);
  if (rc != W8A8_OK) return rc;
  // A split whose partials outgrow the scratch runs unsplit (launch_gemm
  // re-plans when the workspace is too small), with the same result.
  return gemm_entry(a, ws, kScratchBytes);
}

extern "C" int64_t w8a8_gemm_workspace_size(int64_t m, int64_t n, int64_t k) {
  using namespace w8a8;
  if (m <= 0 || n <= 0 || k <= 0 || m >= (1LL << 31) || n >= (1LL << 31) || k >= (1LL << 31)) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int64_t bytes = 0;
  gemm_ksplit(m, n, k, dev, &bytes);
  return bytes;
}

extern "C" int w8a8_dequantize(const W8A8DequantArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_dequantize: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8DequantArgs), "w8a8_dequantize: struct_size %u != %zu",
               a->struct_size, sizeof(W8A8DequantArgs));
  W8A8_REQUIRE(a->epilogue == W8A8_EPI_ROW || a->epilogue == W8A8_EPI_COLUMN,
               "w8a8_dequantize: epilogue must be ROW or COLUMN");
  W8A8_REQUIRE(a->m >= 0 && a->n >= 0 && a->m < (1LL << 31) && a->n < (1LL << 31), "w8a8_dequantize: bad shape");
  if (a->m == 0 || a->n == 0) return W8A8_OK;
  int rc = check_epilogue(a->epilogue, a->out_dtype, a->bias_dtype, a->bias, a->residual, a->ldr, a->gate,
                          a->gate_labels, a->ldg, a->n, a->row_scale, a->col_scale, a->col_scale_stride, a->out,
                          a->ldc);
  if (rc != W8A8_OK) return rc;
  W8A8_REQUIRE(a->acc && a->ldacc >= a->n, "w8a8_dequantize: null acc or ldacc < n");
  W8A8_REQUIRE((a->m * ((a->n + 3) / 4) + 255) / 256 < (1LL << 31), "w8a8_dequantize: too large");
  GemmParams p{};
  fill_epilogue(p, a);
  p.ksplit = 1;
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  if (a->epilogue == W8A8_EPI_ROW) launch_dequant_out<kEpiRow>(a->out_dtype, p, a->acc, a->ldacc, s);
  else launch_dequant_out<kEpiColumn>(a->out_dtype, p, a->acc, a->ldacc, s);
  return launch_status("w8a8_dequantize");
}
