// ABI bookkeeping: version, argument-struct sizes and the per-thread error
// message.
#include "w8a8_host.h"

#include <string.h>

namespace w8a8 {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace w8a8

static_assert(sizeof(W8A8QuantArgs) == 104, "W8A8QuantArgs layout");
static_assert(sizeof(W8A8SwigluArgs) == 104, "W8A8SwigluArgs layout");
static_assert(sizeof(W8A8GemmArgs) == 192, "W8A8GemmArgs layout");
static_assert(sizeof(W8A8RopeEpilogue) == 48, "W8A8RopeEpilogue layout");
static_assert(sizeof(W8A8DequantArgs) == 144, "W8A8DequantArgs layout");
static_assert(sizeof(W8A8NormArgs) == 152, "W8A8NormArgs layout");
static_assert(sizeof(W8A8RmsRopeArgs) == 104, "W8A8RmsRopeArgs layout");
static_assert(sizeof(W8A8AttnPrepareArgs) == 224, "W8A8AttnPrepareArgs layout");
static_assert(sizeof(W8A8AttentionArgs) == 144, "W8A8AttentionArgs layout");

extern "C" int w8a8_abi_version(void) { return W8A8_ABI_VERSION; }

extern "C" int64_t w8a8_struct_size(int32_t which) {
  switch (which) {
    case 0: return (int64_t)sizeof(W8A8QuantArgs);
    case 1: return (int64_t)sizeof(W8A8SwigluArgs);
    case 2: return (int64_t)sizeof(W8A8GemmArgs);
    case 3: return (int64_t)sizeof(W8A8DequantArgs);
    case 4: return (int64_t)sizeof(W8A8NormArgs);
    case 5: return (int64_t)sizeof(W8A8RmsRopeArgs);
    case 6: return (int64_t)sizeof(W8A8AttnPrepareArgs);
    case 7: return (int64_t)sizeof(W8A8AttentionArgs);
    default: return -1;
  }
}

extern "C" const char* w8a8_last_error(void) { return w8a8::g_last_error; }
