// Device-side helpers shared by the gfx950 kernels of the W8A8 path.
//
// Every floating-point expression here is meant to compile to separate IEEE
// binary32 operations (the library is built with -ffp-contract=off and
// without fast-math), in the order written: the CPU oracle evaluates the
// same sequence.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w8a8 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- constants
// fp32(1/127) = 0x3C010204 and the 1e-30 scale floor of the row quantizer.
__device__ constexpr float kR127 = 1.0f / 127.0f;
__device__ constexpr float kScaleFloor = 1e-30f;
__device__ constexpr float kInv16 = 1.0f / 16.0f;
// Fast-path bound of quant1 / quant16: |y - rint(y)| below this means the
// reciprocal product y = x * rcp and the IEEE quotient x / s round to the
// same integer. rcp = 1/s is correctly rounded and the product is rounded
// once, so |y - x/s| <= |x/s| (2^-23 + 2^-48) < 2^-16 for |x/s| < 128 (every
// scale here is at least the absmax / 127); a margin of 2^-15 leaves
// |x/s - rint(y)| < 0.5.
__device__ constexpr float kTieGuard = 0.5f - 1.0f / 32768.0f;

// ---------------------------------------------------------- conversions
__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// fp32 -> fp16 of a value that must first exist as a rounded fp32 (e.g. a
// product): the empty asm hides the producer, so the compiler cannot fold
// fptrunc(fmul) into one v_fma_mix that rounds the exact product to fp16.
__device__ __forceinline__ uint16_t f2h_of_f32(float f) {
  __asm__("" : "+v"(f));
  return f2h(f);
}
typedef float v2f __attribute__((ext_vector_type(2)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
// Two fp32 -> fp16 conversions (round to nearest even) in one packed
// instruction, a in the low half; like f2h_of_f32, each operand first exists
// as a rounded fp32 value.
__device__ __forceinline__ uint32_t f2h2_of_f32(float a, float b) {
  __asm__("" : "+v"(a));
  __asm__("" : "+v"(b));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{a, b}, v2h));
}
// Eight fp32 -> fp16 conversions into four packed words (y[2 i] in the low
// half of w[i]), each value first existing as a rounded fp32. One opaque
// step covers all eight, so the compiler may interleave their producers.
__device__ __forceinline__ void f2h8_of_f32(float (&y)[8], uint32_t (&w)[4]) {
  __asm__("" : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]), "+v"(y[6]), "+v"(y[7]));
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{y[2 * i], y[2 * i + 1]}, v2h));
}
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

enum DType { kF16 = 1, kBF16 = 2, kF32 = 3, kI32 = 4, kI8 = 5 };

// Load 16 consecutive elements of type DT starting at p (16-byte aligned).
template <int DT>
__device__ __forceinline__ void load16(const void* p, float (&v)[16]) {
  if constexpr (DT == kF32) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 t = q[i];
      v[4 * i + 0] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
  } else {
    const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint4 t = q[i];
      uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint16_t lo = (uint16_t)(w[j] & 0xffffu), hi = (uint16_t)(w[j] >> 16);
        v[8 * i + 2 * j + 0] = DT == kF16 ? h2f(lo) : bf2f(lo);
        v[8 * i + 2 * j + 1] = DT == kF16 ? h2f(hi) : bf2f(hi);
      }
    }
  }
}

// The 16 elements of load16 in two phases: raw16 issues the loads (the
// 32 or 64 bytes as uint4 words), unpack16 widens them, so a caller can
// have several units' loads in flight before it uses the first.
template <int DT>
__device__ __forceinline__ void raw16(const void* p, uint4 (&r)[4]) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int i = 0; i < (DT == kF32 ? 4 : 2); ++i) r[i] = q[i];
}

template <int DT>
__device__ __forceinline__ void unpack16(const uint4 (&r)[4], float (&v)[16]) {
  if constexpr (DT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[4 * i + 0] = __builtin_bit_cast(float, r[i].x);
      v[4 * i + 1] = __builtin_bit_cast(float, r[i].y);
      v[4 * i + 2] = __builtin_bit_cast(float, r[i].z);
      v[4 * i + 3] = __builtin_bit_cast(float, r[i].w);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t w[4] = {r[i].x, r[i].y, r[i].z, r[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t lo = (uint16_t)(w[j] & 0xffffu), hi = (uint16_t)(w[j] >> 16);
        v[8 * i + 2 * j + 0] = DT == kF16 ? h2f(lo) : bf2f(lo);
        v[8 * i + 2 * j + 1] = DT == kF16 ? h2f(hi) : bf2f(hi);
      }
    }
  }
}

// Round an fp32 value to the storage dtype DT and back (the rotation of a
// 16-bit input returns a 16-bit tensor).
template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == kF16) return h2f(f2h(x));
  else if constexpr (DT == kBF16) return bf2f(f2bf(x));
  else return x;
}

// ------------------------------------------------------------- exponential
// Cephes single-precision exp (Moshier, Cephes Math Library expf.c):
// Cody-Waite reduction with ln2 = C1 + C2, degree-5 minimax polynomial,
// n rounded half to even, inputs clamped to [-104, 89] (beyond which fp32
// exp is 0 / inf), scaled by ldexp. The reduction steps, the Horner steps and
// the final p*z + r are single-rounding fused multiply-adds (n*C1 is exact,
// so the first step equals x - n*C1).
__device__ __forceinline__ float exp_f32(float x) {
  x = fminf(fmaxf(x, -104.0f), 89.0f);
  const float n = rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(-n, 0.693359375f, x);
  r = __builtin_fmaf(-n, -2.12194440e-4f, r);
  const float z = r * r;
  float p = 1.9875691500e-4f;
  p = __builtin_fmaf(p, r, 1.3981999507e-3f);
  p = __builtin_fmaf(p, r, 8.3334519073e-3f);
  p = __builtin_fmaf(p, r, 4.1665795894e-2f);
  p = __builtin_fmaf(p, r, 1.6666665459e-1f);
  p = __builtin_fmaf(p, r, 5.0000001201e-1f);
  const float y = __builtin_fmaf(p, z, r) + 1.0f;
  return ldexpf(y, (int)n);
}

// SwiGLU in FP32: (g / (1 + exp(-g))) * u with IEEE division.
__device__ __forceinline__ float swiglu(float g, float u) {
  const float den = 1.0f + exp_f32(-g);
  const float act = g / den;
  return act * u;
}

// The same for a gate g that is an fp16 value. For -44 < g < 2^16 (finite
// fp16 gates above -44: then 1 <= 1 + exp(-g) < 2^64) the division takes the
// hardware reciprocal r (within 1 ulp of 1/den), the product q = g * r and
// one residual correction q + (g - den * q) * r, each step a single-rounding
// FMA; the reciprocal, the quotient and the residual stay normal, so no
// operand scaling or special-case fix-up is needed. The quotient equals the
// IEEE one for every such gate: an exact rational evaluation of these steps
// over all 52606 nonzero fp16 gates in the range, with r either fp32
// neighbour of 1/den, leaves one gate (g = 2^-23, den = 2 - 2^-23, whose
// quotient lies 2^-48 above a rounding midpoint) that needs r to be the
// correctly rounded reciprocal, and the GPU parity tests run every finite
// fp16 gate through the kernel. Other gates (below -44, inf, NaN) take the
// IEEE division. The range test |g - 32746| < 32790 is exact for fp16 g
// (the difference fits in 24 bits) and false for inf and NaN.
__device__ __forceinline__ float swiglu_fp16_gate(float g, float u) {
  const float den = 1.0f + exp_f32(-g);
  float act;
  if (__builtin_expect(fabsf(g - 32746.0f) < 32790.0f, 1)) {
    const float r = __builtin_amdgcn_rcpf(den);
    const float q = g * r;
    act = __builtin_fmaf(__builtin_fmaf(-den, q, g), r, q);
  } else {
    act = g / den;
  }
  return act * u;
}

// ------------------------------------------------------------- quantizer
// q = clamp(rne(x / s), -128, 127) with the IEEE quotient x / s.
// rcp = 1/s (IEEE). The product x*rcp is within 2^-16 of the quotient for
// |quotient| < 128 (kTieGuard), so away from half-integers both round to the
// same integer; near a half-integer (or for NaN / inf) the exact quotient is
// computed. Beyond |quotient| >= 128 both saturate to the same code (they
// share the sign, and neither can land on the other side of the clamp).
__device__ __forceinline__ int quant1(float x, float s, float rcp) {
  const float y = x * rcp;
  float n = rintf(y);
  if (!(fabsf(y - n) < kTieGuard)) n = rintf(x / s);
  n = fminf(fmaxf(n, -128.0f), 127.0f);
  return (int)n;
}

__device__ __forceinline__ float row_scale_of(float amax) {
  return fmaxf(amax * kR127, kScaleFloor);
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) |
         ((uint32_t)(c & 0xff) << 16) | ((uint32_t)(d & 0xff) << 24);
}

// ------------------------------------------------------------- ConvRot256
// One radix-4 stage of the regular H4 butterfly on four values e0..e3 that
// differ only in the stage's digit: output digit d negates input 3-d, and
// the sum runs ((p + q) + r) + s in input order. e0 + e1 and e0 - e1 are
// shared: a + (-b) is a - b exactly, and ((-e0) + e1) equals -(e0 - e1)
// except for the sign of a zero sum, which no output of the path keeps
// (absmax and the int8 codes map -0 and +0 alike).
__device__ __forceinline__ void h4(float& e0, float& e1, float& e2, float& e3) {
  const float t = e0 + e1;
  const float u = e0 - e1;
  const float o0 = (t + e2) - e3;
  const float o1 = (t - e2) + e3;
  const float o2 = (u + e2) + e3;
  const float o3 = (e2 - u) + e3;
  e0 = o0; e1 = o1; e2 = o2; e3 = o3;
}

// Stages over the two low digits of a 16-element register block v[i]
// (i = 4*d1 + d0): digit d0 (stride 1), then digit d1 (stride 4).
__device__ __forceinline__ void h4_low_digits(float (&v)[16]) {
#pragma unroll
  for (int b = 0; b < 4; ++b) h4(v[4 * b + 0], v[4 * b + 1], v[4 * b + 2], v[4 * b + 3]);
#pragma unroll
  for (int b = 0; b < 4; ++b) h4(v[b + 0], v[b + 4], v[b + 8], v[b + 12]);
}

// Order LDS traffic between the lanes of one wavefront (lanes execute in
// lockstep; this keeps the compiler from moving accesses across).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// LDS layout of the ConvRot256 lane transpose: each 16-lane slot of a
// wavefront owns kRotSlot floats (256 plus a 16-float skew, so the four
// slots of a wavefront start on different banks), a wavefront kRotWave.
// Lane t's row of 16 floats (elements 16t..16t+15 of the group) is stored
// as four 16-byte chunks with chunk i at position i ^ ((t >> 1) & 3): the
// eight lanes of one 128-byte write then cover distinct banks, and the
// transposed reads (16 lanes reading 16 consecutive floats) stay
// conflict-free.
constexpr int kRotSlot = 272;
constexpr int kRotWave = 4 * kRotSlot;

__device__ __forceinline__ float* rot_slot(float* lds, int wave, int lane) {
  return lds + wave * kRotWave + (lane >> 4) * kRotSlot;
}

// ConvRot256 of one 256-element group held by 16 consecutive lanes, lane t
// holding elements 16t..16t+15 in v (natural order). buf is this group's
// slot (rot_slot). On return, if NATURAL, v again holds elements
// 16t..16t+15; otherwise v[j] holds element 16j + t. The 1/16 factor is
// applied last, as in the reference butterfly.
// SIGNS: smask holds the group's 256 sign words, 0 or 0x80000000 per
// element, XORed into the values first: the rotation diag(s) then H, with s
// a +-1 vector (exact: only signs change). A compile-time choice, so kernels
// without signs hold no registers for them.
template <bool NATURAL, bool SIGNS = false>
__device__ __forceinline__ void convrot256_lanes(float (&v)[16], float* buf, int t,
                                                 const uint32_t* smask = nullptr) {
  if constexpr (SIGNS) {
    const uint4* m = reinterpret_cast<const uint4*>(smask + 16 * t);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 w = m[i];
      v[4 * i] = __uint_as_float(__float_as_uint(v[4 * i]) ^ w.x);
      v[4 * i + 1] = __uint_as_float(__float_as_uint(v[4 * i + 1]) ^ w.y);
      v[4 * i + 2] = __uint_as_float(__float_as_uint(v[4 * i + 2]) ^ w.z);
      v[4 * i + 3] = __uint_as_float(__float_as_uint(v[4 * i + 3]) ^ w.w);
    }
  }
  h4_low_digits(v);
  const int sw = (t >> 1) & 3;
  float4* row = reinterpret_cast<float4*>(buf + 16 * t);
#pragma unroll
  for (int i = 0; i < 4; ++i) row[i ^ sw] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  wave_lds_sync();
  // Element 16 j + t sits in lane j's row, chunk (t >> 2) ^ ((j >> 1) & 3),
  // position t & 3: float 16 j + (t ^ (4 * ((j >> 1) & 3))).
  float w[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) w[j] = buf[16 * j + (t ^ (4 * ((j >> 1) & 3)))];
  // w[j] = element 16 j + t: j = 4*d3 + d2; digit d2 (stride 16), then d3.
#pragma unroll
  for (int b = 0; b < 4; ++b) h4(w[4 * b + 0], w[4 * b + 1], w[4 * b + 2], w[4 * b + 3]);
#pragma unroll
  for (int b = 0; b < 4; ++b) h4(w[b + 0], w[b + 4], w[b + 8], w[b + 12]);
#pragma unroll
  for (int j = 0; j < 16; ++j) w[j] = w[j] * kInv16;
  if constexpr (NATURAL) {
    // Each lane writes back exactly the floats it read (the transposed read
    // is a bijection), so no other lane's read can be overtaken.
#pragma unroll
    for (int j = 0; j < 16; ++j) buf[16 * j + (t ^ (4 * ((j >> 1) & 3)))] = w[j];
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 q = row[i ^ sw];
      v[4 * i] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
    }
    wave_lds_sync();
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = w[j];
    wave_lds_sync();
  }
}

// The 16 int8 codes of elements 16t..16t+15 (natural order), packed for one
// 16-byte store.
// rne(x / s) as an fp32 integer value, without the clamp (quant1's rounding).
__device__ __forceinline__ float quant_round(float x, float s, float rcp) {
  const float y = x * rcp;
  float n = rintf(y);
  if (!(fabsf(y - n) < kTieGuard)) n = rintf(x / s);
  return n;
}

// Sixteen quant1 codes packed little-endian. v_cvt_pk_u8_f32 converts
// n + 128 (exact: n is an integer) with saturation to [0, 255] and packs the
// byte, so the clamp to [-128, 127] and the packing take one instruction per
// code and the XOR with 0x80 turns the biased bytes into two's complement.
// NaN converts to 0 (code -128) and +-inf saturate (127 / -128), as quant1's
// clamp gives them.
__device__ __forceinline__ uint4 quant16(const float (&v)[16], float s, float rcp) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t b = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) b = __builtin_amdgcn_cvt_pk_u8_f32(quant_round(v[4 * i + k], s, rcp) + 128.0f, k, b);
    w[i] = b ^ 0x80808080u;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// ------------------------------------------------------------- reductions
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Max over the 16 lanes of an aligned 16-lane segment.
__device__ __forceinline__ float seg16_max(float v) {
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// -------------------------------------------------------------- epilogue
enum Epilogue { kEpiInt32 = 0, kEpiRow = 1, kEpiColumn = 2 };

template <int EPI>
__device__ __forceinline__ float dequant1(int c, float a, float w) {
  const float cf = (float)c;
  if constexpr (EPI == kEpiRow) {
    const float t = cf * a;
    return t * w;
  } else {
    const float s = a * w;
    return cf * s;
  }
}

}  // namespace w8a8
