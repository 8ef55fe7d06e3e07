// Shared host/device helpers for libnship (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace nship {

// Thread-local last error (read by nsh_last_error).
void set_error(const std::string& msg);

#define NSH_CHECK(expr)                                                          \
  do {                                                                           \
    hipError_t e_ = (expr);                                                      \
    if (e_ != hipSuccess) {                                                      \
      ::nship::set_error(std::string(#expr) + ": " + hipGetErrorString(e_));     \
      return -1;                                                                 \
    }                                                                            \
  } while (0)

// Check a kernel launch issued just before.
#define NSH_LAUNCHED()                                                           \
  do {                                                                           \
    hipError_t e_ = hipGetLastError();                                           \
    if (e_ != hipSuccess) {                                                      \
      ::nship::set_error(std::string("kernel launch: ") + hipGetErrorString(e_)); \
      return -1;                                                                 \
    }                                                                            \
  } while (0)

constexpr int kWave = 64;

// Activation codes shared with the reference's ns_act2 switch
// (codegen.cpp:1244-1255): 0 id, 1 relu, 2 leaky, 3 sigmoid, 4 tanh,
// 5 silu, 6 gelu.
enum Act : int { kActId = 0, kActRelu, kActLeaky, kActSigmoid, kActTanh, kActSilu, kActGelu, kActGeluMoe };

__device__ __forceinline__ float act_apply(float x, int code) {
  switch (code) {
    case kActRelu: return x > 0.f ? x : 0.f;
    case kActLeaky: return x > 0.f ? x : 0.01f * x;
    case kActSigmoid: return 1.f / (1.f + expf(-x));
    case kActTanh: return tanhf(x);
    case kActSilu: return x / (1.f + expf(-x));
    case kActGelu: return 0.5f * x * (1.f + erff(x / 1.41421356f));
    // the MoE expert's spelling of GELU (codegen.cpp:1937)
    case kActGeluMoe: return 0.5f * x * (1.f + erff(x * 0.7071067811865476f));
    default: return x;
  }
}

// d act / dx at the pre-activation x (codegen.cpp:1305-1315).
__device__ __forceinline__ float act_deriv(float x, int code) {
  switch (code) {
    case kActRelu: return x > 0.f ? 1.f : 0.f;
    case kActLeaky: return x > 0.f ? 1.f : 0.01f;
    case kActSigmoid: { float s = 1.f / (1.f + expf(-x)); return s * (1.f - s); }
    case kActTanh: { float t = tanhf(x); return 1.f - t * t; }
    case kActSilu: { float s = x / (1.f + expf(-x)); return s + x * (1.f - s); }
    case kActGelu: {
      float u = x / 1.41421356f;
      float p = 0.5f * (1.f + erff(u));
      return p + x * expf(-u * u) / 2.50662827f;
    }
    // the MoE expert's spelling (codegen.cpp:1427-1428)
    case kActGeluMoe:
      return 0.5f * (1.f + erff(x * 0.7071067811865476f)) + x * expf(-x * x * 0.5f) * 0.3989422804014327f;
    default: return 1.f;
  }
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Lane exchange inside each 16-lane row of a wave through DPP (no LDS round
// trip).  CTRL: 0xB1 = quad_perm [1,0,3,2] (lane ^ 1), 0x4E = quad_perm
// [2,3,0,1] (lane ^ 2), 0x141 = row_half_mirror (lane i <-> 7 - i in each 8),
// 0x140 = row_mirror (lane i <-> 15 - i).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Sum over each aligned group of 8 lanes; every lane of the group gets the
// same bits (each step adds two equal-valued partials in either order).
__device__ __forceinline__ float group8_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  return v;
}

// Sum over each 16-lane row.
__device__ __forceinline__ float row16_sum(float v) {
  v = group8_sum(v);
  return v + dpp_mov<0x140>(v);
}

// 2^x as the hardware's v_exp_f32 computes it (about 1 ulp; results below
// 2^-126 flush to zero, where exp2f would produce the subnormal).  Used for
// softmax probabilities, whose terms below 2^-126 of the row maximum change
// no sum.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float read_lane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Global-address-space views: loads through a pointer fetched from memory
// (not a kernel argument) otherwise compile to flat accesses, which share
// the LDS wait counter and serialise against every LDS exchange.
typedef float fvec4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) float gfloat;
typedef __attribute__((address_space(1))) fvec4 gfloat4;
__device__ __forceinline__ gfloat* as_global(float* p) { return (gfloat*)p; }
__device__ __forceinline__ const gfloat* as_global(const float* p) { return (const gfloat*)p; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace nship
