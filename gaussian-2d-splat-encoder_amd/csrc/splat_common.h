// Shared definitions of the gfx950 splat renderer: the decoded splat record, constants, the error channel
// of the C-ABI, and wave64 helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace splat {

// Decoded splat record: 16 floats (64 bytes) per splat, written once by the decode pass and gathered by
// splat id from every tile the splat overlaps. Slots:
//   0 gy, 1 gx                 centre (normalised y, x)
//   2 A, 3 B, 4 Cc, 5 D        whitened rotation: u = A*dy + B*dx, v = Cc*dy + D*dx with
//                              A = k*cos/sy, B = k*sin/sy, Cc = -k*sin/sx, D = k*cos/sx, k = kWhiten
//   6 op                       opacity
//   7 log2(op)                 (the forward evaluates op * falloff as exp2(log2(op) - m))
//   8..11 colour               up to kMaxC channels
//   12 sy, 13 sx, 14 cos, 15 sin   activated scale and rotation (backward only)
constexpr int kRec = 16;
constexpr int kMaxC = 4;
enum RecSlot : int {
  R_GY = 0, R_GX = 1, R_A = 2, R_B = 3, R_CC = 4, R_D = 5, R_OP = 6, R_LOP = 7,
  R_COL = 8, R_SY = 12, R_SX = 13, R_COS = 14, R_SIN = 15
};

// sqrt(0.5 * log2(e)): with u, v whitened by this factor, u^2 + v^2 = 0.5 * log2(e) * maha, so the
// falloff exp(-maha / 2) is exp2(-(u^2 + v^2)) on the hardware exp2.
constexpr float kWhiten = 0.849321800288019f;
constexpr float kLn2 = 0.693147180559945f;
// Alpha clamp 1 - 1e-4 rounded to float32 (0.99989998...), as the reference compares in fp32.
constexpr float kClamp = 0.99989998340606689453125f;
constexpr float kAsumMin = 1e-8f;
// Above this op * falloff, 1 - a is evaluated as (1 - op) + op * (1 - falloff) with a series for
// 1 - falloff (see one_minus_alpha): a rounding error of one ulp in the hardware exp2 near 1 would
// otherwise cost up to 6e-4 relative in 1 - a at the clamp, which the odds weight a / (1 - a) and the
// backward's 1 / (1 - a) amplify.
constexpr float kNearOpaque = 0.9f;

// Render mode flags of the C-ABI.
constexpr int kFlagFields = 1;   // write raw partial sums (S_log, S_a, S_ac) instead of the composite
constexpr int kFlagOdds = 2;     // weight colour by the odds a / (1 - a) instead of a

// Status codes of the C-ABI.
enum Status : int { kOk = 0, kInvalid = 1, kHipError = 2, kUnsupported = 3, kOverflow = 4, kWorkspace = 5 };

// Error channel (thread-local last message), defined in capi.hip.
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// Workgroups are dispatched round-robin over the 8 XCDs. Map workgroup `bid` so that each XCD receives
// one contiguous range of [0, n): neighbouring tiles share splats, and a contiguous band per XCD keeps
// those splats' records in that XCD's L2. A bijection on [0, n).
__device__ __forceinline__ int xcd_swizzle(int bid, int n) {
  constexpr int kXcd = 8;
  const int q = n / kXcd, r = n % kXcd;
  const int x = bid % kXcd, l = bid / kXcd;
  return x * q + (x < r ? x : r) + l;
}

__device__ __forceinline__ float hw_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float hw_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float hw_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// 1 - a with a = min(op * 2^-m, 1 - 1e-4), given the plainly rounded value `oma` = 1 - a.
// Where op * 2^-m > kNearOpaque (only possible for m < log2(1/0.9), i.e. x = m ln2 < 0.106), use
// 1 - op * e^-x = (1 - op) + op * (1 - e^-x), both terms non-negative, with 1 - e^-x from its Taylor series
// to x^5 (truncation below 2e-8 relative for x < 0.106). The branch is wave-uniform: every lane of the wave
// must be executing (true in both per-tile loops).
__device__ __forceinline__ float one_minus_alpha(float oma, float fo, float m, float op, float one_m_op) {
  if (__any(fo > kNearOpaque)) {
    const float x = m * kLn2;
    float p = fmaf(x, 1.f / 120.f, -1.f / 24.f);
    p = fmaf(p, x, 1.f / 6.f);
    p = fmaf(p, x, -0.5f);
    p = fmaf(p, x, 1.f);
    const float acc = fmaxf(fmaf(op, p * x, one_m_op), 1.f - kClamp);
    oma = fo > kNearOpaque ? acc : oma;
  }
  return oma;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Inclusive prefix sum across the 64 lanes of a wave.
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    T o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

inline int div_up(long long a, long long b) { return (int)((a + b - 1) / b); }

}  // namespace splat
