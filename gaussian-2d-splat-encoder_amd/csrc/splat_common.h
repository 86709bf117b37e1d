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
constexpr float kLog2e = 1.44269504088896f;
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
constexpr int kFlagUps = 4;      // composite adds the coarse levels' upsampled fields; clamp_min gradient of S_a
constexpr int kFlagWide = 8;     // 8x8 tiles: 16 waves per tile (forward: instead of 4, backward: instead of 1)
constexpr int kFlagLogScale = 16; // binning: `scale` holds raw log-scales, activated by the decode pass
constexpr int kFlagDefer = 32;    // splat_bin: return once everything is queued; splat_bin_finish reads the totals

// Status codes of the C-ABI.
enum Status : int { kOk = 0, kInvalid = 1, kHipError = 2, kUnsupported = 3, kOverflow = 4, kWorkspace = 5,
                    kCapacity = 6, kBudget = 7 };

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

// Scale activation of params.py:18-28, softplus(x) + 1e-4, evaluated as torch evaluates F.softplus(x) + 1e-4
// in fp32 (beta 1, threshold 20: x above the threshold passes through; the constant is added as float 1e-4).
__device__ __forceinline__ float activate_scale(float x) {
  const float sp = x > 20.f ? x : log1pf(expf(x));
  return sp + 1e-4f;
}

// Upstream gradient g of activate_scale(x) -> gradient w.r.t. x, as torch's softplus backward evaluates it:
// x > 20 ? g : g * z / (z + 1) with z = e^x (the + 1e-4 passes g through unchanged).
__device__ __forceinline__ float activate_scale_grad(float g, float x) {
  const float z = expf(x);
  return x > 20.f ? g : g * z / (z + 1.f);
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

__device__ __forceinline__ int wave_sum_i(int v) {
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

// ---------------------------------------------------------------------------------------------- levels
// A render may place splats on several canvases ("levels"): level 0 is the native (H, W) canvas, the
// others are coarser canvases whose fields are bilinearly upsampled onto level 0 (the octave and
// coarse/fine renders of render_triton.py:879-980). Level l is tiled by TILE; its tiles take the global
// tile ids [tbase[l], tbase[l+1]) and its pixels the packed field slots [pbase[l], pbase[l+1]).
constexpr int kMaxLevels = 12;

struct LevelTable {
  int n;
  unsigned mask;   // levels holding at least one pair; kernels skip the others
  int H[kMaxLevels], W[kMaxLevels], ntx[kMaxLevels];
  int tbase[kMaxLevels + 1], pbase[kMaxLevels + 1];
  int rbase[kMaxLevels + 1];   // global tile-row ids: level l's tile rows are [rbase[l], rbase[l + 1])
};

// Splat -> level routing, evaluated in the decode pass.
struct Routing {
  int mode;         // 0 single level, 1 octave by scale, 2 split by index
  int max_oct;      // mode 1
  float rep;        // mode 1: float(min(H, W))
  float inv_base;   // mode 1: fp32 1 / base_texels (a tensor divided by a CPU scalar is a multiply by its reciprocal)
  int n_coarse;     // mode 2: splats [0, n_coarse) are level 1
};

// Level of global tile row r.
__device__ __forceinline__ int level_of_row(const LevelTable& L, int r) {
  int l = 0;
  while (l + 1 < L.n && r >= L.rbase[l + 1]) ++l;
  return l;
}

__device__ __forceinline__ int level_of(const LevelTable& L, int t) {
  int l = 0;
  while (l + 1 < L.n && t >= L.tbase[l + 1]) ++l;
  return l;
}

// Level of packed pixel slot pp.
__device__ __forceinline__ int level_of_slot(const LevelTable& L, int pp) {
  int l = 0;
  while (l + 1 < L.n && pp >= L.pbase[l + 1]) ++l;
  return l;
}

// Bilinear source of output index d when upsampling `in` samples to `out` (torch upsample_bilinear2d with
// align_corners=False: src = max(scale * (d + 0.5) - 0.5, 0) with scale = in / out in fp32). Returns the
// first source index; *p1 is 1 when a second source exists, *l1 the weight of the second (the first gets
// 1 - l1).
__device__ __forceinline__ int bilinear_src(int d, int in, float scale, int* p1, float* l1) {
  const float r = fmaxf(fmaf(scale, (float)d + 0.5f, -0.5f), 0.f);
  const int i = (int)r;
  *p1 = i < in - 1 ? 1 : 0;
  *l1 = r - (float)i;
  return i;
}

}  // namespace splat

extern "C" {
// C-ABI description of the levels of a render (mirrors include/splat_render.h).
typedef struct splat_levels {
  int mode;           // 0 single level (H, W); 1 octave routing; 2 coarse/fine split by index
  int max_octaves;    // mode 1: levels 0..max_octaves, level o on (max(8, H >> o), max(8, W >> o))
  float base_texels;  // mode 1: o = clamp(ceil(log2(max(max(sy, sx) * min(H, W) / base_texels, 1e-6))), 0, max_octaves)
  int n_coarse;       // mode 2: splats [0, n_coarse) render on (coarse_H, coarse_W) as level 1, the rest on (H, W)
  int coarse_H, coarse_W;
} splat_levels;
}

namespace splat {

// Host: level geometry of a render of the (H, W) canvas with tile size TILE. Returns 0 or a status.
inline int make_levels(int H, int W, int TILE, const splat_levels* lv, LevelTable* L, Routing* R) {
  LevelTable t{};
  Routing r{};
  int mode = lv ? lv->mode : 0;
  if (mode == 0) {
    t.n = 1;
    t.H[0] = H; t.W[0] = W;
  } else if (mode == 1) {
    if (lv->max_octaves < 0 || !(lv->base_texels > 0.f)) return 1;
    // Octaves at and past the first whose canvas is clamped to (8, 8) in both dims share that canvas; their
    // fields are summed after the same upsample, so they are one level (routing clamps to it).
    int osat = 0;
    while ((H >> osat) > 8 || (W >> osat) > 8) ++osat;
    t.n = (lv->max_octaves < osat ? lv->max_octaves : osat) + 1;
    if (t.n > kMaxLevels) return 1;
    for (int o = 0; o < t.n; ++o) {
      t.H[o] = (H >> o) > 8 ? (H >> o) : 8;
      t.W[o] = (W >> o) > 8 ? (W >> o) : 8;
    }
    if (t.H[0] != H || t.W[0] != W) return 1;   // octave 0 must be the native canvas (H, W >= 8)
    r.max_oct = t.n - 1;
    r.rep = (float)(H < W ? H : W);
    r.inv_base = 1.0f / lv->base_texels;
  } else if (mode == 2) {
    if (lv->coarse_H < 1 || lv->coarse_W < 1 || lv->n_coarse < 0) return 1;
    t.n = 2;
    t.H[0] = H; t.W[0] = W;
    t.H[1] = lv->coarse_H; t.W[1] = lv->coarse_W;
    r.n_coarse = lv->n_coarse;
  } else {
    return 1;
  }
  r.mode = mode;
  t.mask = (t.n >= 32) ? 0xffffffffu : ((1u << t.n) - 1u);
  t.tbase[0] = 0;
  t.pbase[0] = 0;
  t.rbase[0] = 0;
  for (int l = 0; l < t.n; ++l) {
    t.ntx[l] = (t.W[l] + TILE - 1) / TILE;
    const long long nty = (t.H[l] + TILE - 1) / TILE;
    t.tbase[l + 1] = (int)(t.tbase[l] + (long long)t.ntx[l] * nty);
    t.pbase[l + 1] = (int)(t.pbase[l] + (long long)t.H[l] * t.W[l]);
    t.rbase[l + 1] = (int)(t.rbase[l] + nty);
  }
  *L = t;
  if (R) *R = r;
  return 0;
}

}  // namespace splat
