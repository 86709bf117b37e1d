// Per-tile compositing on gfx950: forward and backward of the order-independent alpha composite of
// render_triton.py:423-517 (forward) and 602-720 (backward), plus the exact (unculled) path of :58-266.
//
// Forward: one wave64 per TILE x TILE tile (8 x 8 = one pixel per lane). The tile's pair list is walked in
// pair order; the pair's splat id and its decoded record are wave-uniform, so they are read with scalar
// loads into SGPRs and every lane evaluates its own pixel. Per pixel-pair: whitened offsets u, v; falloff
// exp2(-(u^2 + v^2)); a = min(op * falloff, 1 - 1e-4); S_log += log2(1 - a) (scaled by ln 2 once);
// S_a += w; S_ac += w * colour, with w = a or the odds a / (1 - a).
//
// Backward: one wave per tile, lane = pair. The tile's per-pixel upstream terms (dS_log, dS_a, dS_ac)
// are derived once (lane = pixel) into LDS; each lane then walks the tile's pixels for its own pair and
// accumulates the per-pair sums in registers (the per-tile reduction) and stores them at the pair's
// splat-major index. No global atomics: a reduce pass sums each splat's records (contiguous, in a fixed
// order) into its gradients. Deterministic. The sums become parameter gradients by:
//   q    = da * falloff where op * falloff < 1 - 1e-4 (0 on the clamp)      da: render_triton.py:688-697
//   g_op = sum q,   Qu = sum q u,  Qv = sum q v,  Quu = sum q u^2,  Qvv = sum q v^2,  Quv = sum q u v
//   g_sy = 2 ln2 op Quu / sy,  g_sx = 2 ln2 op Qvv / sx
//   gry  = -op Qu / (k sy),    grx  = -op Qv / (k sx)     (k = kWhiten)
//   g_muy = -(cos gry - sin grx),  g_mux = -(sin gry + cos grx)
//   g_theta = -2 ln2 op Quv (sx^2 - sy^2) / (sx sy)
// which is the reference's per-pixel chain rule (:697-710) with the per-splat factors taken out of the sums.
#include <type_traits>

#include <hip/hip_ext.h>

#include "splat_common.h"

namespace splat {

template <int V>
using IC = std::integral_constant<int, V>;

constexpr int kAcc = 16;       // per-splat accumulator stride of the exact path (floats)
constexpr int kPairRecMax = 10;   // per-pair sums record, at most (floats): Q, Qu, Qv, Quu, Qvv, Quv, colour[C]
template <int C>
__host__ __device__ constexpr int pair_rec() { return 6 + C; }   // record stride of C channels
constexpr int kSums = 10;      // sums carried through the reduction

__host__ __device__ constexpr int tile_threads(int tile) { return tile * tile > 64 ? tile * tile : 64; }

// One pixel-pair of the forward: accumulates the colour weight and its colour sums, returns 1 - a for the
// caller's transmittance product. op * falloff = exp2(log2(op) - m) with m = u^2 + v^2.
template <int C, bool ODDS>
__device__ __forceinline__ float fwd_pair(const float* __restrict__ r, float py, float px, float& s_a, float* sc) {
  const float dy = py - r[R_GY], dx = px - r[R_GX];
  const float u = fmaf(r[R_A], dy, r[R_B] * dx);
  const float v = fmaf(r[R_CC], dy, r[R_D] * dx);
  const float fo = hw_exp2(-fmaf(u, u, fmaf(v, v, -r[R_LOP])));
  const float a = fminf(fo, kClamp);
  float oma = 1.f - a;
  if (ODDS) oma = one_minus_alpha(oma, fo, fmaf(u, u, v * v), r[R_OP], 1.f - r[R_OP]);
  const float w = ODDS ? a * hw_rcp(oma) : a;
  s_a += w;
#pragma unroll
  for (int c = 0; c < C; ++c) sc[c] = fmaf(w, r[R_COL + c], sc[c]);
  return oma;
}

// Opacity bound (as float bits; opacities are non-negative, and any other bit pattern compares above it) at or
// below which op * falloff = exp2(log2(op) - m), m >= 0, stays below 0.99988 plus a few ulps, under the alpha
// clamp 1 - 1e-4: a group of pairs whose opacities are all at or below it needs no min().
constexpr unsigned kNoClampOpBits = 0x3f7ff823u;   // 0.99988f

// Orders the LDS writes of a wave before its later reads (and reads before later writes) without a
// workgroup barrier: the waves of a workgroup run loops of different trip counts.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Sum over the 64 lanes of a wave (every lane active), in a fixed order: within each row of 16 lanes by DPP
// (pairs, quads, half-rows, rows: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror; after the
// first two steps every lane of a quad holds the quad's sum, so each mirror adds the other quad or half-row), then
// the four rows' sums read from lanes 0, 16, 32 and 48 as (r0 + r1) + (r2 + r3). No LDS traffic, unlike shuffles.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  const int b = __float_as_int(v);
  return (__int_as_float(__builtin_amdgcn_readlane(b, 0)) + __int_as_float(__builtin_amdgcn_readlane(b, 16))) +
         (__int_as_float(__builtin_amdgcn_readlane(b, 32)) + __int_as_float(__builtin_amdgcn_readlane(b, 48)));
}

// A value every lane of the wave holds, as a wave-uniform (scalar) value.
__device__ __forceinline__ float uniform_f(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

// Whitened offsets (u, v) of the pixel centre (py0, px0) from a splat with centre (gy, gx) and rotation rows
// (A, B), (Cc, D). A tile's pixels add their own offsets from the tile's reference pixel centre (its middle pixel)
// to these, so their rounding error is shared by the whole tile. The float32 differences py0 - gy, px0 - gx are exact wherever the
// two lie within a factor of two (Sterbenz), which holds for every tile a splat reaches away from the canvas'
// first rows and columns (there the values are small and so is their rounding); each product's rounding error is
// recovered exactly by an fma and added back, so the result is within about one ulp of the exact offsets (a
// float64 evaluation rounded once: half an ulp), at a third of the instructions.
__device__ __forceinline__ float2 offsets_at(float py0, float px0, float gy, float gx, float A, float B, float Cc,
                                             float D) {
  const float dy = py0 - gy, dx = px0 - gx;
  const float pu = A * dy, pv = Cc * dy;
  return make_float2(fmaf(B, dx, pu) + fmaf(A, dy, -pu), fmaf(D, dx, pv) + fmaf(Cc, dy, -pv));
}

// One pixel-pair of the per-tile forward: (u0, v0) are the pair's whitened offsets at the tile's reference pixel
// centre, (ly, lx) the lane's pixel centre relative to it, so u = A ly + B lx + u0 and v = Cc ly + D lx + v0.
// t carries the running product of the group's (1 - a) factors.
template <int C, bool ODDS, bool CLAMP>
__device__ __forceinline__ void fwd_tile_pair(const float* __restrict__ r, float2 uv0, float ly, float lx, float& t,
                                              float& s_a, float* sc) {
  const float u = fmaf(r[R_A], ly, fmaf(r[R_B], lx, uv0.x));
  const float v = fmaf(r[R_CC], ly, fmaf(r[R_D], lx, uv0.y));
  const float fo = hw_exp2(-fmaf(u, u, fmaf(v, v, -r[R_LOP])));
  const float a = CLAMP ? fminf(fo, kClamp) : fo;
  float w;
  if (ODDS) {
    const float oma = one_minus_alpha(1.f - a, fo, fmaf(u, u, v * v), r[R_OP], 1.f - r[R_OP]);
    w = a * hw_rcp(oma);
    t *= oma;
  } else {
    w = a;
    t = fmaf(-a, t, t);   // t (1 - a), one rounding
  }
  s_a += w;
#pragma unroll
  for (int c = 0; c < C; ++c) sc[c] = fmaf(w, r[R_COL + c], sc[c]);
}

// Pairs [b0, b1) of one batch (their offsets at the reference pixel in s_uv[0, b1 - b0)), in groups of four:
// ids and records through scalar loads, offsets by LDS broadcast. The (1 - a) factors of eight pairs (two
// groups) are multiplied before one log2: each factor is >= 1e-4, so the product stays >= 1e-32, a normal float.
template <int C, bool ODDS, bool CLAMP>
__device__ __forceinline__ void fwd_group4(const float* __restrict__ rec, const int* __restrict__ gid, int i, int j,
                                           const float2* s_uv, float ly, float lx, float& t, float& s_a, float* sc) {
  const float* r0 = rec + (size_t)gid[i] * kRec;
  const float* r1 = rec + (size_t)gid[i + 1] * kRec;
  const float* r2 = rec + (size_t)gid[i + 2] * kRec;
  const float* r3 = rec + (size_t)gid[i + 3] * kRec;
  fwd_tile_pair<C, ODDS, CLAMP>(r0, s_uv[j], ly, lx, t, s_a, sc);
  fwd_tile_pair<C, ODDS, CLAMP>(r1, s_uv[j + 1], ly, lx, t, s_a, sc);
  fwd_tile_pair<C, ODDS, CLAMP>(r2, s_uv[j + 2], ly, lx, t, s_a, sc);
  fwd_tile_pair<C, ODDS, CLAMP>(r3, s_uv[j + 3], ly, lx, t, s_a, sc);
}

template <int C, bool ODDS, bool CLAMP>
__device__ __forceinline__ void fwd_batch(const float* __restrict__ rec, const int* __restrict__ gid, int b0, int b1,
                                          const float2* s_uv, float ly, float lx, float& sl, float& s_a, float* sc) {
  int i = b0;
  for (; i + 8 <= b1; i += 8) {
    float t = 1.f;
    fwd_group4<C, ODDS, CLAMP>(rec, gid, i, i - b0, s_uv, ly, lx, t, s_a, sc);
    fwd_group4<C, ODDS, CLAMP>(rec, gid, i + 4, i + 4 - b0, s_uv, ly, lx, t, s_a, sc);
    sl += hw_log2(t);
  }
  if (i < b1) {   // at most seven pairs left: one product, one log2
    float t = 1.f;
    if (i + 4 <= b1) {
      fwd_group4<C, ODDS, CLAMP>(rec, gid, i, i - b0, s_uv, ly, lx, t, s_a, sc);
      i += 4;
    }
    for (; i < b1; ++i) fwd_tile_pair<C, ODDS, CLAMP>(rec + (size_t)gid[i] * kRec, s_uv[i - b0], ly, lx, t, s_a, sc);
    sl += hw_log2(t);
  }
}

// Forward sums of one pixel over pairs [i0, i1) of the tile's list, in batches of 64 pairs. At the start of a
// batch lane j computes the offsets (u0, v0) of pair j at the tile's reference pixel centre (py0, px0) into the
// wave's LDS row s_uv, and a ballot tells whether any pair of the batch can reach the alpha clamp; the pixel loop
// then reads the offsets by broadcast while the pairs' ids and records come through scalar loads (SGPR operands).
// The reference pixel is the tile's middle one (inside the canvas), so that its offsets and the pixels' own offsets
// from it stay within about half the pair's whitened span over the tile: their rounding, about one ulp of that
// size, is shared by the tile's pixels (for a splat far smaller than the tile, a span of hundreds, a few 1e-5 of
// its falloff).
// S_log is accumulated in log2 units, one log2 per eight pairs (see fwd_batch).
template <int C, bool ODDS>
__device__ __forceinline__ void fwd_tile_pixel(const float* __restrict__ rec, const int* __restrict__ gid, int i0,
                                               int i1, float py0, float px0, float ly, float lx, float2* s_uv,
                                               int lane, float& sl, float& s_a, float* sc) {
  for (int b0 = i0; b0 < i1; b0 += 64) {
    const int b1 = min(i1, b0 + 64);
    bool clamp = false;
    if (b0 + lane < b1) {
      const float4* r4 = reinterpret_cast<const float4*>(rec) + (size_t)gid[b0 + lane] * 4;
      const float4 r0 = r4[0];   // gy, gx, A, B
      const float4 r1 = r4[1];   // Cc, D, op, log2(op)
      s_uv[lane] = offsets_at(py0, px0, r0.x, r0.y, r0.z, r0.w, r1.x, r1.y);
      clamp = __float_as_uint(r1.z) > kNoClampOpBits;
    }
    const bool any_clamp = __ballot(clamp) != 0;
    wave_lds_sync();
    if (any_clamp)
      fwd_batch<C, ODDS, true>(rec, gid, b0, b1, s_uv, ly, lx, sl, s_a, sc);
    else
      fwd_batch<C, ODDS, false>(rec, gid, b0, b1, s_uv, ly, lx, sl, s_a, sc);
    wave_lds_sync();
  }
}

template <int C>
__device__ __forceinline__ void store_composite(int p, float sl2, float s_a, const float* sc, const float* __restrict__ bg,
                                                float* __restrict__ out, float* __restrict__ Tout,
                                                float* __restrict__ asum_out, float* __restrict__ fg_out) {
  const float T = hw_exp2(sl2);                 // exp(S_log), S_log = sl2 * ln 2
  const float as = fmaxf(s_a, kAsumMin);
  Tout[p] = T;
  asum_out[p] = as;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const float f = sc[c] / as;
    fg_out[(size_t)p * C + c] = f;
    out[(size_t)p * C + c] = (1.f - T) * f + T * bg[c];
  }
}

// Bilinear samples (torch upsample_bilinear2d, align_corners=False) of the coarse levels' packed fields at
// level-0 pixel (yp, xp), added to the running sums in the reference's order (level 1 first).
template <int C>
__device__ __forceinline__ void add_coarse(const LevelTable& L, int yp, int xp, const float* __restrict__ slog,
                                           const float* __restrict__ sa, const float* __restrict__ sac, float& Sl,
                                           float& Sa, float* Sc) {
  for (int l = 1; l < L.n; ++l) {
    if (!((L.mask >> l) & 1)) continue;
    const int Hl = L.H[l], Wl = L.W[l];
    int py1, px1;
    float ly, lx;
    const int y0 = bilinear_src(yp, Hl, (float)Hl / (float)L.H[0], &py1, &ly);
    const int x0 = bilinear_src(xp, Wl, (float)Wl / (float)L.W[0], &px1, &lx);
    const float h0 = 1.f - ly, w0 = 1.f - lx;
    const size_t i00 = (size_t)L.pbase[l] + (size_t)y0 * Wl + x0, i01 = i00 + px1;
    const size_t i10 = i00 + (size_t)py1 * Wl, i11 = i10 + px1;
    Sl += h0 * (w0 * slog[i00] + lx * slog[i01]) + ly * (w0 * slog[i10] + lx * slog[i11]);
    Sa += h0 * (w0 * sa[i00] + lx * sa[i01]) + ly * (w0 * sa[i10] + lx * sa[i11]);
#pragma unroll
    for (int c = 0; c < C; ++c)
      Sc[c] += h0 * (w0 * sac[i00 * C + c] + lx * sac[i01 * C + c]) + ly * (w0 * sac[i10 * C + c] + lx * sac[i11 * C + c]);
  }
}

// A global tile, its level and coordinates.
struct TileAt {
  int t, l, tx, ty, H, W;
};
__device__ __forceinline__ TileAt tile_of(const LevelTable& L, int t, int l) {
  TileAt a;
  a.t = t;
  a.l = l;
  const int lt = a.t - L.tbase[a.l];
  a.ty = lt / L.ntx[a.l];
  a.tx = lt - a.ty * L.ntx[a.l];
  a.H = L.H[a.l];
  a.W = L.W[a.l];
  return a;
}
// Tile of this workgroup in a launch over tiles [tb0, tb0 + ntiles) (XCD-aware order).
__device__ __forceinline__ TileAt tile_at(const LevelTable& L, int tb0, int ntiles) {
  const int t = tb0 + xcd_swizzle(blockIdx.x, ntiles);
  return tile_of(L, t, level_of(L, t));
}

// Work items of a split launch over the coarse levels of a FIELDS render: every tile of level l is split into
// split[l] contiguous chunks of its pair list, one workgroup each (split 0: the level is not in the launch). Item
// i of level l (ibase[l] <= i < ibase[l + 1]) is chunk (i - ibase[l]) % split[l] of tile
// tbase[l] + (i - ibase[l]) / split[l]. Dense coarse levels hold few tiles with long pair lists: spread over
// separate workgroups, their chunks run on every CU instead of the few CUs that one workgroup per tile would
// occupy. In the forward, the chunks of a level with split > 1 write partial sums (partial item
// pibase[l] + i - ibase[l]) that k_fields_combine adds in chunk order (its workgroup c takes the tile
// c - cbase[l] of level l); the backward's per-pair sums need no combine.
struct SplitTable {
  int split[kMaxLevels];
  int ibase[kMaxLevels + 1];
  int pibase[kMaxLevels];
  int cbase[kMaxLevels + 1];
};

// Tile and chunk of work item `item` (returns the tile; *chunk, *nsplit).
__device__ __forceinline__ TileAt split_item(const LevelTable& L, const SplitTable& P, int item, int* chunk,
                                             int* nsplit) {
  int l = 0;
  while (l + 1 < L.n && item >= P.ibase[l + 1]) ++l;
  const int j = item - P.ibase[l];
  const int s = P.split[l];
  *chunk = j % s;
  *nsplit = s;
  return tile_of(L, L.tbase[l] + j / s, l);
}

// Pixel centres (render_triton.py:455-456, (i + 0.5) / size in float32) of a tile: lane j < TILE divides for row j
// and lane TILE + j for column j, one division for the wave, and each lane takes its own row's and column's by
// shuffles; l is the lane's pixel within the tile, (py0, px0) the centre of its reference pixel: the middle one
// (TILE / 2, TILE / 2), or the canvas' last row or column where the tile extends past it.
template <int TILE>
__device__ __forceinline__ void tile_centres(const TileAt& ta, int l, int lane, float& py, float& px, float& py0,
                                             float& px0) {
  static_assert(2 * TILE <= 64, "one lane per row and column");
  const bool row = lane < TILE;
  const int i = row ? ta.ty * TILE + lane : ta.tx * TILE + (lane - TILE);
  const float c = ((float)i + 0.5f) / (float)(row ? ta.H : ta.W);
  py = __shfl(c, (l / TILE) % TILE, 64);
  px = __shfl(c, TILE + l % TILE, 64);
  const int ry = min(TILE / 2, ta.H - 1 - ta.ty * TILE), rx = min(TILE / 2, ta.W - 1 - ta.tx * TILE);
  py0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), ry));
  px0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), TILE + rx));
}

// Forward over the tiles [tb0, tb0 + ntiles) of the level table (levels without pairs are skipped).
// FIELDS: raw sums into the packed per-level fields slog/sa/sac (slot pbase[l] + pixel).
// Composite (level 0): out, T, asum, fg; with UPS the coarse levels' packed fields (inputs slog/sa/sac) are
// upsampled and added first, and `asum` keeps the unclamped S_a (the clamp_min gradient needs it).
// Waves sharing one 8x8 tile in the forward: each composites a contiguous share of the tile's pair list for
// the tile's 64 pixels, and the partial sums are added in wave order through LDS. More waves per tile hide
// the scalar-load latency of the record stream and even out tiles of different lengths.
// 8x8 tiles: 4 waves per tile, or 16 with kFlagWide (few tiles with long pair lists: the coarse levels of an
// octave render, where a launch may hold a few hundred tiles of thousands of pairs each).
template <int TILE, bool WIDE>
__host__ __device__ constexpr int fwd_split() { return TILE == 8 ? (WIDE ? 16 : 4) : 1; }
template <int TILE, int S>
__host__ __device__ constexpr int fwd_threads() { return tile_threads(TILE) * S; }

template <int C, bool FIELDS, bool ODDS, bool UPS, int TILE, int S>
__global__ __launch_bounds__((fwd_threads<TILE, S>())) void k_fwd_cull(
    const float* __restrict__ rec, const int* __restrict__ gid, const int* __restrict__ starts, LevelTable L, int tb0,
    int ntiles, const float* __restrict__ bg, float* __restrict__ out, float* __restrict__ Tout,
    float* __restrict__ asum_out, float* __restrict__ fg_out, float* __restrict__ slog, float* __restrict__ sa,
    float* __restrict__ sac) {
  constexpr int NW = fwd_threads<TILE, S>() / 64;   // waves per workgroup
  __shared__ float2 s_uv[NW][64];
  const TileAt ta = tile_at(L, tb0, ntiles);
  if (!((L.mask >> ta.l) & 1)) return;
  const int lane = (int)(threadIdx.x & 63);
  const int l = S > 1 ? lane : (int)threadIdx.x;
  const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));   // wave-uniform
  const int wv = S > 1 ? wid : 0;
  const int yp = ta.ty * TILE + l / TILE, xp = ta.tx * TILE + l % TILE;
  const bool valid = l < TILE * TILE && yp < ta.H && xp < ta.W;
  float py, px, py0, px0;   // the lane's pixel centre and the tile's reference pixel centre
  tile_centres<TILE>(ta, l, lane, py, px, py0, px0);
  int g0 = starts[ta.t], g1 = starts[ta.t + 1];
  if (S > 1) {
    const int chunk = ((g1 - g0 + S - 1) / S + 3) & ~3;
    g0 = min(g1, g0 + wv * chunk);
    g1 = min(g1, g0 + chunk);
  }
  float sl = 0.f, s_a = 0.f, sc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) sc[c] = 0.f;
  fwd_tile_pixel<C, ODDS>(rec, gid, g0, g1, py0, px0, py - py0, px - px0, s_uv[wid], lane, sl, s_a, sc);
  if (S > 1) {
    __shared__ float s_part[S > 1 ? S - 1 : 1][2 + C][64];
    if (wv > 0) {
      s_part[wv - 1][0][l] = sl;
      s_part[wv - 1][1][l] = s_a;
#pragma unroll
      for (int c = 0; c < C; ++c) s_part[wv - 1][2 + c][l] = sc[c];
    }
    __syncthreads();
    if (wv > 0) return;
#pragma unroll
    for (int w = 0; w < S - 1; ++w) {
      sl += s_part[w][0][l];
      s_a += s_part[w][1][l];
#pragma unroll
      for (int c = 0; c < C; ++c) sc[c] += s_part[w][2 + c][l];
    }
  }
  if (!valid) return;
  const int p = yp * ta.W + xp;
  if (FIELDS) {
    const size_t pp = (size_t)L.pbase[ta.l] + p;
    slog[pp] = sl * kLn2;
    sa[pp] = s_a;
#pragma unroll
    for (int c = 0; c < C; ++c) sac[pp * C + c] = sc[c];
  } else if (UPS) {
    float Sl = sl * kLn2;
    add_coarse<C>(L, yp, xp, slog, sa, sac, Sl, s_a, sc);
    const float T = hw_exp2(Sl * kLog2e);
    const float as = fmaxf(s_a, kAsumMin);
    Tout[p] = T;
    asum_out[p] = s_a;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float f = sc[c] / as;
      fg_out[(size_t)p * C + c] = f;
      out[(size_t)p * C + c] = (1.f - T) * f + T * bg[c];
    }
  } else {
    store_composite<C>(p, sl, s_a, sc, bg, out, Tout, asum_out, fg_out);
  }
}

// Partial sums of a split FIELDS item, [partial item][2 + C][tile_threads(TILE)] floats: S_log in log2 units,
// S_a, S_ac per channel, one slot per thread of the tile's workgroup.
template <int C, int TILE>
__host__ __device__ constexpr int split_part_floats() { return (2 + C) * tile_threads(TILE); }

// FIELDS forward of the split work items of the coarse levels (SplitTable): one workgroup per item, the tile's
// pixels one per thread, over the item's chunk of the tile's pair list (in pair order, as fwd_tile_pixel walks
// it). A level with split 1 writes its fields; otherwise the item writes partial sums for k_fields_combine.
template <int C, bool ODDS, int TILE>
__global__ __launch_bounds__(tile_threads(TILE)) void k_fwd_fields_split(
    const float* __restrict__ rec, const int* __restrict__ gid, const int* __restrict__ starts, LevelTable L,
    SplitTable P, int nitems, float* __restrict__ slog, float* __restrict__ sa, float* __restrict__ sac,
    float* __restrict__ part) {
  constexpr int NT = tile_threads(TILE);
  __shared__ float2 s_uv[NT / 64][64];
  const int item = xcd_swizzle(blockIdx.x, nitems);
  int chunk, nsplit;
  const TileAt ta = split_item(L, P, item, &chunk, &nsplit);
  const int th = (int)threadIdx.x, lane = th & 63;
  const int wid = __builtin_amdgcn_readfirstlane(th >> 6);
  const int yp = ta.ty * TILE + th / TILE, xp = ta.tx * TILE + th % TILE;
  const bool valid = th < TILE * TILE && yp < ta.H && xp < ta.W;
  const float py = ((float)yp + 0.5f) / (float)ta.H;   // render_triton.py:455-456
  const float px = ((float)xp + 0.5f) / (float)ta.W;
  // the reference pixel: the middle one, or the canvas' last row / column where the tile extends past it
  const float py0 = uniform_f(((float)min(ta.ty * TILE + TILE / 2, ta.H - 1) + 0.5f) / (float)ta.H);
  const float px0 = uniform_f(((float)min(ta.tx * TILE + TILE / 2, ta.W - 1) + 0.5f) / (float)ta.W);
  int g0 = starts[ta.t];
  const int g1t = starts[ta.t + 1];
  const int len = ((g1t - g0 + nsplit - 1) / nsplit + 3) & ~3;
  g0 = min(g1t, g0 + chunk * len);
  const int g1 = min(g1t, g0 + len);
  float sl = 0.f, s_a = 0.f, sc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) sc[c] = 0.f;
  fwd_tile_pixel<C, ODDS>(rec, gid, g0, g1, py0, px0, py - py0, px - px0, s_uv[wid], lane, sl, s_a, sc);
  if (nsplit > 1) {
    float* dst = part + (size_t)(P.pibase[ta.l] + item - P.ibase[ta.l]) * split_part_floats<C, TILE>() + th;
    dst[0] = sl;
    dst[NT] = s_a;
#pragma unroll
    for (int c = 0; c < C; ++c) dst[(2 + c) * NT] = sc[c];
    return;
  }
  if (!valid) return;
  const size_t pp = (size_t)L.pbase[ta.l] + (size_t)yp * ta.W + xp;
  slog[pp] = sl * kLn2;
  sa[pp] = s_a;
#pragma unroll
  for (int c = 0; c < C; ++c) sac[pp * C + c] = sc[c];
}

// Fields of the tiles of split levels: workgroup c is tile c - cbase[l] of level l (cbase[l] <= c < cbase[l + 1]);
// thread = pixel, the partial sums of the tile's split[l] chunks added in chunk order (deterministic).
template <int C, int TILE>
__global__ __launch_bounds__(tile_threads(TILE)) void k_fields_combine(LevelTable L, SplitTable P,
                                                                       const float* __restrict__ part,
                                                                       float* __restrict__ slog, float* __restrict__ sa,
                                                                       float* __restrict__ sac) {
  constexpr int NT = tile_threads(TILE);
  const int cidx = blockIdx.x;
  int l = 0;
  while (l + 1 < L.n && cidx >= P.cbase[l + 1]) ++l;
  const int j = cidx - P.cbase[l];
  const TileAt ta = tile_of(L, L.tbase[l] + j, l);
  const int th = (int)threadIdx.x;
  const int yp = ta.ty * TILE + th / TILE, xp = ta.tx * TILE + th % TILE;
  if (!(th < TILE * TILE && yp < ta.H && xp < ta.W)) return;
  const int s = P.split[l];
  const float* src = part + (size_t)(P.pibase[l] + j * s) * split_part_floats<C, TILE>() + th;
  float sl = 0.f, s_a = 0.f, sc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) sc[c] = 0.f;
  for (int k = 0; k < s; ++k, src += split_part_floats<C, TILE>()) {
    sl += src[0];
    s_a += src[NT];
#pragma unroll
    for (int c = 0; c < C; ++c) sc[c] += src[(2 + c) * NT];
  }
  const size_t pp = (size_t)L.pbase[l] + (size_t)yp * ta.W + xp;
  slog[pp] = sl * kLn2;
  sa[pp] = s_a;
#pragma unroll
  for (int c = 0; c < C; ++c) sac[pp * C + c] = sc[c];
}

// Exact path forward (render_triton.py:58-125): 64 pixels per workgroup in flat pixel order, pixel centres
// supplied by the caller (render.py:61-65 linspace), every splat in splat order.
template <int C>
__global__ __launch_bounds__(64) void k_fwd_exact(const float* __restrict__ rec, int N, const float* __restrict__ pyv,
                                                  const float* __restrict__ pxv, int P, const float* __restrict__ bg,
                                                  float* __restrict__ out, float* __restrict__ Tout,
                                                  float* __restrict__ asum_out, float* __restrict__ fg_out) {
  const int p = blockIdx.x * 64 + threadIdx.x;
  const bool valid = p < P;
  const float py = valid ? pyv[p] : 0.f, px = valid ? pxv[p] : 0.f;
  float sl = 0.f, s_a = 0.f, sc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) sc[c] = 0.f;
  for (int g = 0; g < N; ++g) sl += hw_log2(fwd_pair<C, false>(rec + (size_t)g * kRec, py, px, s_a, sc));
  if (valid) store_composite<C>(p, sl, s_a, sc, bg, out, Tout, asum_out, fg_out);
}

// Per-pixel upstream terms of the backward (render_triton.py:640-654). Masked pixels give zeros.
// FIELDS: loaded from the packed fields at slot pp. Composite: derived from T, asum, fg, gout and bg; with
// UPS, `asum` holds the unclamped S_a and dS_a follows torch's clamp_min gradient (0 below 1e-8,
// render_triton.py:976), and the terms are also stored at pixel p of dslog/dsa/dsac for the adjoint of
// the coarse levels' upsample.
template <int C, bool FIELDS, bool UPS>
__device__ __forceinline__ void pixel_upstream(int p, size_t pp, const float* __restrict__ bg,
                                               const float* __restrict__ Tin, const float* __restrict__ asum_in,
                                               const float* __restrict__ fg_in, const float* __restrict__ gout,
                                               float* __restrict__ dslog, float* __restrict__ dsa,
                                               float* __restrict__ dsac, float4& pa, float2& pb, float* bgp) {
  float dl, da, dc[kMaxC] = {0.f, 0.f, 0.f, 0.f};
  if (FIELDS) {
    dl = dslog[pp];
    da = dsa[pp];
#pragma unroll
    for (int c = 0; c < C; ++c) dc[c] = dsac[pp * C + c];
  } else {
    const float T = Tin[p], a_in = asum_in[p];
    const float ras = 1.f / (UPS ? fmaxf(a_in, kAsumMin) : a_in);   // one division for the pixel's terms
    float dTp = 0.f, sfg = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float go = gout[(size_t)p * C + c], f = fg_in[(size_t)p * C + c];
      const float dfg = go * (1.f - T);
      dTp += go * (bg[c] - f);
      sfg += dfg * f;
      dc[c] = dfg * ras;
      bgp[c] += go * T;
    }
    dl = dTp * T;
    da = -sfg * ras;
    if (UPS) {
      if (!(a_in >= kAsumMin)) da = 0.f;
      dslog[p] = dl;
      dsa[p] = da;
#pragma unroll
      for (int c = 0; c < C; ++c) dsac[(size_t)p * C + c] = dc[c];
    }
  }
  pa = make_float4(dl, da, dc[0], dc[1]);
  pb = make_float2(dc[2], dc[3]);
}

// Per-pair sums over pixels, in registers.
template <int C>
struct PairSums {
  float q = 0.f, qu = 0.f, qv = 0.f, quu = 0.f, qvv = 0.f, quv = 0.f, gc[C];
  __device__ PairSums() {
#pragma unroll
    for (int c = 0; c < C; ++c) gc[c] = 0.f;
  }
};

// The backward evaluates 1 - a = 1 - op * f with one fma while op * f <= kNearOpaqueBwd: the rounding of
// the hardware exp2 (about 1 ulp of f) then costs at most ~1.2e-5 of 1 - a, and of the 1 / (1 - a) factors
// of the gradient. Above it (op * f within 1e-2 of 1, at most a few pixels around the centre of a
// near-opaque splat) 1 - a is evaluated as (1 - op) + op (1 - f) with a series for 1 - f.
constexpr float kNearOpaqueBwd = 0.99f;

// Per-pair constants of the backward loop: opacity, the falloff above which op * f > kNearOpaqueBwd, and 1/op.
struct PairOp {
  float op, thr, rop;
};
__device__ __forceinline__ PairOp pair_op(float op) {
  const float rop = hw_rcp(op);
  return {op, kNearOpaqueBwd * rop, rop};
}

// One pixel-pair of the backward from its falloff f (0 for a lane on the clamp) and 1 - a: adds the colour
// terms to gc (as sum w' * dS_ac with w' = w / op; the caller multiplies by op once per pair) and returns
// q = da * falloff, the pixel's weight in the pair's moment sums.
template <int C, bool ODDS>
__device__ __forceinline__ float bwd_q(float f, float oma, const float4& col, const float4& pa, const float2& pb,
                                       float* gc) {
  const float rr = hw_rcp(oma);
  float ct = fmaf(pa.z, col.x, pa.y);   // dS_a + sum_c dS_ac[c] col[c]
  if (C > 1) ct = fmaf(pa.w, col.y, ct);
  if (C > 2) ct = fmaf(pb.x, col.z, ct);
  if (C > 3) ct = fmaf(pb.y, col.w, ct);
  float da, cw;
  if (ODDS) {
    da = fmaf(-pa.x, rr, ct * (rr * rr));
    cw = f * rr;
  } else {
    da = fmaf(-pa.x, rr, ct);
    cw = f;
  }
  gc[0] = fmaf(cw, pa.z, gc[0]);
  if (C > 1) gc[1] = fmaf(cw, pa.w, gc[1]);
  if (C > 2) gc[2] = fmaf(cw, pb.x, gc[2]);
  if (C > 3) gc[3] = fmaf(cw, pb.y, gc[3]);
  return da * f;
}

// Accumulation of one pixel-pair of the backward with its whitened offsets u, v.
template <int C, bool ODDS>
__device__ __forceinline__ void bwd_acc(float u, float v, float f, float oma, const float4& col, const float4& pa,
                                        const float2& pb, PairSums<C>& s) {
  const float q = bwd_q<C, ODDS>(f, oma, col, pa, pb, s.gc);
  const float qu = q * u, qv = q * v;
  s.q += q;
  s.qu += qu;
  s.qv += qv;
  s.quu = fmaf(qu, u, s.quu);
  s.qvv = fmaf(qv, v, s.qvv);
  s.quv = fmaf(qu, v, s.quv);
}

// One pixel-pair where some lane may be near-opaque (per-lane selection, no wave-level branch): 1 - a as in
// one_minus_alpha above kNearOpaqueBwd; a lane on the clamp (a = 1 - 1e-4) has no gradient through the
// falloff (render_triton.py:686, 697), so it adds its colour term here and continues with f = 0.
template <int C, bool ODDS>
__device__ __forceinline__ void bwd_px_near(float u, float v, float m, float f, const PairOp& po, const float4& col,
                                            const float4& pa, const float2& pb, PairSums<C>& s) {
  const float fo = po.op * f;
  float oma = fmaf(-po.op, f, 1.f);
  if (fo > kNearOpaqueBwd) {
    const float x = m * kLn2;
    float p = fmaf(x, 1.f / 120.f, -1.f / 24.f);
    p = fmaf(p, x, 1.f / 6.f);
    p = fmaf(p, x, -0.5f);
    p = fmaf(p, x, 1.f);
    oma = fmaxf(fmaf(po.op, p * x, 1.f - po.op), 1.f - kClamp);
    if (!(fo < kClamp)) {
      const float cw = ODDS ? kClamp * po.rop * hw_rcp(oma) : kClamp * po.rop;   // min(op f, clamp) w / (a op)
      s.gc[0] = fmaf(cw, pa.z, s.gc[0]);
      if (C > 1) s.gc[1] = fmaf(cw, pa.w, s.gc[1]);
      if (C > 2) s.gc[2] = fmaf(cw, pb.x, s.gc[2]);
      if (C > 3) s.gc[3] = fmaf(cw, pb.y, s.gc[3]);
      f = 0.f;
    }
  }
  bwd_acc<C, ODDS>(u, v, f, oma, col, pa, pb, s);
}

// One pixel-pair of the backward, given whitened offsets u, v, with its own wave-uniform choice between the
// one-fma 1 - a and bwd_px_near (every lane of the wave must be executing).
template <int C, bool ODDS>
__device__ __forceinline__ void bwd_px(float u, float v, const PairOp& po, const float4& col, const float4& pa,
                                       const float2& pb, PairSums<C>& s) {
  const float m = fmaf(u, u, v * v);
  const float f = hw_exp2(-m);
  if (__any(f > po.thr))
    bwd_px_near<C, ODDS>(u, v, m, f, po, col, pa, pb, s);
  else
    bwd_acc<C, ODDS>(u, v, f, fmaf(-po.op, f, 1.f), col, pa, pb, s);
}

template <int C>
__device__ __forceinline__ void xor_reduce(PairSums<C>& s, int d) {
  s.q += __shfl_xor(s.q, d, 64);
  s.qu += __shfl_xor(s.qu, d, 64);
  s.qv += __shfl_xor(s.qv, d, 64);
  s.quu += __shfl_xor(s.quu, d, 64);
  s.qvv += __shfl_xor(s.qvv, d, 64);
  s.quv += __shfl_xor(s.quv, d, 64);
#pragma unroll
  for (int c = 0; c < C; ++c) s.gc[c] += __shfl_xor(s.gc[c], d, 64);
}

// Record of splat-major pair q at psum + q * pair_rec<C>() (4-byte aligned); the colour sums get the
// pair's opacity factor here.
template <int C>
__device__ __forceinline__ void store_pair(float* __restrict__ dst, const PairSums<C>& s, float op) {
  dst[0] = s.q; dst[1] = s.qu; dst[2] = s.qv; dst[3] = s.quu; dst[4] = s.qvv; dst[5] = s.quv;
#pragma unroll
  for (int c = 0; c < C; ++c) dst[6 + c] = op * s.gc[c];
}

// Per-splat sums (Q, Qu, Qv, Quu, Qvv, Quv, colour[C]) -> parameter gradients (formulas at the top).
template <int C>
__device__ __forceinline__ void splat_grads(int g, const float* __restrict__ rec, const float* sums,
                                            float* __restrict__ g_mu, float* __restrict__ g_scale,
                                            float* __restrict__ g_theta, float* __restrict__ g_op,
                                            float* __restrict__ g_col, const float* __restrict__ lsc) {
  const float4* r4 = reinterpret_cast<const float4*>(rec) + (size_t)g * 4;
  const float op = r4[1].z;
  const float4 r3 = r4[3];
  const float sy = r3.x, sx = r3.y, cs = r3.z, sn = r3.w;
  const float gry = -op * sums[1] / (kWhiten * sy);
  const float grx = -op * sums[2] / (kWhiten * sx);
  g_mu[2 * g + 0] = -(cs * gry - sn * grx);
  g_mu[2 * g + 1] = -(sn * gry + cs * grx);
  float gsy = 2.f * kLn2 * op * sums[3] / sy;
  float gsx = 2.f * kLn2 * op * sums[4] / sx;
  if (lsc) {   // w.r.t. the raw log-scales: chain through the activation
    const float2 x = reinterpret_cast<const float2*>(lsc)[g];
    gsy = activate_scale_grad(gsy, x.x);
    gsx = activate_scale_grad(gsx, x.y);
  }
  g_scale[2 * g + 0] = gsy;
  g_scale[2 * g + 1] = gsx;
  if (g_theta) g_theta[g] = -2.f * kLn2 * op * sums[5] * ((sx - sy) * (sx + sy) / (sx * sy));
  g_op[g] = sums[0];
#pragma unroll
  for (int c = 0; c < C; ++c) g_col[(size_t)g * C + c] = sums[6 + c];
}

// log2(kNearOpaqueBwd), and a margin on the exponent bound below that covers the rounding of m and of the
// hardware exp2 (op * f > kNearOpaqueBwd needs m < log2(op) - log2(kNearOpaqueBwd); the clamp needs 0.0144
// less than that).
constexpr float kLog2NearOpaqueBwd = -0.014499569695115f;
constexpr float kNearMargin = 1e-3f;

// Whether op * falloff can exceed kNearOpaqueBwd at a pixel centre in the box [y0, y1] x [x0, x1]: with
// m = u^2 + v^2 >= kWhiten^2 (dy^2 + dx^2) / max(sy, sx)^2, a splat centre farther than
// max(sy, sx) sqrt(log2(op / kNearOpaqueBwd)) / kWhiten from the box cannot reach it.
__device__ __forceinline__ bool near_possible(float op, float lop, float gy, float gx, float smax, float y0, float y1,
                                              float x0, float x1) {
  const float dy = fmaxf(fmaxf(y0 - gy, gy - y1), 0.f);
  const float dx = fmaxf(fmaxf(x0 - gx, gx - x1), 0.f);
  const float d2 = fmaf(dy, dy, dx * dx) * (kWhiten * kWhiten);
  return op > kNearOpaqueBwd && d2 < smax * smax * (lop - kLog2NearOpaqueBwd + kNearMargin);
}

// Geometry of one pair in the backward's lane-per-pair loops: the splat centre (gy, gx) and the rotation rows
// (A, B) and (Cc, D), so that at the pixel centre (py, px) u = A (py - gy) + B (px - gx) and
// v = Cc (py - gy) + D (px - gx). The offsets py - gy and px - gx are float32 differences of absolute
// coordinates, exact where the pixel lies near the splat (Sterbenz), so u and v carry a rounding error relative
// to their own terms there. Offsets taken from any other reference point (the tile's first pixel centre, its
// centre) would carry that point's rounding times the whitening factor, about 2,000 per unit of the canvas for
// a splat of a third of a pixel: 1e-4 of u^2 at the few pixels of such a splat.
struct PairGeo {
  float gy, gx, A, B, Cc, D;
};

__device__ __forceinline__ PairGeo pair_geo(const float4& r0, const float4& r1) {
  return {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y};
}

// A lane whose pair was taken out: a centre at 1e30 with u = -(py - gy) = 1e30 at every pixel, so u^2
// overflows, the falloff is 0, 1 - a = 1 and every sum of the lane stays 0 (no product of 0 and infinity:
// u stays finite).
__device__ __forceinline__ void mute_pair(bool mute, PairGeo& g) {
  if (mute) {
    g.gy = 1e30f;
    g.A = 1.f;
    g.B = g.Cc = g.D = 0.f;
  }
}

// The tile's per-pixel upstream terms in LDS, row by row: TILE float4 (dS_log, dS_a, dS_ac[0], dS_ac[1]), the row's
// pixel centre (one float4 slot, in .x), then TILE float2 (dS_ac[2], dS_ac[3]). A row's reads take one base address
// and immediate offsets. Rows are 6 TILE + 4 words (52 for 8 x 8 tiles, a multiple of four words for the 16-byte
// reads), so the rows that different lanes read at once (row-split remainder chunks) start on different banks.
template <int TILE>
struct UpRows {
  static constexpr int RF = 6 * TILE + 4;   // floats per row
  static_assert(RF % 4 == 0, "rows start 16-byte aligned (float4 reads)");
  static_assert((4 * TILE + 4) % 2 == 0, "the float2 part starts 8-byte aligned");
  float* base;
  __device__ __forceinline__ const float* row(int yy) const { return base + yy * RF; }
  __device__ __forceinline__ static float4 pa(const float* r, int xx) {
    return *reinterpret_cast<const float4*>(r + 4 * xx);
  }
  template <int C>
  __device__ __forceinline__ static float2 pb(const float* r, int xx) {
    return C > 2 ? *reinterpret_cast<const float2*>(r + 4 * TILE + 4 + 2 * xx) : make_float2(0.f, 0.f);
  }
  __device__ __forceinline__ static float py(const float* r) { return r[4 * TILE]; }
  __device__ __forceinline__ void put(int yy, int xx, const float4& a, const float2& b) const {
    float* r = base + yy * RF;
    *reinterpret_cast<float4*>(r + 4 * xx) = a;
    *reinterpret_cast<float2*>(r + 4 * TILE + 4 + 2 * xx) = b;
  }
};

// The tile's pixel centres (render_triton.py:455-456): the first and last row and column (py0, py1, px0, px1),
// the half extents cy = (py1 - py0) / 2, cx = (px1 - px0) / 2, and every column's centre as a wave-uniform
// value; the rows' centres are in LDS.
template <int TILE>
struct TileCentres {
  float py0, py1, px0, px1, cy, cx;
  float pxa[TILE];
};

// Pairs whose falloff stays below 2^-kCullLog2 (about 1e-9) of the splat's own falloff at each of the 3 x 3 pixel
// centres around the one nearest its centre, at every pixel centre of the tile, add nothing the backward keeps:
// their sums would change the splat's gradients by about 1e-9 of their size. They get a zero record and no lanes
// of the row loops. The bound is relative to the splat's own pixels: a splat far smaller than a pixel whose
// centre lies between pixel centres may reach only 2^-20 at its best pixel, and an absolute cut at 2^-30 would drop
// tiles worth 1e-3 of its scale gradient (sum q u^2 weighs its far pixels by u^2). It takes in the ring around the
// nearest centre because a splat far thinner than a pixel has its moments across the thin axis (sum q v^2 with v
// along it) from that ring alone: v vanishes at a centre on its axis, and the ring's falloff can be 2^-31 of the
// centre's (a 0.15 px sigma one pixel away), so a cut relative to the nearest centre alone dropped half of such a
// moment where the splat's axis fell on a tile edge. The test is on the falloff alone, not on
// op * falloff: the opacity gradient sum da * falloff (render_triton.py:698) carries no opacity factor, so a
// near-transparent splat's far tiles weigh as much in it as an opaque one's. At the 768 x 768 benchmark about a
// tenth of the pairs qualify, mostly elongated splats' tiles across their narrow axis. The test is a lower bound
// of m = u^2 + v^2 over the box of the tile's pixel centres: u and v are linear in the pixel offsets, so over
// the box each lies in an interval given by the corners, and m >= dist(0, u-interval)^2 + dist(0, v-interval)^2.
constexpr float kCullLog2 = 30.f;

// An upper bound of m = u^2 + v^2 of a splat over the 3 x 3 pixel centres around the centre of the canvas pixel that
// holds its centre (clamped to the canvas of H x W pixels, rH = 1 / H, rW = 1 / W): u and v at that centre plus
// their largest change over one pixel step in y and in x (the centre position need not be the exact float32 pixel
// centre for a cut, and the bound may take in centres past the canvas' edge: it only keeps more pairs).
__device__ __forceinline__ float ring_pixel_m(float gy, float gx, float A, float B, float Cc, float D, float fH,
                                              float fW, float rH, float rW) {
  const float ny = fmaf(__builtin_amdgcn_fmed3f(floorf(gy * fH), 0.f, fH - 1.f) + 0.5f, rH, -gy);
  const float nx = fmaf(__builtin_amdgcn_fmed3f(floorf(gx * fW), 0.f, fW - 1.f) + 0.5f, rW, -gx);
  const float u = fabsf(fmaf(A, ny, B * nx)) + fmaf(fabsf(A), rH, fabsf(B) * rW);
  const float v = fabsf(fmaf(Cc, ny, D * nx)) + fmaf(fabsf(Cc), rH, fabsf(D) * rW);
  return fmaf(u, u, v * v);
}

// Lower bound of u^2 + v^2 over the box of the tile's pixel centres, from u, v at the box's middle (uc, vc) and
// their half-spans over the box (su, sv): u and v are affine in the pixel position, so over the box u lies in
// [uc - su, uc + su] and v in [vc - sv, vc + sv].
__device__ __forceinline__ float box_min_m(float uc, float vc, float su, float sv) {
  const float du = fmaxf(fabsf(uc) - su, 0.f), dv = fmaxf(fabsf(vc) - sv, 0.f);
  return fmaf(du, du, dv * dv);
}

// Two forms of the per-pair sums over whole rows of the tile (lane = pair):
//  * direct: per pixel u and v from the offsets to the splat centre (one fma each from the row terms) and the
//    five moments of q in (u, v), eight operations;
//  * moments: offsets (ly', lx') from the pair's own centre, the splat centre clamped into the box of the
//    tile's pixel centres (both exact float32 differences of absolute coordinates); per pixel m = u^2 + v^2
//    as a quadratic in lx' with per-row coefficients (no u or v) and three row sums (q, q lx', q lx'^2); each
//    row folds its sums into the six moments of q in (ly', lx'), which map onto sum q u, ..., sum q u v once
//    per pair since u, v are linear in (ly', lx'). Four fewer operations per pixel.
// The moment form evaluates sum q u^2 as up^2 sum q + 2 up sum q du + sum q du^2 (up = u at the pair's
// centre, du = u - up): the terms cancel where q sits away from that centre, and the rounding error grows
// with the pair's whitened span over the tile, max |du|. In a float32 emulation of the form (random pair
// geometries, spans up to 8, 8x8 tiles, signed upstream) each sum's error stays below 1.2e-5 of the sum of its
// terms' magnitudes; the GPU tests hold every splat's gradients to 1e-4 of their own term magnitudes across this
// limit. Pairs with a span above kMomentSpan take the direct form, and so do those of very elongated splats with
// a span above kElongSpan (moment_form_ok).
constexpr float kMomentSpan = 8.f;

// Half-spans of u and v over the box of the tile's pixel centres (half extents cy, cx) for the rotation rows
// (A, B), (Cc, D).
template <int TILE>
__device__ __forceinline__ float2 half_spans(float A, float B, float Cc, float D, const TileCentres<TILE>& tc) {
  return make_float2(fmaf(fabsf(A), tc.cy, fabsf(B) * tc.cx), fmaf(fabsf(Cc), tc.cy, fabsf(D) * tc.cx));
}

// Whether a pair takes the moment form, from its half-spans hs and the splat's scales sc = (sy, sx): a span at most
// kMomentSpan, and at most kElongSpan for a splat more elongated than kElongAspect. Along an elongated splat's long
// axis a pair's q sits where u (or v) nearly vanishes while the tile spans large values of it: sum q u^2 is then a
// small difference of the mapped moments' terms (A^2 sum q ly'^2, 2 A B sum q lx' ly', B^2 sum q lx'^2), and a
// randomized sweep found a splat of aspect 139 whose pairs at spans 6 to 8 missed the per-splat bar by 4.6e-4 of its
// scale gradient.
constexpr float kElongSpan = 4.f;
constexpr float kElongAspect = 16.f;
__device__ __forceinline__ bool moment_form_ok(float2 hs, float2 sc) {
  const float span = fmaxf(hs.x, hs.y);
  return span <= kMomentSpan && (span <= kElongSpan || fmaxf(sc.x, sc.y) <= kElongAspect * fminf(sc.x, sc.y));
}

// Geometry of one pair in the direct form: the splat centre, the rotation (cs, sn) and the whitening factors
// ky = k / sy, kx = k / sx (the decode pass's own values), so that u = ky (cs dy + sn dx) and
// v = kx (cs dx - sn dy). The rotated offsets are formed before the scaling, each as one rounding of the exact
// sum (the row's product and its rounding error, by fma): an elongated rotated splat's narrow-axis offset is a
// small difference of two large products along its long axis, and the whitened rows (A, B), (Cc, D) of the
// moment form would add their own roundings to it (at an aspect ratio of 100, 1e-4 of its rotation gradient).
// This is the order in which the reference rotates (render_triton.py:476-480), with fewer roundings.
struct DirectGeo {
  float gy, gx, cs, sn, ky, kx;
};

__device__ __forceinline__ DirectGeo direct_geo(const float4& r0, const float4& r3) {
  return {r0.x, r0.y, r3.z, r3.w, kWhiten / r3.x, kWhiten / r3.y};
}

// A lane whose pair was taken out of the direct form (see mute_pair).
__device__ __forceinline__ void mute_direct(bool mute, DirectGeo& g) {
  if (mute) {
    g.gy = 1e30f;
    g.cs = g.ky = 1.f;
    g.sn = g.kx = 0.f;
  }
}

// The row terms of u and v at a row offset dy: cs dy and -sn dy with their rounding errors.
struct RowTerms {
  float au, eu, av, ev;
};
__device__ __forceinline__ RowTerms row_terms(const DirectGeo& g, float dy) {
  RowTerms t;
  t.au = g.cs * dy;
  t.eu = fmaf(g.cs, dy, -t.au);
  t.av = -g.sn * dy;
  t.ev = fmaf(-g.sn, dy, -t.av);
  return t;
}

// Whitened offsets (u, v) at column offset dx of a row.
__device__ __forceinline__ float2 direct_uv(const DirectGeo& g, const RowTerms& t, float dx) {
  return make_float2(g.ky * (fmaf(g.sn, dx, t.au) + t.eu), g.kx * (fmaf(g.cs, dx, t.av) + t.ev));
}

// Direct form over rows [row0, row0 + nrows), with 1 - a = 1 - op f by one fma: the caller has taken every
// pair that may be near-opaque in the tile (near_possible) out of the wave's lanes.
template <int C, bool ODDS, int TILE>
__device__ __forceinline__ void pair_rows_direct(const DirectGeo& g, float op, const float4& col, int row0, int nrows,
                                                 const UpRows<TILE>& ups, const TileCentres<TILE>& tc, PairSums<C>& s) {
  float dx[TILE];   // the columns' offsets from the splat centre, once per pair
#pragma unroll
  for (int xx = 0; xx < TILE; ++xx) dx[xx] = tc.pxa[xx] - g.gx;
#pragma nounroll
  for (int yy = row0; yy < row0 + nrows; ++yy) {
    const float* r = ups.row(yy);
    const RowTerms rt = row_terms(g, UpRows<TILE>::py(r) - g.gy);
#pragma unroll
    for (int xx = 0; xx < TILE; ++xx) {
      const float4 pa = UpRows<TILE>::pa(r, xx);
      const float2 pb = UpRows<TILE>::template pb<C>(r, xx);
      const float2 uv = direct_uv(g, rt, dx[xx]);
      const float u = uv.x, v = uv.y;
      const float f = hw_exp2(-fmaf(u, u, v * v));
      bwd_acc<C, ODDS>(u, v, f, fmaf(-op, f, 1.f), col, pa, pb, s);
    }
  }
}

// Moment form over rows [row0, row0 + nrows) (nrows >= 1) for pairs with moment_form_ok (and not near-opaque), into
// a fresh s (its six moment sums are set here, its colour sums accumulate from zero). FULL: every row of the tile
// (row0 = 0, nrows = TILE), one row at a time for the whole wave, so the row index and the loop's bookkeeping stay
// in scalar registers. The first row is peeled: it sets the running sums instead of adding to zeros.
template <int C, bool ODDS, int TILE, bool FULL>
__device__ __forceinline__ void pair_rows_moments(const PairGeo& g, float op, const float4& col, int row0, int nrows,
                                                  const UpRows<TILE>& ups, const TileCentres<TILE>& tc, PairSums<C>& s) {
  // the pair's centre (ey, ex): the splat centre clamped into the box of the tile's pixel centres; u, v there
  const float ey = __builtin_amdgcn_fmed3f(g.gy, tc.py0, tc.py1), ex = __builtin_amdgcn_fmed3f(g.gx, tc.px0, tc.px1);
  const float eyg = ey - g.gy, exg = ex - g.gx;
  const float up = fmaf(g.A, eyg, g.B * exg);
  const float vp = fmaf(g.Cc, eyg, g.D * exg);
  // along a row, u = uy + B lx' and v = vy + D lx', so m = (uy^2 + vy^2) + 2 (uy B + vy D) lx' + (B^2 + D^2) lx'^2
  const float a2 = fmaf(g.B, g.B, g.D * g.D), b2 = 2.f * g.B, d2 = 2.f * g.D;
  float lxp[TILE];   // the column offsets lx', once per pair
#pragma unroll
  for (int xx = 0; xx < TILE; ++xx) lxp[xx] = tc.pxa[xx] - ex;
  // sum q {1, ly', ly'^2, lx' ly'} by rows; sum q {lx', lx'^2} from the column sums cq of q after the rows
  float m0, my, myy, mxy, cq[TILE];
  auto row = [&](int yy, auto first) {
    constexpr bool FIRST = decltype(first)::value != 0;
    const float* r = ups.row(yy);
    const float ly = UpRows<TILE>::py(r) - ey;
    const float uy = fmaf(g.A, ly, up), vy = fmaf(g.Cc, ly, vp);
    const float a0 = fmaf(uy, uy, vy * vy), a1 = fmaf(uy, b2, vy * d2);
    float r0 = 0.f, r1 = 0.f;
#pragma unroll
    for (int xx = 0; xx < TILE; ++xx) {
      const float4 pa = UpRows<TILE>::pa(r, xx);
      const float2 pb = UpRows<TILE>::template pb<C>(r, xx);
      const float lx = lxp[xx];
      const float f = hw_exp2(-fmaf(fmaf(a2, lx, a1), lx, a0));
      const float q = bwd_q<C, ODDS>(f, fmaf(-op, f, 1.f), col, pa, pb, s.gc);
      r0 += q;
      cq[xx] = FIRST ? q : cq[xx] + q;
      r1 = fmaf(q, lx, r1);
    }
    if (FIRST) {
      m0 = r0;
      my = ly * r0;
      myy = (ly * ly) * r0;
      mxy = ly * r1;
    } else {
      m0 += r0;
      my = fmaf(ly, r0, my);
      myy = fmaf(ly * ly, r0, myy);
      mxy = fmaf(ly, r1, mxy);
    }
  };
  row(row0, IC<1>{});
  if constexpr (FULL) {
#pragma nounroll
    for (int yy = 1; yy < TILE; ++yy) row(yy, IC<0>{});
  } else {
#pragma nounroll
    for (int yy = row0 + 1; yy < row0 + nrows; ++yy) row(yy, IC<0>{});
  }
  float mx = 0.f, mxx = 0.f;
#pragma unroll
  for (int xx = 0; xx < TILE; ++xx) {
    const float t = cq[xx] * lxp[xx];
    mx += t;
    mxx = fmaf(t, lxp[xx], mxx);
  }
  // with du = u - up = A ly' + B lx' and dv = v - vp = Cc ly' + D lx':
  const float su = fmaf(g.A, my, g.B * mx);                                   // sum q du
  const float sv = fmaf(g.Cc, my, g.D * mx);                                  // sum q dv
  const float suu = fmaf(g.A * g.A, myy, fmaf(2.f * g.A * g.B, mxy, g.B * g.B * mxx));
  const float svv = fmaf(g.Cc * g.Cc, myy, fmaf(2.f * g.Cc * g.D, mxy, g.D * g.D * mxx));
  const float suv = fmaf(g.A * g.Cc, myy, fmaf(fmaf(g.A, g.D, g.B * g.Cc), mxy, g.B * g.D * mxx));
  s.q = m0;
  s.qu = fmaf(up, m0, su);
  s.qv = fmaf(vp, m0, sv);
  s.quu = fmaf(up, fmaf(up, m0, 2.f * su), suu);
  s.qvv = fmaf(vp, fmaf(vp, m0, 2.f * sv), svv);
  s.quv = fmaf(up, fmaf(vp, m0, sv), fmaf(vp, su, suv));
}

// Per-pair sums over the pixels [j0, j0 + npx) of one row of the tile (lane = pair, lane-varying j0): the
// remainder chunks that give a pair fewer pixels than a row.
template <int C, bool ODDS, int TILE>
__device__ __forceinline__ void pair_row_part(const DirectGeo& g, float op, const float4& col, int j0, int npx,
                                              const UpRows<TILE>& ups, const float* s_pxa, PairSums<C>& s) {
  const int yy = j0 / TILE;
  const float* r = ups.row(yy);
  const RowTerms rt = row_terms(g, UpRows<TILE>::py(r) - g.gy);
  for (int l = j0; l < j0 + npx; ++l) {
    const int xx = l - yy * TILE;
    const float2 uv = direct_uv(g, rt, s_pxa[xx] - g.gx);
    const float u = uv.x, v = uv.y;
    const float f = hw_exp2(-fmaf(u, u, v * v));
    bwd_acc<C, ODDS>(u, v, f, fmaf(-op, f, 1.f), col, UpRows<TILE>::pa(r, xx), UpRows<TILE>::template pb<C>(r, xx),
                     s);
  }
}

// Sums of pair g (wave-uniform) over the tile's pixels with lane = pixel and 1 - a evaluated carefully at
// every pixel (bwd_px_near), reduced over the wave: every lane returns the totals. For the pairs taken out
// of the lane-per-pair loops (a few near-opaque splats around their centre tile, and splats far smaller than
// the tile).
template <int C, bool ODDS, int TILE>
__device__ __forceinline__ PairSums<C> careful_pair(const float* __restrict__ rec, int g, const UpRows<TILE>& ups,
                                                    const float* s_pxa, int lane, float& op) {
  const float4* r4 = reinterpret_cast<const float4*>(rec) + (size_t)g * 4;
  const float4 r0 = r4[0], r1 = r4[1], col = r4[2];
  const DirectGeo dg = direct_geo(r0, r4[3]);
  const PairOp po = pair_op(r1.z);
  op = r1.z;
  PairSums<C> s;
  for (int l = lane; l < TILE * TILE; l += 64) {
    const int yy = l / TILE, xx = l % TILE;
    const float* r = ups.row(yy);
    const float2 uv = direct_uv(dg, row_terms(dg, UpRows<TILE>::py(r) - dg.gy), s_pxa[xx] - dg.gx);
    const float u = uv.x, v = uv.y;
    const float m = fmaf(u, u, v * v);
    bwd_px_near<C, ODDS>(u, v, m, hw_exp2(-m), po, col, UpRows<TILE>::pa(r, xx), UpRows<TILE>::template pb<C>(r, xx),
                         s);
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) xor_reduce<C>(s, d);
  return s;
}

// Backward over the tiles [tb0, tb0 + ntiles) of the level table (levels without pairs are skipped).
// Composite (level 0): upstream from T/asum/fg/gout (see pixel_upstream for UPS); per-tile partials of
// sum_p gout * T go to bg_part[c * ntiles + (t - tb0)]. FIELDS: upstream from the packed fields.
// S waves per tile (S = 1, or 16 with kFlagWide for few tiles with long pair lists: the dense coarse levels of
// an octave render): the per-pixel upstream terms are staged in LDS once for the tile, then each wave takes a
// contiguous share of the tile's pair list (every pair's sums are independent) 64 at a time (lane = pair) in
// the moment form, the pairs that need the direct form in passes of their own.
// The last r < 64 pairs of a pass get L lanes each (the largest power of two with r L <= 64), each lane
// covering a 1/L share of the tile's pixels (whole rows when that share is at least a row) and the L partial
// sums are combined with xor shuffles. At 5 waves per SIMD (at most 96 VGPRs, no spills) there are enough waves
// to cover the latency of the VALU, LDS and transcendental pipes.
// SPLIT (FIELDS only, S = 1): workgroup = a work item of the SplitTable, the item's chunk of its tile's pairs.
template <int C, bool FIELDS, bool ODDS, bool UPS, int TILE, int S, bool SPLIT = false>
__global__ __launch_bounds__(64 * S) __attribute__((amdgpu_waves_per_eu(5))) void k_bwd_cull(
    const float* __restrict__ rec, const int* __restrict__ gid, const int* __restrict__ starts, LevelTable L, int tb0,
    int ntiles, const float* __restrict__ bg, const float* __restrict__ Tin, const float* __restrict__ asum_in,
    const float* __restrict__ fg_in, const float* __restrict__ gout, float* __restrict__ dslog,
    float* __restrict__ dsa, float* __restrict__ dsac, const int* __restrict__ pair_q, float* __restrict__ psum,
    float* __restrict__ bg_part, SplitTable P) {
  static_assert(!SPLIT || (FIELDS && S == 1), "split items: FIELDS backward, one wave per item");
  constexpr int NP = TILE * TILE;
  __shared__ float4 s_up4[TILE * UpRows<TILE>::RF / 4];
  const UpRows<TILE> ups{reinterpret_cast<float*>(s_up4)};
  __shared__ float s_pya[TILE], s_pxa[TILE];
  __shared__ int s_defer_w[S][128], s_mi_w[S][128];
  int chunk = 0, nsplit = 1;
  const TileAt ta = SPLIT ? split_item(L, P, xcd_swizzle(blockIdx.x, ntiles), &chunk, &nsplit) : tile_at(L, tb0, ntiles);
  if (!((L.mask >> ta.l) & 1)) return;
  const int t = ta.t;
  const int lane = threadIdx.x & 63;
  const int wid = S > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;   // wave-uniform
  int* s_defer = s_defer_w[wid];
  int* s_mi = s_mi_w[wid];
  float bgp[kMaxC] = {0.f, 0.f, 0.f, 0.f};
  for (int l = (int)threadIdx.x; l < NP; l += 64 * S) {
    const int yp = ta.ty * TILE + l / TILE, xp = ta.tx * TILE + l % TILE;
    float4 pa = make_float4(0.f, 0.f, 0.f, 0.f);
    float2 pb = make_float2(0.f, 0.f);
    if (yp < ta.H && xp < ta.W) {
      const int p = yp * ta.W + xp;
      pixel_upstream<C, FIELDS, UPS>(p, (size_t)L.pbase[ta.l] + p, bg, Tin, asum_in, fg_in, gout, dslog, dsa, dsac,
                                     pa, pb, bgp);
    }
    ups.put(l / TILE, l % TILE, pa, pb);
  }
  if (!FIELDS && bg_part) {   // the tile's partial sums, waves added in wave order
    __shared__ float s_bgw[S][kMaxC];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float v = wave_sum_dpp(bgp[c]);
      if (lane == 0) s_bgw[wid][c] = v;
    }
    __syncthreads();
    if (threadIdx.x < C) {
      float v = 0.f;
      for (int w = 0; w < S; ++w) v += s_bgw[w][threadIdx.x];
      bg_part[(size_t)threadIdx.x * ntiles + (t - tb0)] = v;
    }
  }
  // the tile's pixel centres (render_triton.py:455-456): rows and columns in LDS, columns also wave-uniform
  const float fH = (float)ta.H, fW = (float)ta.W;
  if (threadIdx.x < TILE) {
    const float pyc = ((float)(ta.ty * TILE + lane) + 0.5f) / fH;
    s_pya[lane] = pyc;
    ups.base[lane * UpRows<TILE>::RF + 4 * TILE] = pyc;
    s_pxa[lane] = ((float)(ta.tx * TILE + lane) + 0.5f) / fW;
  }
  __syncthreads();
  TileCentres<TILE> tc;
  tc.py0 = uniform_f(s_pya[0]);
  tc.py1 = uniform_f(s_pya[TILE - 1]);
  tc.px0 = uniform_f(s_pxa[0]);
  tc.px1 = uniform_f(s_pxa[TILE - 1]);
  tc.cy = 0.5f * (tc.py1 - tc.py0);
  tc.cx = 0.5f * (tc.px1 - tc.px0);
#pragma unroll
  for (int xx = 0; xx < TILE; ++xx) tc.pxa[xx] = uniform_f(s_pxa[xx]);
  const float py0 = tc.py0, px0 = tc.px0, py1 = tc.py1, px1 = tc.px1;
  const float pym = py0 + tc.cy, pxm = px0 + tc.cx;   // the middle of the box of the tile's pixel centres
  const float rH = uniform_f(hw_rcp(fH)), rW = uniform_f(hw_rcp(fW));   // for ring_pixel_m's bound only
  int g0 = starts[t], g1 = starts[t + 1];
  if (SPLIT) {   // the item's chunk: whole passes of 64 pairs where the tile's list allows
    const int len = (((g1 - g0 + nsplit - 1) / nsplit) + 63) & ~63;
    g0 = min(g1, g0 + chunk * len);
    g1 = min(g1, g0 + len);
  }
  if (S > 1) {   // this wave's share of the tile's pairs
    const int chunk = (g1 - g0 + S - 1) / S;
    g0 = min(g1, g0 + wid * chunk);
    g1 = min(g1, g0 + chunk);
  }
  const unsigned long long below = (1ull << lane) - 1ull;
  // Classification of the tile's pairs, 64 at a time (lane = pair), into: negligible (falloff below 2^-kCullLog2
  // of the splat's falloff at the pixel centres around its nearest one, at every pixel centre: a zero record),
  // near-opaque
  // (summed by careful_pair at once), small
  // (span above kMomentSpan: queued in s_defer for a direct pass) and the others (queued in s_mi for a moment
  // pass). Only queued pairs occupy lanes of the row loops. The classification bounds u and v over the tile from
  // their values at the middle of the tile's pixel centres and their half-spans (which also decide the form).
  int nmain = 0, ndefer = 0;
  auto classify = [&](int c0) {
    const int i = c0 + lane;
    const bool act = i < g1;
    const int g = act ? gid[i] : 0;
    const float4* r4 = reinterpret_cast<const float4*>(rec) + (size_t)g * 4;
    const float4 r0 = r4[0], r1 = r4[1];
    const float2 sc = *reinterpret_cast<const float2*>(rec + (size_t)g * kRec + R_SY);
    const float2 uv = offsets_at(pym, pxm, r0.x, r0.y, r0.z, r0.w, r1.x, r1.y);
    const float2 hs = half_spans<TILE>(r0.z, r0.w, r1.x, r1.y, tc);
    const bool negl = act && box_min_m(uv.x, uv.y, hs.x, hs.y) >
                                 kCullLog2 + ring_pixel_m(r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, fH, fW, rH, rW);
    const bool near = act && !negl && near_possible(r1.z, r1.w, r0.x, r0.y, fmaxf(sc.x, sc.y), py0, py1, px0, px1);
    const bool defer = act && !negl && !near && !moment_form_ok(hs, sc);
    const bool mom = act && !negl && !near && !defer;
    const int q = (negl || near) ? pair_q[i] : 0;
    if (negl) store_pair<C>(psum + (size_t)q * pair_rec<C>(), PairSums<C>(), 1.f);
    for (unsigned long long nm = __ballot(near); nm; nm &= nm - 1) {
      const int j = __builtin_ctzll(nm);
      float opj;
      const PairSums<C> cs = careful_pair<C, ODDS, TILE>(rec, __builtin_amdgcn_readlane(g, j), ups, s_pxa, lane, opj);
      if (lane == 0) store_pair<C>(psum + (size_t)__builtin_amdgcn_readlane(q, j) * pair_rec<C>(), cs, opj);
    }
    const unsigned long long dm = __ballot(defer), mm = __ballot(mom);
    if (defer) s_defer[ndefer + __popcll(dm & below)] = i;
    if (mom) s_mi[nmain + __popcll(mm & below)] = i;
    ndefer += __popcll(dm);
    nmain += __popcll(mm);
  };
  // One pass over np <= 64 queued pairs: Lp lanes per pair (the largest power of two with np Lp <= 64, at most
  // NP), lane = (pair pr = lane / Lp, share sub = lane % Lp of the tile's pixels: whole rows when that share is
  // at least a row); the Lp partial sums are combined with xor shuffles. MOM: the moment form over s_mi, else the
  // direct form over s_defer.
  auto pass = [&](int np, auto mom) {
    constexpr bool MOM = decltype(mom)::value != 0;
    int lg = 0;   // Lp = 2^lg (shifts, not divisions: Lp is a runtime value)
    while ((np << (lg + 1)) <= 64 && (2 << lg) <= NP) ++lg;
    const int Lp = 1 << lg;
    const int pr = lane >> lg, sub = lane & (Lp - 1);
    const int npx = NP >> lg;
    const bool act = pr < np;
    const int i = act ? (MOM ? s_mi[pr] : s_defer[pr]) : 0;
    const int g = act ? gid[i] : 0;
    const float4* r4 = reinterpret_cast<const float4*>(rec) + (size_t)g * 4;
    const float4 r0 = r4[0], r1 = r4[1], col = r4[2];
    const float op = r1.z;
    PairSums<C> s;
    if (MOM && npx >= TILE) {   // whole rows (uniform branch; the loops' bounds are wave-uniform)
      PairGeo pg = pair_geo(r0, r1);
      mute_pair(!act, pg);
      if (TILE <= 8 && lg == 0)   // one lane per pair: every row
        pair_rows_moments<C, ODDS, TILE, true>(pg, op, col, 0, TILE, ups, tc, s);
      else
        pair_rows_moments<C, ODDS, TILE, false>(pg, op, col, sub * (npx / TILE), npx / TILE, ups, tc, s);
    } else {
      DirectGeo dg = direct_geo(r0, r4[3]);
      mute_direct(!act, dg);
      if (npx >= TILE)
        pair_rows_direct<C, ODDS, TILE>(dg, op, col, sub * (npx / TILE), npx / TILE, ups, tc, s);
      else
        pair_row_part<C, ODDS, TILE>(dg, op, col, sub * npx, npx, ups, s_pxa, s);
    }
    for (int d = 1; d < Lp; d <<= 1) xor_reduce<C>(s, d);
    if (act && sub == 0) store_pair<C>(psum + (size_t)pair_q[i] * pair_rec<C>(), s, op);
  };
  // Queued pairs run in passes of 64 as soon as 64 wait (so at most 127 wait in either queue), the rest once
  // the tile's pairs are classified; a pass's entries leave the queue and the rest move to its front.
  int done = g0;
  for (;;) {
    if (ndefer >= 64 || (done >= g1 && ndefer > 0)) {
      wave_lds_sync();
      const int np = min(ndefer, 64);
      pass(np, IC<0>{});
      const int rest = ndefer - np;
      const int moved = lane < rest ? s_defer[np + lane] : 0;
      wave_lds_sync();
      if (lane < rest) s_defer[lane] = moved;
      ndefer = rest;
    } else if (nmain >= 64 || (done >= g1 && nmain > 0)) {
      wave_lds_sync();
      const int np = min(nmain, 64);
      pass(np, IC<1>{});
      const int rest = nmain - np;
      const int mi = lane < rest ? s_mi[np + lane] : 0;
      wave_lds_sync();
      if (lane < rest) s_mi[lane] = mi;
      nmain = rest;
    } else if (done < g1) {
      classify(done);
      done += 64;
    } else {
      break;
    }
  }
}

// Sum of per-tile partials part[c * nparts + i] over i for every channel, by one 256-thread workgroup (fixed
// order: deterministic). The C * nparts floats are read as one flat array, by float4 loads when `part` is
// 16-byte aligned, 16 loads per thread in flight before any is added: at 9,216 tiles (27,648 floats) that is
// two memory round trips, short enough to stay hidden behind the splat waves of the same launch.
template <int C>
__device__ __forceinline__ void block_bg_sum(const float* __restrict__ part, int nparts, float* __restrict__ g_bg) {
  constexpr int kU = 16;
  __shared__ float s_w[4][kMaxC];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n = C * nparts;
  float acc[kMaxC] = {0.f, 0.f, 0.f, 0.f};
  // adds x (flat index i) to its channel's sum
  auto add = [&](int i, float x) {
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] += (i >= c * nparts && i < (c + 1) * nparts) ? x : 0.f;
  };
  int done = 0;
  if ((reinterpret_cast<uintptr_t>(part) & 15) == 0) {
    const float4* p4 = reinterpret_cast<const float4*>(part);
    const int n4 = n / 4;
    for (int j0 = threadIdx.x; j0 < n4; j0 += 256 * kU) {
      float4 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int j = j0 + u * 256;
        v[u] = j < n4 ? p4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = 4 * (j0 + u * 256);
        add(i, v[u].x);
        add(i + 1, v[u].y);
        add(i + 2, v[u].z);
        add(i + 3, v[u].w);
      }
    }
    done = 4 * n4;
  }
  for (int i0 = done + (int)threadIdx.x; i0 < n; i0 += 256 * kU) {
    float v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = i0 + u * 256;
      v[u] = i < n ? part[i] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) add(i0 + u * 256, v[u]);
  }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const float x = wave_sum(acc[c]);
    if (lane == 0) s_w[wv][c] = x;
  }
  __syncthreads();
  if (threadIdx.x < C) g_bg[threadIdx.x] = (s_w[0][threadIdx.x] + s_w[1][threadIdx.x]) + (s_w[2][threadIdx.x] + s_w[3][threadIdx.x]);
}

template <int C>
__device__ __forceinline__ void zero_grads(int g, float* __restrict__ g_mu, float* __restrict__ g_scale,
                                           float* __restrict__ g_theta, float* __restrict__ g_op,
                                           float* __restrict__ g_col) {
  g_mu[2 * g] = 0.f; g_mu[2 * g + 1] = 0.f;
  g_scale[2 * g] = 0.f; g_scale[2 * g + 1] = 0.f;
  if (g_theta) g_theta[g] = 0.f;
  g_op[g] = 0.f;
#pragma unroll
  for (int c = 0; c < C; ++c) g_col[(size_t)g * C + c] = 0.f;
}

// Per-splat reduction of the per-pair records (contiguous, splat-major: splat g owns q in
// [offsets[g], offsets[g+1])) into parameter gradients, in one launch. kSumLanes consecutive lanes share a
// splat: lane r of the group sums records r, r + kSumLanes, ... in order (kSumUnroll loads in flight), and
// the group's partial sums are combined by a fixed xor tree. A splat with more than kLightPairs pairs is
// left out of that loop and summed afterwards by its whole wave (lane-strided partial sums, then a fixed
// xor tree), so one heavy splat does not serialise its wave. The order of every addition is fixed:
// deterministic. Splats with no pair (none for valid rects) get zeros. With g_bg set, the grid's first
// workgroup sums the per-tile background partials instead.
// Measured at C2 (about 20 records per splat) and C4: 8 lanes per splat 17.2 us and 261 us per launch, against 18.1
// and 265 with 4 lanes, 20.9 and 278 with 2, 19.9 and 270 with 16; with 8 lanes, 2 loads in flight instead of 4
// 18.1 and 284 us. Splats of more than 128 pairs go to the whole-wave path: 16.3 us at C2 against 17.2 with 64
// and 256 (C4 unchanged, 262 us).
constexpr int kSumLanes = 8;
constexpr int kLightPairs = 128;
constexpr int kSumUnroll = 4;

// s += records q, q + step, ... below qe, in that order. The records of kSumUnroll steps are loaded before
// any is added (clamped to the last valid one), so each lane keeps kSumUnroll loads in flight.
template <int R>
__device__ __forceinline__ void sum_pair_recs(float* s, const float* __restrict__ psum, int q, int qe, int step) {
  for (; q < qe; q += kSumUnroll * step) {
    float a[kSumUnroll][R];
#pragma unroll
    for (int u = 0; u < kSumUnroll; ++u) {
      const float* r = psum + (size_t)min(q + u * step, qe - 1) * R;
#pragma unroll
      for (int k = 0; k < R; ++k) a[u][k] = r[k];
    }
#pragma unroll
    for (int u = 0; u < kSumUnroll; ++u)
      if (q + u * step < qe) {
#pragma unroll
        for (int k = 0; k < R; ++k) s[k] += a[u][k];
      }
  }
}

template <int C>
__global__ __launch_bounds__(256) void k_splat_sum(const float* __restrict__ rec, const float* __restrict__ psum,
                                                   const int* __restrict__ offsets, int N, float* __restrict__ g_mu,
                                                   float* __restrict__ g_scale, float* __restrict__ g_theta,
                                                   float* __restrict__ g_op, float* __restrict__ g_col,
                                                   const float* __restrict__ bg_part, int nparts,
                                                   float* __restrict__ g_bg, const float* __restrict__ lsc) {
  constexpr int R = pair_rec<C>();
  constexpr int kPerBlock = 256 / kSumLanes;
  if (g_bg && blockIdx.x == 0) {   // first, so it overlaps the splat waves
    block_bg_sum<C>(bg_part, nparts, g_bg);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int r = lane % kSumLanes;
  const int g = (blockIdx.x - (g_bg ? 1 : 0)) * kPerBlock + (int)threadIdx.x / kSumLanes;
  int q0 = 0, q1 = 0;
  if (g < N) {
    q0 = offsets[g];
    q1 = offsets[g + 1];
  }
  const bool heavy = q1 - q0 > kLightPairs;
  float s[R];
#pragma unroll
  for (int k = 0; k < R; ++k) s[k] = 0.f;
  if (!heavy) sum_pair_recs<R>(s, psum, q0 + r, q1, kSumLanes);
#pragma unroll
  for (int d = 1; d < kSumLanes; d <<= 1)
#pragma unroll
    for (int k = 0; k < R; ++k) s[k] += __shfl_xor(s[k], d, 64);
  for (unsigned long long hm = __ballot(heavy && r == 0); hm; hm &= hm - 1) {
    const int j = __builtin_ctzll(hm);
    const int h0 = __builtin_amdgcn_readlane(q0, j), h1 = __builtin_amdgcn_readlane(q1, j);
    float t[R];
#pragma unroll
    for (int k = 0; k < R; ++k) t[k] = 0.f;
    sum_pair_recs<R>(t, psum, h0 + lane, h1, 64);
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const float x = wave_sum(t[k]);
      if (lane == j) s[k] = x;
    }
  }
  if (g >= N || r != 0) return;
  if (q1 > q0)
    splat_grads<C>(g, rec, s, g_mu, g_scale, g_theta, g_op, g_col, lsc);
  else
    zero_grads<C>(g, g_mu, g_scale, g_theta, g_op, g_col);
}

// Zero gradients for every splat (a render with no pairs), plus g_bg from the partials in the first block.
template <int C>
__global__ __launch_bounds__(256) void k_zero_grads(int N, float* __restrict__ g_mu, float* __restrict__ g_scale,
                                                    float* __restrict__ g_theta, float* __restrict__ g_op,
                                                    float* __restrict__ g_col, const float* __restrict__ bg_part,
                                                    int nparts, float* __restrict__ g_bg) {
  if (g_bg && blockIdx.x == 0) {
    block_bg_sum<C>(bg_part, nparts, g_bg);
    return;
  }
  const int g = (blockIdx.x - (g_bg ? 1 : 0)) * 256 + threadIdx.x;
  if (g < N) zero_grads<C>(g, g_mu, g_scale, g_theta, g_op, g_col);
}

// Exact path backward (render_triton.py:161-266): lane = splat over every pixel; the per-pixel upstream
// terms of each 64-pixel chunk are staged in LDS. Each splat is owned by one lane: plain stores.
template <int C>
__global__ __launch_bounds__(64) void k_bwd_exact(const float* __restrict__ rec, int N, const float* __restrict__ pyv,
                                                  const float* __restrict__ pxv, int P, const float* __restrict__ bg,
                                                  const float* __restrict__ Tin, const float* __restrict__ asum_in,
                                                  const float* __restrict__ fg_in, const float* __restrict__ gout,
                                                  float* __restrict__ acc) {
  __shared__ float4 s_pa[64];
  __shared__ float2 s_pb[64], s_pyx[64];
  const int lane = threadIdx.x;
  const int g = blockIdx.x * 64 + lane;
  const int gs = g < N ? g : N - 1;
  const float4* r4 = reinterpret_cast<const float4*>(rec) + (size_t)gs * 4;
  const float4 r0 = r4[0], r1 = r4[1], col = r4[2];
  const float gy = r0.x, gx = r0.y, A = r0.z, B = r0.w, Cc = r1.x, D = r1.y;
  const PairOp po = pair_op(r1.z);
  PairSums<C> s;
  float bgp[kMaxC] = {0.f, 0.f, 0.f, 0.f};
  for (int p0 = 0; p0 < P; p0 += 64) {
    const int p = p0 + lane;
    float4 pa = make_float4(0.f, 0.f, 0.f, 0.f);
    float2 pb = make_float2(0.f, 0.f), pyx = pb;
    if (p < P) {
      pixel_upstream<C, false, false>(p, 0, bg, Tin, asum_in, fg_in, gout, nullptr, nullptr, nullptr, pa, pb, bgp);
      pyx = make_float2(pyv[p], pxv[p]);
    }
    __syncthreads();
    s_pa[lane] = pa;
    s_pb[lane] = pb;
    s_pyx[lane] = pyx;
    __syncthreads();
    const int np = P - p0 < 64 ? P - p0 : 64;
    for (int j = 0; j < np; ++j) {
      const float2 q = s_pyx[j];
      const float dy = q.x - gy, dx = q.y - gx;
      bwd_px<C, false>(fmaf(A, dy, B * dx), fmaf(Cc, dy, D * dx), po, col, s_pa[j],
                               C > 2 ? s_pb[j] : make_float2(0.f, 0.f), s);
    }
  }
  if (g >= N) return;
  float* dst = acc + (size_t)g * kAcc;
  dst[0] = s.q; dst[1] = s.qu; dst[2] = s.qv; dst[3] = s.quu; dst[4] = s.qvv; dst[5] = s.quv;
#pragma unroll
  for (int c = 0; c < C; ++c) dst[6 + c] = po.op * s.gc[c];
}

// sum_p gout[p, c] * T[p] partials over 256-pixel chunks (the exact path's g_bg, render_triton.py:301).
template <int C>
__global__ __launch_bounds__(256) void k_bg_partial(const float* __restrict__ gout, const float* __restrict__ Tin, int P,
                                                    float* __restrict__ part) {
  __shared__ float s_w[4][kMaxC];
  const int p = blockIdx.x * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    float v = p < P ? gout[(size_t)p * C + c] * Tin[p] : 0.f;
    v = wave_sum(v);
    if (lane == 0) s_w[wv][c] = v;
  }
  __syncthreads();
  if (threadIdx.x < C) part[(size_t)threadIdx.x * gridDim.x + blockIdx.x] = s_w[0][threadIdx.x] + s_w[1][threadIdx.x] +
                                                                             s_w[2][threadIdx.x] + s_w[3][threadIdx.x];
}

// g_bg[c] = sum of the nparts channel-major partials part[c * nparts + i], one 1024-thread workgroup.
template <int C>
__global__ __launch_bounds__(1024) void k_bg_sum(const float* __restrict__ part, int nparts, float* __restrict__ g_bg) {
  __shared__ float s_w[16][kMaxC];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const float* row = part + (size_t)c * nparts;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int i = threadIdx.x;
    for (; i + 3 * 1024 < nparts; i += 4 * 1024) {
      a0 += row[i]; a1 += row[i + 1024]; a2 += row[i + 2048]; a3 += row[i + 3072];
    }
    for (; i < nparts; i += 1024) a0 += row[i];
    const float x = wave_sum((a0 + a1) + (a2 + a3));
    if (lane == 0) s_w[wv][c] = x;
  }
  __syncthreads();
  if (threadIdx.x < C) {
    float x = 0.f;
    for (int w = 0; w < 16; ++w) x += s_w[w][threadIdx.x];
    g_bg[threadIdx.x] = x;
  }
}

// Exact path: per-splat sums (stride kAcc) -> parameter gradients.
template <int C>
__global__ __launch_bounds__(256) void k_acc_finalize(const float* __restrict__ rec, const float* __restrict__ acc, int N,
                                                      float* __restrict__ g_mu, float* __restrict__ g_scale,
                                                      float* __restrict__ g_theta, float* __restrict__ g_op,
                                                      float* __restrict__ g_col) {
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= N) return;
  float v[kSums];
  for (int k = 0; k < kSums; ++k) v[k] = acc[(size_t)g * kAcc + k];
  splat_grads<C>(g, rec, v, g_mu, g_scale, g_theta, g_op, g_col, nullptr);
}

// ------------------------------------------------------------------------------------ upsample adjoint
// The level-0 composite adds bilinear upsamples of the coarse levels' fields (torch upsample_bilinear2d,
// align_corners=False, render_triton.py:864-876). Its exact adjoint maps the level-0 upstream dS_0 to each
// coarse level: dS_l[i, j] = sum_{y, x} wy(y -> i) wx(x -> j) dS_0[y, x], computed as two gather passes
// (columns, then rows) with no atomics. Terms per pixel: S_log, S_a and C colour sums, 2 + C in all.

// Level-0 upsample weight of destination d on source texel i (scale = in / out).
__device__ __forceinline__ float ups_weight(int d, int i, int in, float scale) {
  int p1;
  float l1;
  const int i0 = bilinear_src(d, in, scale, &p1, &l1);
  return (i0 == i ? 1.f - l1 : 0.f) + (i0 + p1 == i ? l1 : 0.f);
}

// Destinations d in [0, out) whose bilinear sources may include texel i: every d with src(d) in [i - 1, i + 1),
// widened by one on each side against rounding (weights are evaluated exactly inside).
__device__ __forceinline__ void ups_window(int i, int out, float scale, int* lo, int* hi) {
  const float inv = 1.f / scale;
  const int a = (int)floorf(((float)i - 0.5f) * inv - 0.5f) - 1;
  const int b = (int)ceilf(((float)i + 1.5f) * inv - 0.5f) + 1;
  *lo = a > 0 ? a : 0;
  *hi = b < out - 1 ? b : out - 1;
}

// Pass 1: workgroup = level-0 row y; tmp[k][y][j] = sum_x wx(x -> ix) dS_0[k][y, x] for the coarse column slots
// j = cbase(l) + ix of every masked level l. Staged modes: the row's 2 + C planes are first copied into LDS
// (coalesced loads; rows whose planes fit in kAdjStageMax floats), so the window loops read LDS. The window of a
// texel of level l spans about 2^(l+1) destinations (131 at the coarsest octave of a 2048-wide canvas) while the
// level has W0 / 2^l texels, so every level is about 2 W0 window steps: the levels are taken one after another by
// the whole workgroup, and a level narrower than the workgroup gives each texel tpc lanes (a power of two, at
// most 64), lane s summing the destinations x0 + s, x0 + s + tpc, ... of the texel's window; the tpc partial sums
// are added by a fixed xor tree (deterministic).
constexpr int kAdjStageMax = 16384;   // floats of LDS per workgroup (64 KiB)

// Where the window loops read the row. kAdjGlobal: from global memory (rows too wide for LDS). kAdjSource: the
// row staged in LDS as it lies in memory, [S_log W0][S_a W0][S_ac W0 x C]. kAdjRotated: plane p (0: S_log, 1: S_a,
// 2 + c: S_ac[c], de-interleaved) at s_row[p * adj_plane(W0) + adj_slot(x)], each 64-word row r = x / 64 of a
// plane rotated by 9 r words, so the lanes of a wave that read destinations 2^l apart (a texel each, or a few
// lanes per texel) mostly fall on different banks: 1.8 lanes per bank on average over the levels of 384- to
// 2048-wide rows, against 3.5 to 5.1 unrotated (a simulation of this kernel's reads). The rotated layout costs an
// LDS read per colour channel instead of one per two or three, which pays on wide rows only (measured against the
// source layout with the same loops: 2048 wide, 98 -> 81 us per launch; 768 wide, about 10.8 -> 13.2 us), so rows
// from kAdjRotateMin pixels take it.
enum AdjMode { kAdjGlobal = 0, kAdjSource = 1, kAdjRotated = 2 };
constexpr int kAdjRotateMin = 1024;
__device__ __forceinline__ int adj_slot(int x) { return (x & ~63) | ((x + 9 * (x >> 6)) & 63); }
__host__ __device__ constexpr int adj_plane(int W0) { return (W0 + 63) & ~63; }

template <int C, int MODE>
__global__ __launch_bounds__(256) void k_adj_cols(LevelTable L, int ncols, const float* __restrict__ dslog,
                                                  const float* __restrict__ dsa, const float* __restrict__ dsac,
                                                  float* __restrict__ tmp) {
  extern __shared__ float s_row[];   // kAdjSource: (2 + C) W0 floats; kAdjRotated: 2 + C planes of adj_plane(W0)
  const int y = blockIdx.x, H0 = L.H[0], W0 = L.W[0];
  const int P = adj_plane(W0);
  const size_t plane = (size_t)H0 * ncols;
  const int t = threadIdx.x;
  const float* rl = dslog + (size_t)y * W0;
  const float* ra = dsa + (size_t)y * W0;
  const float* rc = dsac + (size_t)y * W0 * C;
  if (MODE != kAdjGlobal) {   // the row's (2 + C) W0 floats in source order, 16 loads per thread in flight
    constexpr int kU = 16;
    const int n = (2 + C) * W0;
    for (int i0 = t; i0 < n; i0 += 256 * kU) {
      float v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int k = i0 + u * 256;
        v[u] = k < W0 ? rl[k] : k < 2 * W0 ? ra[k - W0] : k < n ? rc[k - 2 * W0] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int k = i0 + u * 256;
        if (k >= n) continue;
        if (MODE == kAdjSource) {
          s_row[k] = v[u];
          continue;
        }
        int pl, x;
        if (k < 2 * W0) {
          pl = k < W0 ? 0 : 1;
          x = k - pl * W0;
        } else {
          const int j = k - 2 * W0;
          x = j / C;
          pl = 2 + (j - x * C);
        }
        s_row[pl * P + adj_slot(x)] = v[u];
      }
    }
    __syncthreads();
  }
  // the 2 + C values of destination x
  auto fetch = [&](int x, float& vl, float& va, float* vc) {
    if (MODE == kAdjSource) {
      vl = s_row[x];
      va = s_row[W0 + x];
#pragma unroll
      for (int c = 0; c < C; ++c) vc[c] = s_row[2 * W0 + x * C + c];
    } else if (MODE == kAdjRotated) {
      const int sl = adj_slot(x);
      vl = s_row[sl];
      va = s_row[P + sl];
#pragma unroll
      for (int c = 0; c < C; ++c) vc[c] = s_row[(2 + c) * P + sl];
    } else {
      vl = rl[x];
      va = ra[x];
#pragma unroll
      for (int c = 0; c < C; ++c) vc[c] = rc[(size_t)x * C + c];
    }
  };
  int cb = 0;
  for (int l = 1; l < L.n; cb += L.W[l], ++l) {
    if (!((L.mask >> l) & 1)) continue;
    const int Wl = L.W[l];
    const float sx = (float)Wl / (float)W0;
    int tpc = 1;   // lanes per texel (block-uniform)
    while (tpc < 64 && Wl * tpc * 2 <= 256) tpc *= 2;
    const int sub = t & (tpc - 1);
    for (int j0 = 0; j0 < Wl * tpc; j0 += 256) {   // block-uniform trip count (the xor tree needs every lane)
      const int ix = (j0 + t) / tpc;
      float al = 0.f, aa = 0.f, ac[kMaxC] = {0.f, 0.f, 0.f, 0.f};
      if (ix < Wl) {
        int x0, x1;
        ups_window(ix, W0, sx, &x0, &x1);
        int x = x0 + sub;
        // The weight of texel ix for destination x at source position r = max(sx (x + 0.5) - 0.5, 0) (x + 0.5
        // carried as a float: exact): max(0, 1 - |r - ix|), what ups_weight gives (1 - (r - i) on texel
        // i = floor(r), r - i on texel i + 1), except that the last texel also takes its missing right
        // neighbour's share, (1 - d) + d for d = r - ix > 0.
        const float fix = (float)ix;
        const bool last = ix == Wl - 1;
        float xf = (float)x + 0.5f;
        auto weight = [&](float xh) {
          const float d = fmaxf(fmaf(sx, xh, -0.5f), 0.f) - fix;
          return (last && d > 0.f) ? (1.f - d) + d : fmaxf(1.f - fabsf(d), 0.f);
        };
        const float step = (float)tpc;
        // four destinations per step, their loads issued before any is added (the additions keep the order of x)
        for (; x + 3 * tpc <= x1; x += 4 * tpc, xf += 4.f * step) {
          float w[4], vl[4], va[4], vc[4][kMaxC];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            w[u] = weight(xf + (float)u * step);
            fetch(x + u * tpc, vl[u], va[u], vc[u]);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            al += w[u] * vl[u];
            aa += w[u] * va[u];
#pragma unroll
            for (int c = 0; c < C; ++c) ac[c] += w[u] * vc[u][c];
          }
        }
        for (; x <= x1; x += tpc, xf += step) {
          const float w = weight(xf);
          float vl, va, vc[kMaxC];
          fetch(x, vl, va, vc);
          al += w * vl;
          aa += w * va;
#pragma unroll
          for (int c = 0; c < C; ++c) ac[c] += w * vc[c];
        }
      }
      for (int d = 1; d < tpc; d <<= 1) {
        al += __shfl_xor(al, d, 64);
        aa += __shfl_xor(aa, d, 64);
#pragma unroll
        for (int c = 0; c < C; ++c) ac[c] += __shfl_xor(ac[c], d, 64);
      }
      if (ix < Wl && sub == 0) {
        const size_t o = (size_t)y * ncols + cb + ix;
        tmp[o] = al;
        tmp[plane + o] = aa;
#pragma unroll
        for (int c = 0; c < C; ++c) tmp[(2 + c) * plane + o] = ac[c];
      }
    }
  }
}

// Pass 2: thread = coarse texel (l, iy, ix) of a masked level, q = packed slot - pbase[1];
// dS_l[iy, ix] = sum_y wy(y -> iy) tmp[k][y][cbase(l) + ix], written to the packed fields at pbase[l].
template <int C>
__global__ __launch_bounds__(256) void k_adj_rows(LevelTable L, int ncols, const float* __restrict__ tmp,
                                                  float* __restrict__ dslog, float* __restrict__ dsa,
                                                  float* __restrict__ dsac) {
  const int q = blockIdx.x * 256 + threadIdx.x;
  if (q >= L.pbase[L.n] - L.pbase[1]) return;
  const int pp = L.pbase[1] + q;
  const int l = level_of_slot(L, pp);
  if (!((L.mask >> l) & 1)) return;
  int cb = 0;
  for (int k = 1; k < l; ++k) cb += L.W[k];
  const int Hl = L.H[l], Wl = L.W[l], H0 = L.H[0];
  const int r = pp - L.pbase[l], iy = r / Wl, ix = r - iy * Wl;
  const float sy = (float)Hl / (float)H0;
  const size_t plane = (size_t)H0 * ncols;
  int y0, y1;
  ups_window(iy, H0, sy, &y0, &y1);
  float al = 0.f, aa = 0.f, ac[kMaxC] = {0.f, 0.f, 0.f, 0.f};
  int y = y0;
  // four source rows per step, their loads issued before any is added (rows of weight 0 add nothing, as below)
  for (; y + 3 <= y1; y += 4) {
    float w[4], vl[4], va[4], vc[4][kMaxC];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      w[u] = ups_weight(y + u, iy, Hl, sy);
      const size_t o = (size_t)(y + u) * ncols + cb + ix;
      vl[u] = va[u] = 0.f;
#pragma unroll
      for (int c = 0; c < C; ++c) vc[u][c] = 0.f;
      if (w[u] != 0.f) {   // rows of the widened window outside the texel's support are not fetched
        vl[u] = tmp[o];
        va[u] = tmp[plane + o];
#pragma unroll
        for (int c = 0; c < C; ++c) vc[u][c] = tmp[(2 + c) * plane + o];
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (w[u] == 0.f) continue;
      al += w[u] * vl[u];
      aa += w[u] * va[u];
#pragma unroll
      for (int c = 0; c < C; ++c) ac[c] += w[u] * vc[u][c];
    }
  }
  for (; y <= y1; ++y) {
    const float w = ups_weight(y, iy, Hl, sy);
    if (w == 0.f) continue;
    const size_t o = (size_t)y * ncols + cb + ix;
    al += w * tmp[o];
    aa += w * tmp[plane + o];
#pragma unroll
    for (int c = 0; c < C; ++c) ac[c] += w * tmp[(2 + c) * plane + o];
  }
  dslog[pp] = al;
  dsa[pp] = aa;
#pragma unroll
  for (int c = 0; c < C; ++c) dsac[(size_t)pp * C + c] = ac[c];
}

// ---------------------------------------------------------------------------------------------------- dispatch
template <typename F>
int with_c(int C, F&& f) {
  switch (C) {
    case 1: return f(IC<1>{});
    case 2: return f(IC<2>{});
    case 3: return f(IC<3>{});
    case 4: return f(IC<4>{});
  }
  return set_error(kUnsupported, "colour channels C=%d not supported (1..%d)", C, kMaxC);
}

template <typename F>
int with_tile(int TILE, F&& f) {
  switch (TILE) {
    case 4: return f(IC<4>{});
    case 8: return f(IC<8>{});
    case 16: return f(IC<16>{});
  }
  return set_error(kUnsupported, "TILE=%d not supported (4, 8 or 16)", TILE);
}

// FIELDS, ODDS, UPS (UPS only with the composite: the caller rejects FIELDS | UPS).
template <typename F>
int with_flags(int flags, F&& f) {
  switch (flags & 7) {
    case 0: return f(IC<0>{}, IC<0>{}, IC<0>{});
    case 1: return f(IC<1>{}, IC<0>{}, IC<0>{});
    case 2: return f(IC<0>{}, IC<1>{}, IC<0>{});
    case 3: return f(IC<1>{}, IC<1>{}, IC<0>{});
    case 4: return f(IC<0>{}, IC<0>{}, IC<1>{});
    default: return f(IC<0>{}, IC<1>{}, IC<1>{});
  }
}

// Host: level table and the tile range [tb0, tb0 + ntiles) of a launch over levels [lev_begin, lev_end).
static int launch_levels(const char* who, int H, int W, int TILE, const splat_levels* lv, int lev_begin, int lev_end,
                         unsigned levmask, int flags, LevelTable* L, int* tb0, int* ntiles) {
  if (H < 1 || W < 1) return set_error(kInvalid, "%s: H=%d W=%d", who, H, W);
  if ((flags & kFlagFields) && (flags & kFlagUps)) return set_error(kInvalid, "%s: FIELDS and UPS exclude each other", who);
  if (make_levels(H, W, TILE, lv, L, nullptr)) return set_error(kInvalid, "%s: bad levels for H=%d W=%d", who, H, W);
  if (lev_begin < 0 || lev_end > L->n || lev_begin >= lev_end)
    return set_error(kInvalid, "%s: levels [%d, %d) outside [0, %d)", who, lev_begin, lev_end, L->n);
  if (!(flags & kFlagFields) && (lev_begin != 0 || lev_end != 1))
    return set_error(kInvalid, "%s: the composite renders level 0 only", who);
  L->mask = levmask & L->mask;
  *tb0 = L->tbase[lev_begin];
  *ntiles = L->tbase[lev_end] - L->tbase[lev_begin];
  return kOk;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace splat

using namespace splat;

extern "C" {

}  // extern "C"

namespace {

// Events for the next tile-kernel launch of this thread (splat_time_next_launch), or nulls.
thread_local hipEvent_t g_time_start = nullptr, g_time_stop = nullptr;

// Launch of a forward or backward tile kernel; with events armed by splat_time_next_launch the kernel records
// them itself at its start and end (hipExtLaunchKernel), and the events are disarmed.
template <typename... KArgs, typename... Args>
void launch_tile_kernel(void (*kernel)(KArgs...), unsigned grid, unsigned block, hipStream_t st, Args... args) {
  if (g_time_start && g_time_stop) {
    hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(block), 0, st, g_time_start, g_time_stop, 0, args...);
    g_time_start = g_time_stop = nullptr;
  } else {
    kernel<<<grid, block, 0, st>>>(args...);
  }
}

}  // namespace

extern "C" {

int splat_time_next_launch(void* start, void* stop) {
  const int pending = g_time_start != nullptr;
  g_time_start = (hipEvent_t)start;
  g_time_stop = (hipEvent_t)stop;
  return pending;
}

int splat_render_fwd(const float* rec, const int* gid_sorted, const int* tile_starts, int C, int H, int W, int TILE,
                     int flags, const splat_levels* lv, int lev_begin, int lev_end, unsigned levmask, const float* bg,
                     float* out, float* T, float* asum, float* fg, float* slog, float* sa, float* sac, void* stream) {
  LevelTable L;
  int tb0, ntiles;
  if (int e = launch_levels("splat_render_fwd", H, W, TILE, lv, lev_begin, lev_end, levmask, flags, &L, &tb0, &ntiles))
    return e;
  if (!rec || !gid_sorted || !tile_starts) return set_error(kInvalid, "splat_render_fwd: null pair list");
  const bool fields = flags & kFlagFields;
  const bool coarse_in = (flags & kFlagUps) && (L.mask & ~1u);
  if (fields || coarse_in ? (!slog || !sa || !sac) : false)
    return set_error(kInvalid, "splat_render_fwd: null fields for flags=%d", flags);
  if (!fields && (!bg || !out || !T || !asum || !fg))
    return set_error(kInvalid, "splat_render_fwd: null output for flags=%d", flags);
  if (ntiles == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  return with_c(C, [&](auto cc) {
    return with_tile(TILE, [&](auto tt) {
      return with_flags(flags, [&](auto fl, auto od, auto up) {
        constexpr int CC = decltype(cc)::value, TT = decltype(tt)::value;
        constexpr bool FL = decltype(fl)::value != 0, OD = decltype(od)::value != 0, UP = decltype(up)::value != 0;
        if (TT == 8 && (flags & kFlagWide)) {
          constexpr int S = fwd_split<TT, true>();
          launch_tile_kernel(k_fwd_cull<CC, FL, OD, UP, TT, S>, ntiles, fwd_threads<TT, S>(), st, rec, gid_sorted,
                             tile_starts, L, tb0, ntiles, bg, out, T, asum, fg, slog, sa, sac);
        } else {
          constexpr int S = fwd_split<TT, false>();
          launch_tile_kernel(k_fwd_cull<CC, FL, OD, UP, TT, S>, ntiles, fwd_threads<TT, S>(), st, rec, gid_sorted,
                             tile_starts, L, tb0, ntiles, bg, out, T, asum, fg, slog, sa, sac);
        }
        return check_launch("k_fwd_cull");
      });
    });
  });
}

size_t splat_pair_sums_bytes(long long tot) { return sizeof(float) * kPairRecMax * (size_t)(tot > 0 ? tot : 1); }

int splat_render_bwd(const float* rec, const int* gid_sorted, const int* tile_starts, const int* pair_q, long long tot,
                     int C, int H, int W, int TILE, int flags, const splat_levels* lv, int lev_begin, int lev_end,
                     unsigned levmask, const float* bg, const float* T, const float* asum, const float* fg,
                     const float* gout, float* dslog, float* dsa, float* dsac, float* pair_sums, float* bg_part,
                     void* stream) {
  LevelTable L;
  int tb0, ntiles;
  if (int e = launch_levels("splat_render_bwd", H, W, TILE, lv, lev_begin, lev_end, levmask, flags, &L, &tb0, &ntiles))
    return e;
  if (tot < 0 || tot > 0x7fffffffLL - 64) return set_error(kInvalid, "splat_render_bwd: tot=%lld", tot);
  if (!rec || !gid_sorted || !tile_starts || !pair_sums || (tot > 0 && !pair_q))
    return set_error(kInvalid, "splat_render_bwd: null pointer");
  const bool fields = flags & kFlagFields;
  if ((fields || (flags & kFlagUps)) && (!dslog || !dsa || !dsac))
    return set_error(kInvalid, "splat_render_bwd: null upstream fields for flags=%d", flags);
  if (!fields && (!bg || !T || !asum || !fg || !gout))
    return set_error(kInvalid, "splat_render_bwd: null upstream for flags=%d", flags);
  if (fields && bg_part) return set_error(kInvalid, "splat_render_bwd: no background partials in FIELDS mode");
  if (ntiles == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  return with_c(C, [&](auto cc) {
    return with_tile(TILE, [&](auto tt) {
      return with_flags(flags, [&](auto fl, auto od, auto up) {
        constexpr int CC = decltype(cc)::value, TT = decltype(tt)::value;
        constexpr bool FL = decltype(fl)::value != 0, OD = decltype(od)::value != 0, UP = decltype(up)::value != 0;
        if (TT == 8 && (flags & kFlagWide))
          launch_tile_kernel(k_bwd_cull<CC, FL, OD, UP, TT, 16>, ntiles, 64 * 16, st, rec, gid_sorted, tile_starts, L,
                             tb0, ntiles, bg, T, asum, fg, gout, dslog, dsa, dsac, pair_q, pair_sums, bg_part,
                             SplitTable{});
        else
          launch_tile_kernel(k_bwd_cull<CC, FL, OD, UP, TT, 1>, ntiles, 64, st, rec, gid_sorted, tile_starts, L, tb0,
                             ntiles, bg, T, asum, fg, gout, dslog, dsa, dsac, pair_q, pair_sums, bg_part, SplitTable{});
        return check_launch("k_bwd_cull");
      });
    });
  });
}

// Host: the SplitTable of a split launch over the levels [lev_begin, lev_end) present in L.mask (levels outside
// take no items); *nitems work items, *ncomb tiles to combine, *npart partial items.
constexpr int kMaxSplit = 1024;
static int make_split(const char* who, const LevelTable& L, int lev_begin, int lev_end, const int* splits,
                      SplitTable* P, int* nitems, int* ncomb, long long* npart) {
  if (!splits) return set_error(kInvalid, "%s: null splits", who);
  SplitTable t{};
  long long items = 0, comb = 0, part = 0;
  for (int l = 0; l < L.n; ++l) {
    t.ibase[l] = (int)items;
    t.cbase[l] = (int)comb;
    t.pibase[l] = (int)part;
    const bool in = l >= lev_begin && l < lev_end && ((L.mask >> l) & 1);
    const int s = in ? splits[l] : 0;
    if (in && (s < 1 || s > kMaxSplit))
      return set_error(kInvalid, "%s: splits[%d] = %d outside [1, %d]", who, l, s, kMaxSplit);
    t.split[l] = s;
    const long long nt = L.tbase[l + 1] - L.tbase[l];
    items += nt * s;
    if (s > 1) {
      comb += nt;
      part += nt * s;
    }
    if (items > 0x3fffffffLL) return set_error(kOverflow, "%s: %lld work items", who, items);
  }
  t.ibase[L.n] = (int)items;
  t.cbase[L.n] = (int)comb;
  *P = t;
  *nitems = (int)items;
  *ncomb = (int)comb;
  *npart = part;
  return kOk;
}

static size_t split_part_bytes(int C, int TILE, long long npart) {
  return sizeof(float) * (size_t)(2 + C) * (size_t)tile_threads(TILE) * (size_t)npart;
}

size_t splat_fields_split_workspace_bytes(int C, int H, int W, int TILE, const splat_levels* lv, int lev_begin,
                                          int lev_end, unsigned levmask, const int* splits) {
  LevelTable L;
  int tb0, ntiles, nitems, ncomb;
  long long npart;
  SplitTable P;
  if (C < 1 || C > kMaxC || (TILE != 4 && TILE != 8 && TILE != 16) ||
      launch_levels("splat_fields_split_workspace_bytes", H, W, TILE, lv, lev_begin, lev_end, levmask, kFlagFields,
                    &L, &tb0, &ntiles) ||
      make_split("splat_fields_split_workspace_bytes", L, lev_begin, lev_end, splits, &P, &nitems, &ncomb, &npart))
    return 0;
  return split_part_bytes(C, TILE, npart);
}

int splat_render_fields_split(const float* rec, const int* gid_sorted, const int* tile_starts, int C, int H, int W,
                              int TILE, int flags, const splat_levels* lv, int lev_begin, int lev_end,
                              unsigned levmask, const int* splits, float* slog, float* sa, float* sac, void* ws,
                              size_t ws_bytes, void* stream) {
  LevelTable L;
  int tb0, ntiles, nitems, ncomb;
  long long npart;
  SplitTable P;
  if (flags & ~kFlagOdds) return set_error(kInvalid, "splat_render_fields_split: flags=%d (only ODDS)", flags);
  if (int e = launch_levels("splat_render_fields_split", H, W, TILE, lv, lev_begin, lev_end, levmask,
                            flags | kFlagFields, &L, &tb0, &ntiles))
    return e;
  if (int e = make_split("splat_render_fields_split", L, lev_begin, lev_end, splits, &P, &nitems, &ncomb, &npart))
    return e;
  if (!rec || !gid_sorted || !tile_starts || !slog || !sa || !sac)
    return set_error(kInvalid, "splat_render_fields_split: null pointer");
  if (nitems == 0) return kOk;
  if (ncomb && (!ws || ws_bytes < split_part_bytes(C, TILE, npart)))
    return set_error(kWorkspace, "splat_render_fields_split: workspace of %zu bytes, %zu needed", ws_bytes,
                     split_part_bytes(C, TILE, npart));
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)ws;
  return with_c(C, [&](auto cc) {
    return with_tile(TILE, [&](auto tt) {
      constexpr int CC = decltype(cc)::value, TT = decltype(tt)::value;
      if (flags & kFlagOdds)
        launch_tile_kernel(k_fwd_fields_split<CC, true, TT>, nitems, tile_threads(TT), st, rec, gid_sorted,
                           tile_starts, L, P, nitems, slog, sa, sac, part);
      else
        launch_tile_kernel(k_fwd_fields_split<CC, false, TT>, nitems, tile_threads(TT), st, rec, gid_sorted,
                           tile_starts, L, P, nitems, slog, sa, sac, part);
      if (ncomb) k_fields_combine<CC, TT><<<ncomb, tile_threads(TT), 0, st>>>(L, P, part, slog, sa, sac);
      return check_launch("k_fwd_fields_split");
    });
  });
}

int splat_render_fields_split_bwd(const float* rec, const int* gid_sorted, const int* tile_starts, const int* pair_q,
                                  long long tot, int C, int H, int W, int TILE, int flags, const splat_levels* lv,
                                  int lev_begin, int lev_end, unsigned levmask, const int* splits, float* dslog,
                                  float* dsa, float* dsac, float* pair_sums, void* stream) {
  LevelTable L;
  int tb0, ntiles, nitems, ncomb;
  long long npart;
  SplitTable P;
  if (flags & ~kFlagOdds) return set_error(kInvalid, "splat_render_fields_split_bwd: flags=%d (only ODDS)", flags);
  if (int e = launch_levels("splat_render_fields_split_bwd", H, W, TILE, lv, lev_begin, lev_end, levmask,
                            flags | kFlagFields, &L, &tb0, &ntiles))
    return e;
  if (int e = make_split("splat_render_fields_split_bwd", L, lev_begin, lev_end, splits, &P, &nitems, &ncomb, &npart))
    return e;
  if (tot < 0 || tot > 0x7fffffffLL - 64) return set_error(kInvalid, "splat_render_fields_split_bwd: tot=%lld", tot);
  if (!rec || !gid_sorted || !tile_starts || !pair_sums || !dslog || !dsa || !dsac || (tot > 0 && !pair_q))
    return set_error(kInvalid, "splat_render_fields_split_bwd: null pointer");
  if (nitems == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  return with_c(C, [&](auto cc) {
    return with_tile(TILE, [&](auto tt) {
      constexpr int CC = decltype(cc)::value, TT = decltype(tt)::value;
      if (flags & kFlagOdds)
        launch_tile_kernel(k_bwd_cull<CC, true, true, false, TT, 1, true>, nitems, 64, st, rec, gid_sorted,
                           tile_starts, L, 0, nitems, nullptr, nullptr, nullptr, nullptr, nullptr, dslog, dsa, dsac,
                           pair_q, pair_sums, nullptr, P);
      else
        launch_tile_kernel(k_bwd_cull<CC, true, false, false, TT, 1, true>, nitems, 64, st, rec, gid_sorted,
                           tile_starts, L, 0, nitems, nullptr, nullptr, nullptr, nullptr, nullptr, dslog, dsa, dsac,
                           pair_q, pair_sums, nullptr, P);
      return check_launch("k_bwd_cull(split)");
    });
  });
}

static int adjoint_cols(const LevelTable& L) {
  int n = 0;
  for (int l = 1; l < L.n; ++l) n += L.W[l];
  return n;
}

size_t splat_upsample_adjoint_workspace_bytes(int C, int H, int W, int TILE, const splat_levels* lv) {
  LevelTable L;
  if (C < 1 || C > kMaxC || H < 1 || W < 1 || make_levels(H, W, TILE, lv, &L, nullptr)) return 0;
  return align256(sizeof(float) * (size_t)(2 + C) * (size_t)L.H[0] * (size_t)(adjoint_cols(L) > 0 ? adjoint_cols(L) : 1));
}

int splat_upsample_adjoint(int C, int H, int W, int TILE, const splat_levels* lv, unsigned levmask, float* dslog,
                           float* dsa, float* dsac, void* ws, size_t ws_bytes, void* stream) {
  LevelTable L;
  if (C < 1 || C > kMaxC || H < 1 || W < 1 || make_levels(H, W, TILE, lv, &L, nullptr))
    return set_error(kInvalid, "splat_upsample_adjoint: C=%d H=%d W=%d or bad levels", C, H, W);
  if (!dslog || !dsa || !dsac) return set_error(kInvalid, "splat_upsample_adjoint: null fields");
  L.mask = levmask & L.mask & ~1u;
  if (L.n < 2 || !L.mask) return kOk;
  if (!ws || ws_bytes < splat_upsample_adjoint_workspace_bytes(C, H, W, TILE, lv))
    return set_error(kWorkspace, "splat_upsample_adjoint: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  const int ncols = adjoint_cols(L);
  const int ncoarse = L.pbase[L.n] - L.pbase[1];
  float* tmp = (float*)ws;
  return with_c(C, [&](auto cc) {
    constexpr int CC = decltype(cc)::value;
    const int W0 = L.W[0];
    const size_t src = sizeof(float) * (size_t)(2 + CC) * (size_t)W0;
    const size_t rot = sizeof(float) * (size_t)(2 + CC) * (size_t)adj_plane(W0);
    if (W0 >= kAdjRotateMin && rot <= sizeof(float) * kAdjStageMax)
      k_adj_cols<CC, kAdjRotated><<<L.H[0], 256, rot, st>>>(L, ncols, dslog, dsa, dsac, tmp);
    else if (src <= sizeof(float) * kAdjStageMax)
      k_adj_cols<CC, kAdjSource><<<L.H[0], 256, src, st>>>(L, ncols, dslog, dsa, dsac, tmp);
    else
      k_adj_cols<CC, kAdjGlobal><<<L.H[0], 256, 0, st>>>(L, ncols, dslog, dsa, dsac, tmp);
    k_adj_rows<CC><<<(ncoarse + 255) / 256, 256, 0, st>>>(L, ncols, tmp, dslog, dsa, dsac);
    return check_launch("splat_upsample_adjoint");
  });
}

int splat_reduce_pairs(const float* rec, const int* offsets, const int* pair_splat, long long tot,
                       int N, int C, const float* pair_sums, const float* bg_part, int nparts, const float* log_scale,
                       float* g_mu, float* g_scale, float* g_theta, float* g_op, float* g_color, float* g_bg, void* stream) {
  if (N < 0 || tot < 0 || tot > 0x7fffffffLL - 64 || (N == 0 && tot > 0))
    return set_error(kInvalid, "splat_reduce_pairs: N=%d tot=%lld", N, tot);
  if ((N > 0 && (!rec || !offsets || !g_mu || !g_scale || !g_op || !g_color)) ||
      (tot > 0 && !pair_sums) || (g_bg && (!bg_part || nparts < 1)))
    return set_error(kInvalid, "splat_reduce_pairs: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const unsigned extra = g_bg ? 1u : 0u;
  return with_c(C, [&](auto cc) {
    constexpr int CC = decltype(cc)::value;
    if (tot > 0)
      k_splat_sum<CC><<<(unsigned)((N + 256 / kSumLanes - 1) / (256 / kSumLanes)) + extra, 256, 0, st>>>(
          rec, pair_sums, offsets, N, g_mu, g_scale, g_theta, g_op, g_color, bg_part, nparts, g_bg, log_scale);
    else if (N > 0 || g_bg)
      k_zero_grads<CC><<<(unsigned)((N + 255) / 256) + extra, 256, 0, st>>>(N, g_mu, g_scale, g_theta, g_op,
                                                                            g_color, bg_part, nparts, g_bg);
    return check_launch("splat_reduce_pairs");
  });
}

int splat_exact_fwd(const float* rec, int N, int C, const float* py, const float* px, int P, const float* bg, float* out,
                    float* T, float* asum, float* fg, void* stream) {
  if (N < 0 || P < 1 || !rec || !py || !px || !bg || !out || !T || !asum || !fg)
    return set_error(kInvalid, "splat_exact_fwd: bad arguments N=%d P=%d", N, P);
  hipStream_t st = (hipStream_t)stream;
  return with_c(C, [&](auto cc) {
    k_fwd_exact<decltype(cc)::value><<<(P + 63) / 64, 64, 0, st>>>(rec, N, py, px, P, bg, out, T, asum, fg);
    return check_launch("k_fwd_exact");
  });
}

size_t splat_exact_bwd_workspace_bytes(int N, int C, int P) {
  return align256(sizeof(float) * kAcc * (size_t)(N > 0 ? N : 1)) +
         align256(sizeof(float) * (size_t)((P + 255) / 256 + 1) * (C > 0 ? C : 1));
}

int splat_exact_bwd(const float* rec, int N, int C, const float* py, const float* px, int P, const float* bg,
                    const float* T, const float* asum, const float* fg, const float* gout, float* g_mu, float* g_scale,
                    float* g_theta, float* g_op, float* g_color, float* g_bg, void* ws, size_t ws_bytes, void* stream) {
  if (N < 0 || P < 1 || !py || !px || !bg || !T || !asum || !fg || !gout ||
      (N > 0 && (!rec || !g_mu || !g_scale || !g_op || !g_color)))
    return set_error(kInvalid, "splat_exact_bwd: bad arguments N=%d P=%d", N, P);
  if (ws_bytes < splat_exact_bwd_workspace_bytes(N, C, P)) return set_error(kWorkspace, "splat_exact_bwd: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  float* acc = (float*)ws;
  float* part = (float*)((char*)ws + align256(sizeof(float) * kAcc * (size_t)(N > 0 ? N : 1)));
  const int nchunk = (P + 255) / 256;
  return with_c(C, [&](auto cc) {
    constexpr int CC = decltype(cc)::value;
    if (N > 0) k_bwd_exact<CC><<<(N + 63) / 64, 64, 0, st>>>(rec, N, py, px, P, bg, T, asum, fg, gout, acc);
    if (g_bg) {
      k_bg_partial<CC><<<nchunk, 256, 0, st>>>(gout, T, P, part);
      k_bg_sum<CC><<<1, 1024, 0, st>>>(part, nchunk, g_bg);
    }
    if (N > 0)
      k_acc_finalize<CC><<<(N + 255) / 256, 256, 0, st>>>(rec, acc, N, g_mu, g_scale, g_theta, g_op, g_color);
    return check_launch("splat_exact_bwd");
  });
}

}  // extern "C"
