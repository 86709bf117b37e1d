// Splat -> tile binning on gfx950, bit-exact with render_triton.py:351-409 (`_build_tiles`):
//   k_decode_count   one coalesced pass over the splat parameters: the decoded render record, the tile
//                    rect and the pair count of every splat, and per-block count sums
//   k_offsets_fused  exclusive scan of the counts into per-splat pair offsets (offsets[N] = tot), and the
//                    totals, also into the caller's pinned host buffer (no copy before the host's one read);
//                    k_scan_sums + k_offsets beyond kFusedScanBlocks blocks
//   k_scatter_pairs  load-balanced expansion of every splat's rect into (tile, splat) pairs, splat-major
//                    as the reference generates them (:396-404), fused with the first radix histogram
//   k_radix_*        stable radix passes on the tile id; the values carried are the splat id and (for
//                    the backward) the pair's splat-major index, which the first pass takes from the pair's
//                    position: within a tile the splats keep ascending order, the order of the reference's
//                    stable argsort (:405-407)
//   k_local_sort     tile ids of 10 to 14 bits: one radix pass orders the pairs by super-tile (tile >> lb),
//                    then a workgroup per super-tile sorts its pairs on the low lb bits and writes the
//                    super-tile's CSR starts
//   k_tile_starts    otherwise (LSD passes over the whole id): CSR starts, starts[t] = number of pairs with
//                    tile < t (:408)
//
// This file is compiled with -ffp-contract=off: the rect arithmetic below must round every float32
// operation separately (a fused mu*W - r*W changes floor() near tile edges).
#include <limits.h>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <sys/syscall.h>
#include <unistd.h>


#include "splat_common.h"

namespace splat {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kItems = 8;                       // keys per thread in the pair/sort kernels
constexpr int kSortKeys = kBlock * kItems;      // 2048 keys per block
constexpr int kWaveKeys = kSortKeys / kWaves;   // 512 consecutive keys per wave
constexpr long long kBadBit = 1LL << 62;        // marks a block holding an empty or inverted rect
constexpr int kMaxRadixBits = 9;                // radix passes sort on digits of at most 9 bits
constexpr int kMaxRadix = 1 << kMaxRadixBits;

// Exclusive prefix of `v` over a 256-thread block (4 waves) with op = sum (MAX = false) or max (MAX = true,
// identity -1). Returns the block total / maximum in `total`. Every thread must call it.
template <bool MAX>
__device__ __forceinline__ int block256_excl(int v, int* s_w, int& total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(inc, d, 64);
    if (lane >= d) inc = MAX ? max(inc, o) : inc + o;
  }
  if (lane == 63) s_w[wv] = inc;
  __syncthreads();
  int pre = MAX ? -1 : 0, tot = MAX ? -1 : 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int x = s_w[w];
    if (w < wv) pre = MAX ? max(pre, x) : pre + x;
    tot = MAX ? max(tot, x) : tot + x;
  }
  int ex = __shfl_up(inc, 1, 64);
  if (lane == 0) ex = MAX ? -1 : 0;
  total = tot;
  __syncthreads();
  return MAX ? max(pre, ex) : pre + ex;
}

// ----------------------------------------------------------------------------------------------------
// decode + level + rect + count. block_sums[blk * kSumCols + 0] = the block's pair count (| kBadBit),
// block_sums[blk * kSumCols + 1 + l] = its pairs on level l.
// With `rowhist` (the row plan of the pair phase, below): also the block's histogram over the global tile rows
// of its splats' units (one unit = one splat x one tile row of its rect), rowhist[r * nb + blk] = (units of
// row r, pairs of row r) for every row r < L.rbase[L.n], from difference arrays in LDS.
constexpr int kSumCols = 1 + kMaxLevels;
constexpr int kMaxRows = 1024;   // the row plan takes level tables of at most this many tile rows

template <int C>
__global__ __launch_bounds__(kBlock) void k_decode_count(
    const float* __restrict__ mu, const float* __restrict__ scale, const float* __restrict__ theta,
    const float* __restrict__ opacity, const float* __restrict__ color, int N, LevelTable L, Routing R, float fT,
    float cutoff, int do_bin, int act, float4* __restrict__ rec, int4* __restrict__ rect, int* __restrict__ counts,
    long long* __restrict__ block_sums, int2* __restrict__ rowhist, int nb) {
  __shared__ long long s_part[kWaves];
  __shared__ int s_lev[kMaxLevels];
  __shared__ int s_du[kMaxRows + 1], s_dp[kMaxRows + 1];
  __shared__ float4 s_rec[kBlock * 4];   // the block's records, written out coalesced
  const int g = blockIdx.x * kBlock + threadIdx.x;
  const int nrows = L.rbase[L.n];
  // float4 k of splat t of the block sits at s_rec[4 t + (k ^ ((t >> 2) & 3))]: 16 consecutive lanes then write
  // 16 different 16-byte bank groups (slot mod 16) and read back 16 consecutive slots
  auto rec_slot = [](int t, int k) { return 4 * t + (k ^ ((t >> 2) & 3)); };
  if (do_bin) {
    for (int i = threadIdx.x; i < kMaxLevels; i += kBlock) s_lev[i] = 0;
    if (rowhist)
      for (int i = threadIdx.x; i <= nrows; i += kBlock) {
        s_du[i] = 0;
        s_dp[i] = 0;
      }
    __syncthreads();
  }
  int cnt = 0, lev = 0;
  bool bad = false;
  if (g < N) {
    const float2 m = reinterpret_cast<const float2*>(mu)[g];      // (y, x)
    float2 s = reinterpret_cast<const float2*>(scale)[g];   // (sy, sx), or raw log-scales with act
    if (act) s = make_float2(activate_scale(s.x), activate_scale(s.y));
    float sn = 0.f, cs = 1.f;
    if (theta) {   // the float32 values nearest cos and sin of the float32 angle (double sincos, rounded once)
      double sd, cd;
      sincos((double)theta[g], &sd, &cd);
      sn = (float)sd;
      cs = (float)cd;
    }
    const float ky = kWhiten / s.x, kx = kWhiten / s.y;
    float4 col = make_float4(0.f, 0.f, 0.f, 0.f);
    col.x = color[(size_t)g * C];
    if (C > 1) col.y = color[(size_t)g * C + 1];
    if (C > 2) col.z = color[(size_t)g * C + 2];
    if (C > 3) col.w = color[(size_t)g * C + 3];
    const int t = threadIdx.x;
    s_rec[rec_slot(t, 0)] = make_float4(m.x, m.y, cs * ky, sn * ky);
    const float op = opacity[g];
    s_rec[rec_slot(t, 1)] = make_float4(-sn * kx, cs * kx, op, log2f(op));
    s_rec[rec_slot(t, 2)] = col;
    s_rec[rec_slot(t, 3)] = make_float4(s.x, s.y, cs, sn);
    if (do_bin) {
      // level: render_triton.py:925-932 + 950-952 (octave), :904-913 (coarse/fine split)
      if (R.mode == 1) {
        const float px = fmaxf(s.x, s.y) * R.rep;
        const float o = ceilf(log2f(fmaxf(px * R.inv_base, 1e-6f)));
        lev = (int)fminf(fmaxf(o, 0.f), (float)R.max_oct);
      } else if (R.mode == 2) {
        lev = g < R.n_coarse ? 1 : 0;
      }
      const float fH = (float)L.H[lev], fW = (float)L.W[lev];
      const float xmax = (float)(L.ntx[lev] - 1);
      const float ymax = (float)((L.tbase[lev + 1] - L.tbase[lev]) / L.ntx[lev] - 1);
      // render_triton.py:367-377, one rounding per operation.
      const float cx = m.y * fW;
      const float cy = m.x * fH;
      const float rr = cutoff * fmaxf(s.x, s.y);
      const float rx = rr * fW;
      const float ry = rr * fH;
      const int tx0 = (int)fminf(fmaxf(floorf((cx - rx) / fT), 0.f), xmax);
      const int tx1 = (int)fminf(fmaxf(floorf((cx + rx) / fT), 0.f), xmax);
      const int ty0 = (int)fminf(fmaxf(floorf((cy - ry) / fT), 0.f), ymax);
      const int ty1 = (int)fminf(fmaxf(floorf((cy + ry) / fT), 0.f), ymax);
      const int w = tx1 - tx0 + 1, h = ty1 - ty0 + 1;
      bad = (w < 1) || (h < 1);
      cnt = bad ? 0 : w * h;
      rect[g] = make_int4(tx0, ty0, w, lev);   // the rect height is not needed past this point
      counts[g] = cnt;
      if (cnt) {
        if (rowhist) {   // rows [r0, r0 + h) each get one unit of w pairs
          const int r0 = L.rbase[lev] + ty0;
          atomicAdd(&s_du[r0], 1);
          atomicAdd(&s_du[r0 + h], -1);
          atomicAdd(&s_dp[r0], w);
          atomicAdd(&s_dp[r0 + h], -w);
        }
      }
    }
  }
  if (do_bin) {   // per-level pair sums: one LDS atomic per level present in the wave (lanes of a level summed)
    const int lane = threadIdx.x & 63;
    for (unsigned long long rem = __ballot(cnt != 0); rem;) {
      const int l0 = __shfl(lev, __ffsll((long long)rem) - 1, 64);
      const unsigned long long m = __ballot(cnt != 0 && lev == l0);
      const int sum = wave_sum_i(((m >> lane) & 1ull) ? cnt : 0);
      if (lane == 0) atomicAdd(&s_lev[l0], sum);
      rem &= ~m;
    }
  }
  __syncthreads();
  {   // the block's records: 16 consecutive bytes per thread and store
    const int nrec = 4 * min(kBlock, N - (int)blockIdx.x * kBlock);
    float4* dst = rec + (size_t)blockIdx.x * kBlock * 4;
    for (int i = threadIdx.x; i < nrec; i += kBlock) dst[i] = s_rec[rec_slot(i >> 2, i & 3)];
  }
  if (!do_bin) return;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  long long v = cnt;
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) v += __shfl_xor(v, msk, 64);
  const bool any_bad = __any(bad);
  if (lane == 0) s_part[wv] = v | (any_bad ? kBadBit : 0);
  __syncthreads();
  if (threadIdx.x == 0) {
    long long t = 0, b = 0;
    for (int i = 0; i < kWaves; ++i) { t += s_part[i] & ~kBadBit; b |= s_part[i] & kBadBit; }
    block_sums[(size_t)blockIdx.x * kSumCols] = t | b;
  }
  if (threadIdx.x < kMaxLevels) block_sums[(size_t)blockIdx.x * kSumCols + 1 + threadIdx.x] = s_lev[threadIdx.x];
  if (!rowhist) return;
  // inclusive scan of the difference arrays over the rows: thread t takes rows [4 t, 4 t + 4); up to 256 rows
  // wave 0 alone (no barrier)
  static_assert(kMaxRows <= 4 * kBlock, "rows per thread");
  const bool one_wave = nrows <= 256;
  if (one_wave && wv != 0) return;
  __shared__ int s_w[kWaves];
  int du[4], dp[4], su = 0, sp = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = 4 * (int)threadIdx.x + k;
    du[k] = r < nrows ? s_du[r] : 0;
    dp[k] = r < nrows ? s_dp[r] : 0;
    su += du[k];
    sp += dp[k];
  }
  int pu, pp;
  if (one_wave) {
    pu = wave_incl_scan<int>(su, lane) - su;
    pp = wave_incl_scan<int>(sp, lane) - sp;
  } else {
    int t_u, t_p;
    pu = block256_excl<false>(su, s_w, t_u);
    pp = block256_excl<false>(sp, s_w, t_p);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = 4 * (int)threadIdx.x + k;
    pu += du[k];
    pp += dp[k];
    if (r < nrows) rowhist[(size_t)r * nb + blockIdx.x] = make_int2(pu, pp);
  }
}

// One entry of the count phase's totals, into `info` and, when the caller gave one, into its mirror in pinned
// host memory (a system-scope store: the host polls the mirror until every entry it preset has been written).
__device__ __forceinline__ void put_info(long long* info, long long* mirror, int i, long long v) {
  info[i] = v;
  if (mirror) __hip_atomic_store(mirror + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Exclusive scan of the per-block count sums in one workgroup. info[0] = total pairs, info[1] = error bits
// (1: empty/inverted rect, 2: total exceeds int32), info[2 + l] = pairs on level l < nlev (also into mirror).
__global__ __launch_bounds__(1024) void k_scan_sums(long long* __restrict__ sums, int n, int nlev,
                                                    long long* __restrict__ info, long long* __restrict__ mirror) {
  __shared__ long long s_w[16];
  __shared__ long long s_carry;
  __shared__ long long s_bad;
  __shared__ long long s_lev[kMaxLevels];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (threadIdx.x == 0) { s_carry = 0; s_bad = 0; }
  if (threadIdx.x < kMaxLevels) s_lev[threadIdx.x] = 0;
  __syncthreads();
  long long lev[kMaxLevels];
#pragma unroll
  for (int l = 0; l < kMaxLevels; ++l) lev[l] = 0;
  for (int base = 0; base < n; base += 1024) {
    const int i = base + threadIdx.x;
    long long v = i < n ? sums[(size_t)i * kSumCols] : 0;
    if (i < n) {
#pragma unroll
      for (int l = 0; l < kMaxLevels; ++l) lev[l] += sums[(size_t)i * kSumCols + 1 + l];
    }
    if (v & kBadBit) atomicOr((unsigned long long*)&s_bad, 1ull);
    v &= ~kBadBit;
    long long inc = wave_incl_scan(v, lane);
    if (lane == 63) s_w[wv] = inc;
    __syncthreads();
    if (threadIdx.x < 16) {
      long long x = s_w[threadIdx.x];
      for (int d = 1; d < 16; d <<= 1) {
        long long o = __shfl_up(x, d, 64);
        if ((int)threadIdx.x >= d) x += o;
      }
      s_w[threadIdx.x] = x;
    }
    __syncthreads();
    const long long carry = s_carry;
    const long long excl = carry + (wv ? s_w[wv - 1] : 0) + inc - v;
    if (i < n) sums[(size_t)i * kSumCols] = excl;
    __syncthreads();
    if (threadIdx.x == 0) s_carry = carry + s_w[15];
    __syncthreads();
  }
#pragma unroll
  for (int l = 0; l < kMaxLevels; ++l) {
    long long x = lev[l];
    for (int msk = 32; msk >= 1; msk >>= 1) x += __shfl_xor(x, msk, 64);
    if (lane == 0 && x) atomicAdd((unsigned long long*)&s_lev[l], (unsigned long long)x);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const long long tot = s_carry;
    put_info(info, mirror, 0, tot);
    put_info(info, mirror, 1, (s_bad ? 1 : 0) | (tot > 0x7fffffffLL - 64 ? 2 : 0));
  }
  if (threadIdx.x < nlev) put_info(info, mirror, 2 + threadIdx.x, s_lev[threadIdx.x]);
  if (mirror) __threadfence_system();
}

// counts -> exclusive offsets in place; offsets[N] = total. Block prefixes come from k_scan_sums.
__global__ __launch_bounds__(kBlock) void k_offsets(int* __restrict__ offsets, const long long* __restrict__ block_pre,
                                                    int N, const long long* __restrict__ info) {
  __shared__ int s_w[kWaves];
  const int g = blockIdx.x * kBlock + threadIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = g < N ? offsets[g] : 0;
  const int inc = wave_incl_scan(c, lane);
  if (lane == 63) s_w[wv] = inc;
  __syncthreads();
  int pre = 0;
  for (int i = 0; i < wv; ++i) pre += s_w[i];
  if (info[1] & 2) return;   // total overflows int32: the host raises, offsets are not used
  if (g < N) offsets[g] = (int)block_pre[(size_t)blockIdx.x * kSumCols] + pre + inc - c;
  if (g == N - 1) offsets[N] = (int)info[0];
}

// Row r of the row histogram (row plan): rowhist[r * nb + b].x, the units of row r in block b, becomes the
// exclusive prefix over the blocks before b; rtot[r] = (units, pairs) of row r over all blocks. 256 threads.
__device__ __forceinline__ void row_scan(int2* __restrict__ rowhist, int nb, int r, int2* __restrict__ rtot) {
  __shared__ int s_w[kWaves];
  __shared__ int s_wp[kWaves];
  int2* row = rowhist + (size_t)r * nb;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int carry = 0, pairs = 0;
  for (int base = 0; base < nb; base += kBlock * 8) {
    const int i0 = base + (int)threadIdx.x * 8;
    int v[8], sum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int2 e = i0 + k < nb ? row[i0 + k] : make_int2(0, 0);
      v[k] = e.x;
      sum += e.x;
      pairs += e.y;
    }
    int total;
    int run = carry + block256_excl<false>(sum, s_w, total);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (i0 + k < nb) row[i0 + k].x = run;
      run += v[k];
    }
    carry += total;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) pairs += __shfl_xor(pairs, m, 64);
  if (lane == 0) s_wp[wv] = pairs;
  __syncthreads();
  if (threadIdx.x == 0) rtot[r] = make_int2(carry, s_wp[0] + s_wp[1] + s_wp[2] + s_wp[3]);
}

__global__ __launch_bounds__(kBlock) void k_row_scan(int2* __restrict__ rowhist, int nb, int2* __restrict__ rtot) {
  row_scan(rowhist, nb, blockIdx.x, rtot);
}

// counts -> exclusive offsets in place without a separate scan launch (for up to kFusedScanBlocks blocks):
// every block sums its predecessors' block totals itself (L2-resident, at most a few thousand loads per
// block). The last block also writes info (and its mirror): total pairs, error bits and the per-level totals
// (l < nlev). With rowhist, workgroups nb, nb + 1, ... scan the row plan's histogram rows (row_scan).
constexpr int kFusedScanBlocks = 4096;

__global__ __launch_bounds__(kBlock) void k_offsets_fused(int* __restrict__ offsets,
                                                          const long long* __restrict__ sums, int N, int nb,
                                                          int nlev, long long* __restrict__ info,
                                                          long long* __restrict__ mirror, int2* __restrict__ rowhist,
                                                          int2* __restrict__ rtot) {
  if ((int)blockIdx.x >= nb) {   // the row plan's histogram rows, one workgroup each, in the same launch
    row_scan(rowhist, nb, blockIdx.x - nb, rtot);
    return;
  }
  __shared__ long long s_r[kWaves];
  __shared__ long long s_lev[kMaxLevels];
  __shared__ int s_w[kWaves];
  __shared__ int s_bad;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int blk = blockIdx.x;
  const bool last = blk == nb - 1;
  if (threadIdx.x == 0) s_bad = 0;
  if (threadIdx.x < kMaxLevels) s_lev[threadIdx.x] = 0;
  // every global load up front (one round trip): the splat's count, and the prefix over predecessors (all
  // blocks for the last one, to get the total, the error bits and the per-level totals)
  const int g = blk * kBlock + threadIdx.x;
  const int c = g < N ? offsets[g] : 0;
  long long acc = 0, lev[kMaxLevels];
#pragma unroll
  for (int l = 0; l < kMaxLevels; ++l) lev[l] = 0;
  int bad = 0;
  const int upto = last ? nb : blk;
  for (int b = threadIdx.x; b < upto; b += kBlock) {
    const long long v = sums[(size_t)b * kSumCols];
    if (b < blk) acc += v & ~kBadBit;
    bad |= (v & kBadBit) ? 1 : 0;
    if (last) {
#pragma unroll
      for (int l = 0; l < kMaxLevels; ++l)
        if (l < nlev) lev[l] += sums[(size_t)b * kSumCols + 1 + l];
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (lane == 0) s_r[wv] = acc;
  __syncthreads();
  if (bad) atomicOr(&s_bad, 1);
  long long pre_blk = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) pre_blk += s_r[w];
  const int inc = wave_incl_scan(c, lane);
  if (lane == 63) s_w[wv] = inc;
  __syncthreads();
  int pre = 0, btot = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    if (i < wv) pre += s_w[i];
    btot += s_w[i];
  }
  if (g < N) offsets[g] = (int)(pre_blk + pre + inc - c);   // garbage only when the total overflows int32
  if (!last) return;
  const long long tot = pre_blk + btot;
  if (g == N - 1) offsets[N] = (int)tot;
#pragma unroll
  for (int l = 0; l < kMaxLevels; ++l) {
    if (l >= nlev) break;
    long long x = lev[l];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
    if (lane == 0 && x) atomicAdd((unsigned long long*)&s_lev[l], (unsigned long long)x);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    put_info(info, mirror, 0, tot);
    put_info(info, mirror, 1, (s_bad ? 1 : 0) | (tot > 0x7fffffffLL - 64 ? 2 : 0));
  }
  if (threadIdx.x < nlev) put_info(info, mirror, 2 + threadIdx.x, s_lev[threadIdx.x]);
  if (mirror) __threadfence_system();
}

// Pair count of a pair-phase launch. With `info` (a launch queued before the host has read the count,
// sized for `cap` pairs): the count written by the count phase, or 0 when it exceeds cap or the count phase
// flagged an error (the launch then leaves an empty pair list and the host redoes the pair phase).
// Without `info`: cap is the count.
__device__ __forceinline__ int pair_count(const long long* __restrict__ info, int cap) {
  if (!info) return cap;
  const long long t = info[0];
  return (t > cap || (info[1] & 3)) ? 0 : (int)t;
}

// Quotient of k >= 0 by w >= 1: a float estimate (within one of the quotient while k < 2^24), corrected to
// the exact integer quotient.
__device__ __forceinline__ int div_rect(int k, int w) {
  int q = (int)((float)k * __builtin_amdgcn_rcpf((float)w));
  while (q > 0 && q * w > k) --q;
  while ((q + 1) * w <= k) ++q;
  return q;
}

// ----------------------------------------------------------------------------------------------------
// pair expansion (render_triton.py:396-404): pair p belongs to the last splat g with offsets[g] <= p, and
// k = p - offsets[g] walks that splat's rect row by row.
__device__ __forceinline__ int last_le(const int* __restrict__ a, int lo, int hi, int p) {
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a[mid] <= p) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Block-cooperative last_le over a[0, n): 1024 samples per round (4 per thread) narrow the bracket
// 1024-fold, so the search costs ceil(log1024 n) rounds of independent loads instead of log2 n dependent
// loads. Requires a[0] <= p. Every thread must call it; all get the result.
__device__ __forceinline__ int block_last_le(const int* __restrict__ a, int n, int p, int* s_w) {
  constexpr int S = kBlock * 4;
  int lo = 0, hi = n - 1;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  while (hi > lo) {
    const int step = (hi - lo + S) / S;                      // ceil((hi - lo + 1) / S)
    int cnt_t = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {                            // sample j = 4 t + k at lo + j * step
      const int idx = lo + ((int)threadIdx.x * 4 + k) * step;
      cnt_t += (idx <= hi && a[idx] <= p) ? 1 : 0;           // true for a prefix of the samples (j = 0 always)
    }
    int c = cnt_t;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) c += __shfl_xor(c, m, 64);
    if (lane == 0) s_w[wv] = c;
    __syncthreads();
    int cnt = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) cnt += s_w[w];
    __syncthreads();
    const int nlo = lo + (cnt - 1) * step;
    hi = min(hi, nlo + step - 1);
    lo = nlo;
  }
  return lo;
}


// Block = kSortKeys consecutive pairs. Each splat with pairs in the block marks its first pair there with its
// id; an inclusive max-scan over the block then gives every pair its owner (splat ids grow with p).
// The block's first splat comes from a cooperative search; when the block holds at most kBlock splats
// (always at a few pairs per splat or more) their offsets and rects are loaded once, one per thread, into
// LDS, and the pair loop reads only LDS. Writes keys[p] = tile, pair_splat[p] = splat and the block's
// histogram of the first radix digit, (tile >> shift) & dmask.
__global__ __launch_bounds__(kBlock) void k_scatter_pairs(const int4* __restrict__ rect, const int* __restrict__ offsets,
                                                          int N, LevelTable L, const long long* __restrict__ info,
                                                          int cap, int shift, int dmask, int* __restrict__ keys,
                                                          int* __restrict__ pair_splat, int* __restrict__ hist,
                                                          int nblocks) {
  __shared__ int4 s_own4[kSortKeys / 4];
  __shared__ int4 s_rect[kBlock];
  __shared__ int s_o0[kBlock];
  __shared__ int s_hist[kMaxRadix];
  __shared__ int s_w[kWaves];
  int* s_own = reinterpret_cast<int*>(s_own4);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int tot = pair_count(info, cap);
  const int p_base = blockIdx.x * kSortKeys;
  if (p_base >= tot) {   // a block past the pairs of this launch: an empty histogram column
    for (int d = threadIdx.x; d <= dmask; d += kBlock) hist[d * nblocks + blockIdx.x] = 0;
    return;
  }
  const int n_here = min(kSortKeys, tot - p_base);
  const int p_last = p_base + n_here - 1;
  for (int i = threadIdx.x; i <= dmask; i += kBlock) s_hist[i] = 0;
  for (int i = threadIdx.x; i < kSortKeys / 4; i += kBlock) s_own4[i] = make_int4(-1, -1, -1, -1);
  const int glo = block_last_le(offsets, N, p_base, s_w);
  // window of the next kBlock splats: offsets and rect, one per thread
  const int gw = glo + (int)threadIdx.x;
  int o0 = 0x7fffffff, o1 = 0x7fffffff;
  int4 rw = make_int4(0, 0, 1, 0);
  if (gw < N) {
    o0 = offsets[gw];
    o1 = offsets[gw + 1];
    rw = rect[gw];
  }
  const bool in_win = o0 <= p_last;   // prefix of the threads
  {
    const unsigned long long m = __ballot(in_win);
    if (lane == 0) s_w[wv] = __popcll(m);
  }
  s_o0[threadIdx.x] = o0;
  s_rect[threadIdx.x] = rw;
  __syncthreads();
  int cnt = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) cnt += s_w[w];
  // the window covers the block unless all kBlock splats start in it and more may follow
  const bool fast = cnt < kBlock || glo + kBlock >= N;
  __syncthreads();
  if (fast) {
    if (in_win && o1 > o0) atomicMax(&s_own[max(o0, p_base) - p_base], gw);
  } else {
    const int ghi = block_last_le(offsets, N, p_last, s_w);
    for (int g = glo + (int)threadIdx.x; g <= ghi; g += kBlock) {
      const int a0 = offsets[g], a1 = offsets[g + 1];
      if (a1 > a0) atomicMax(&s_own[max(a0, p_base) - p_base], g);   // a0 <= offsets[ghi] <= last pair here
    }
  }
  __syncthreads();
  {
    // thread t scans entries [8 t, 8 t + 8)
    int loc[8];
    int run = -1;
#pragma unroll
    for (int k4 = 0; k4 < 2; ++k4) {
      const int4 x = s_own4[threadIdx.x * 2 + k4];
      run = max(run, x.x); loc[4 * k4 + 0] = run;
      run = max(run, x.y); loc[4 * k4 + 1] = run;
      run = max(run, x.z); loc[4 * k4 + 2] = run;
      run = max(run, x.w); loc[4 * k4 + 3] = run;
    }
    int total;
    const int ex = block256_excl<true>(run, s_w, total);
#pragma unroll
    for (int k4 = 0; k4 < 2; ++k4)
      s_own4[threadIdx.x * 2 + k4] = make_int4(max(loc[4 * k4], ex), max(loc[4 * k4 + 1], ex),
                                               max(loc[4 * k4 + 2], ex), max(loc[4 * k4 + 3], ex));
  }
  __syncthreads();
  // The histogram adds runs: consecutive lanes with equal digits (a splat's tiles along a rect row) count in
  // one LDS atomic by the run's first lane.
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int i = wv * kWaveKeys + j * 64 + lane;
    const bool act = i < n_here;
    int d = -1;
    if (act) {
      const int p = p_base + i;
      const int g = s_own[i];
      int k;
      int4 rc;
      if (fast) {
        k = p - s_o0[g - glo];
        rc = s_rect[g - glo];
      } else {
        k = p - offsets[g];
        rc = rect[g];
      }
      const int ky = div_rect(k, rc.z);
      const int kx = k - ky * rc.z;
      const int tile = L.tbase[rc.w] + (rc.y + ky) * L.ntx[rc.w] + rc.x + kx;
      keys[p] = tile;
      pair_splat[p] = g;
      d = (tile >> shift) & dmask;
    }
    const int dprev = __shfl_up(d, 1, 64);
    const bool brk = !act || lane == 0 || dprev != d;   // a run starts here (inactive lanes: the tail)
    const unsigned long long bound = __ballot(brk);
    if (act && brk) {
      const unsigned long long after = bound & ~((2ull << lane) - 1ull);
      atomicAdd(&s_hist[d], (after ? __builtin_ctzll(after) : 64) - lane);
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d <= dmask; d += kBlock) hist[d * nblocks + blockIdx.x] = s_hist[d];
}

__global__ __launch_bounds__(kBlock) void k_radix_hist(const int* __restrict__ keys, const long long* __restrict__ info,
                                                       int cap, int shift, int dmask, int* __restrict__ hist,
                                                       int nblocks) {
  __shared__ int s_hist[kMaxRadix];
  const int tot = pair_count(info, cap);
  for (int i = threadIdx.x; i <= dmask; i += kBlock) s_hist[i] = 0;
  __syncthreads();
  const int p_base = blockIdx.x * kSortKeys;
  int kv[kItems];
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int p = p_base + j * kBlock + threadIdx.x;
    kv[j] = p < tot ? keys[p] : -1;
  }
#pragma unroll
  for (int j = 0; j < kItems; ++j)
    if (kv[j] >= 0) atomicAdd(&s_hist[(kv[j] >> shift) & dmask], 1);
  __syncthreads();
  for (int d = threadIdx.x; d <= dmask; d += kBlock) hist[d * nblocks + blockIdx.x] = s_hist[d];
}

// Workgroup d scans histogram row d (the counts of digit d in every block) in place into exclusive
// per-block offsets within the digit, and stores the digit's total in rowtot[d].
__global__ __launch_bounds__(kBlock) void k_hist_row_scan(int* __restrict__ hist, int nblocks, int* __restrict__ rowtot) {
  __shared__ int s_w[kWaves];
  int* row = hist + (size_t)blockIdx.x * nblocks;
  int carry = 0;
  for (int base = 0; base < nblocks; base += kBlock * 8) {
    const int i0 = base + threadIdx.x * 8;
    int v[8], sum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) { v[k] = i0 + k < nblocks ? row[i0 + k] : 0; sum += v[k]; }
    int total;
    int run = carry + block256_excl<false>(sum, s_w, total);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (i0 + k < nblocks) row[i0 + k] = run;
      run += v[k];
    }
    carry += total;
  }
  if (threadIdx.x == 0) rowtot[blockIdx.x] = carry;
}

// Stable scatter of one radix pass. Wave w of the block owns keys [base + w*512, base + (w+1)*512) and
// walks them 64 at a time in index order; lanes holding the same digit are ranked among themselves with
// ballots (lane order = index order), on top of the wave's running count for that digit. The block's keys
// are then placed in LDS in (digit, index) order and written out by consecutive threads, so each digit's
// run of the block lands in consecutive global positions: the digit's global start (prefix of the row
// totals) plus the block's offset within the digit (the row-scanned histogram).
// Values moved with each key: the splat id (vals) and, with q_out set, the pair's splat-major index (q_in, or
// the key's input position when q_in is null: the first pass reads the splat-major list).
// DPT digits per thread in the per-digit steps: radix up to 256 DPT (DPT = 2 for 9-bit digits). The keys are
// loaded first, so their memory round trip overlaps the loads of the digit totals and offsets.
template <int DPT>
__global__ __launch_bounds__(kBlock) void k_radix_scatter(const int* __restrict__ keys_in, const int* __restrict__ vals_in,
                                                          const int* __restrict__ q_in,
                                                          const long long* __restrict__ info, int cap, int shift,
                                                          int dbits, const int* __restrict__ hist_scan,
                                                          const int* __restrict__ rowtot, int nblocks,
                                                          int* __restrict__ keys_out, int* __restrict__ vals_out,
                                                          int* __restrict__ q_out) {
  constexpr int MAXR = 256 * DPT;
  __shared__ int s_cnt[kWaves][MAXR];
  __shared__ int s_gbase[MAXR];    // global position of the block's first key with digit d
  __shared__ int s_lbase[MAXR];    // LDS position of the block's first key with digit d
  __shared__ int s_key[kSortKeys];
  __shared__ int s_val[kSortKeys];
  __shared__ int s_q[kSortKeys];
  __shared__ int s_w[kWaves];
  const int dmask = (1 << dbits) - 1;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int tot = pair_count(info, cap);
  if ((int)blockIdx.x * kSortKeys >= tot) return;   // no keys here (uniform: before any barrier)
  const int p_base = blockIdx.x * kSortKeys;
  const int n_here = min(kSortKeys, tot - p_base);
  const int p0 = p_base + wv * kWaveKeys + lane;
  int key[kItems], val[kItems], qv[kItems], rank[kItems];
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int p = p0 + j * 64;
    const bool act = p < tot;
    key[j] = act ? keys_in[p] : 0;
    val[j] = act ? vals_in[p] : 0;
    qv[j] = q_out ? (q_in ? (act ? q_in[p] : 0) : p) : 0;
  }
  for (int i = threadIdx.x; i < kWaves * MAXR; i += kBlock) (&s_cnt[0][0])[i] = 0;
  {
    // thread t: digits DPT t ... DPT t + DPT - 1
    int rt[DPT], hs[DPT], sum = 0;
#pragma unroll
    for (int k = 0; k < DPT; ++k) {
      const int d = DPT * (int)threadIdx.x + k;
      rt[k] = d <= dmask ? rowtot[d] : 0;
      hs[k] = d <= dmask ? hist_scan[d * nblocks + blockIdx.x] : 0;
      sum += rt[k];
    }
    int total;
    int dstart = block256_excl<false>(sum, s_w, total);
#pragma unroll
    for (int k = 0; k < DPT; ++k) {
      const int d = DPT * (int)threadIdx.x + k;
      if (d <= dmask) s_gbase[d] = dstart + hs[k];
      dstart += rt[k];
    }
  }
  __syncthreads();
  const unsigned long long lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const bool act = p0 + j * 64 < tot;
    const int d = (key[j] >> shift) & dmask;
    unsigned long long peers = __ballot(act);
    for (int b = 0; b < dbits; ++b) {
      const bool bit = (d >> b) & 1;
      const unsigned long long m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int below = __popcll(peers & lt);
    const int before = s_cnt[wv][d];
    if (act && below == 0) s_cnt[wv][d] = before + __popcll(peers);
    rank[j] = before + below;
  }
  __syncthreads();
  {
    // per digit: wave offsets within the block's run of that digit, and the run's LDS start
    int run[DPT], sum = 0;
#pragma unroll
    for (int k = 0; k < DPT; ++k) {
      const int d = DPT * (int)threadIdx.x + k;
      run[k] = 0;
      if (d <= dmask)
        for (int w = 0; w < kWaves; ++w) { const int c = s_cnt[w][d]; s_cnt[w][d] = run[k]; run[k] += c; }
      sum += run[k];
    }
    int total;
    int lstart = block256_excl<false>(sum, s_w, total);
#pragma unroll
    for (int k = 0; k < DPT; ++k) {
      const int d = DPT * (int)threadIdx.x + k;
      if (d <= dmask) s_lbase[d] = lstart;
      lstart += run[k];
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    if (p0 + j * 64 >= tot) continue;
    const int d = (key[j] >> shift) & dmask;
    const int lpos = s_lbase[d] + s_cnt[wv][d] + rank[j];
    s_key[lpos] = key[j];
    s_val[lpos] = val[j];
    if (q_out) s_q[lpos] = qv[j];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n_here; i += kBlock) {
    const int k = s_key[i];
    const int d = (k >> shift) & dmask;
    const int pos = s_gbase[d] + (i - s_lbase[d]);
    keys_out[pos] = k;
    vals_out[pos] = s_val[i];
    if (q_out) q_out[pos] = s_q[i];
  }
}

// Second phase of the two-phase sort: workgroup s takes super-tile s, the tiles [s R, s R + R) with R = 2^lb,
// whose pairs [sb, se) a radix pass on tile >> lb has put together in splat-major order (sb = sum of rowtot
// over the super-tiles before s). A stable counting sort on the low lb bits of the tile puts them in (tile,
// splat) order: gid_sorted / pair_q (when given) at [sb, se), and tile_starts of its tiles (render_triton.py:
// 405-408). The pairs go in rounds of kLocalKeys: wave w holds 512 consecutive ones (loaded at once) and ranks
// them 64 at a time, equal digits by ballots on top of its running counts; the waves' counts are scanned per
// digit in wave order (16 lanes per digit). The round is staged in LDS in (digit, index) order and written
// out by consecutive threads, so every digit's run of the round lands in consecutive positions. A super-tile
// of one round takes its digit histogram from the round's counts (its output is then one contiguous run); a
// larger one counts its digits first (LDS atomics).
constexpr int kLocalThreads = 1024;
constexpr int kLocalWaves = kLocalThreads / 64;
constexpr int kLocalWaveKeys = 512;
constexpr int kLocalKeys = kLocalWaves * kLocalWaveKeys;
constexpr int kLocalMaxBits = 5;

__global__ __launch_bounds__(kLocalThreads) void k_local_sort(const int* __restrict__ keys, const int* __restrict__ vals,
                                                              const int* __restrict__ q_in,
                                                              const long long* __restrict__ info, int cap, int lb,
                                                              int nt, int nsuper, const int* __restrict__ rowtot,
                                                              int* __restrict__ gid_sorted, int* __restrict__ pair_q,
                                                              int* __restrict__ tile_starts) {
  constexpr int RM = 1 << kLocalMaxBits;
  constexpr int J = kLocalWaveKeys / 64;
  static_assert(kLocalWaves == 16 && RM * kLocalWaves <= kLocalThreads, "digit scan layout");
  __shared__ int s_part[kLocalWaves];
  __shared__ int s_dig[RM];    // start of digit d within the super-tile, plus its pairs in earlier rounds
  __shared__ int s_rt[RM];     // the round's pairs of digit d
  __shared__ int s_lst[RM];    // LDS start of digit d's run in the round
  __shared__ int s_gb[RM];     // start of the round's digit-d run within the super-tile
  __shared__ int s_cnt[kLocalWaves][RM];
  __shared__ int s_g[kLocalKeys];
  __shared__ int s_q[kLocalKeys];
  __shared__ unsigned char s_d[kLocalKeys];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int s = blockIdx.x;
  const int R = 1 << lb;
  const int tot = pair_count(info, cap);
  // sb = sum of rowtot[0, s) (s < 512 <= kLocalThreads: one load per thread)
  const int mine = (tot > 0 && (int)threadIdx.x < s) ? rowtot[threadIdx.x] : 0;
  const int cnt_s = tot > 0 ? rowtot[s] : 0;
  const int part = wave_sum_i(mine);
  if (lane == 0) s_part[wv] = part;
  if (threadIdx.x < RM) s_dig[threadIdx.x] = 0;
  __syncthreads();
  int sb = 0;
#pragma unroll
  for (int w = 0; w < kLocalWaves; ++w) sb += s_part[w];
  const int se = sb + cnt_s;
  const bool one_round = cnt_s <= kLocalKeys;
  if (s == nsuper - 1 && threadIdx.x == 0) {
    tile_starts[nt] = tot;
    if (tot == 0) gid_sorted[0] = 0;   // empty list: gid_sorted = {0} (render_triton.py:392-394)
  }
  if (!one_round) {   // the super-tile's digit histogram first, kLocalKeys keys per step
    for (int rb = sb; rb < se; rb += kLocalKeys) {
      int kv[J];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int i = rb + j * kLocalThreads + (int)threadIdx.x;
        kv[j] = i < se ? keys[i] : -1;
      }
#pragma unroll
      for (int j = 0; j < J; ++j)
        if (kv[j] >= 0) atomicAdd(&s_dig[kv[j] & (R - 1)], 1);
    }
    __syncthreads();
    if (wv == 0) {
      const int h = lane < RM ? s_dig[lane] : 0;
      const int ex = wave_incl_scan<int>(h, lane) - h;
      if (lane < R) {
        s_dig[lane] = ex;
        if (s * R + lane < nt) tile_starts[s * R + lane] = sb + ex;
      }
    }
  }
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int rb = sb; rb < se || (one_round && rb == sb); rb += kLocalKeys) {
    const int i0 = rb + wv * kLocalWaveKeys + lane;
    const int n_round = min(kLocalKeys, se - rb);
    int dg[J], rank[J], gv[J], qv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int i = i0 + j * 64;
      const bool act = i < se;
      dg[j] = act ? keys[i] & (R - 1) : 0;
      gv[j] = act ? vals[i] : 0;
      qv[j] = (act && pair_q) ? q_in[i] : 0;
    }
    if (threadIdx.x < kLocalWaves * RM) (&s_cnt[0][0])[threadIdx.x] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const bool act = i0 + j * 64 < se;
      const int d = dg[j];
      unsigned long long peers = __ballot(act);
      for (int b = 0; b < lb; ++b) {
        const bool bit = (d >> b) & 1;
        const unsigned long long m = __ballot(bit);
        peers &= bit ? m : ~m;
      }
      const int below = __popcll(peers & lt);
      const int before = s_cnt[wv][d];
      if (act && below == 0) s_cnt[wv][d] = before + __popcll(peers);
      rank[j] = before + below;
    }
    __syncthreads();
    if (threadIdx.x < kLocalWaves * RM) {   // digit d = t / 16, wave w = t % 16: wave offsets in wave order
      const int d = threadIdx.x >> 4, w = threadIdx.x & 15;
      const int c = s_cnt[w][d];
      int inc = c;
#pragma unroll
      for (int k = 1; k < 16; k <<= 1) {
        const int o = __shfl_up(inc, k, 16);
        if (w >= k) inc += o;
      }
      s_cnt[w][d] = inc - c;
      if (w == 15) s_rt[d] = inc;
    }
    __syncthreads();
    if (wv == 0) {   // lane d: LDS start of the digit's run, its place in the super-tile
      const int d = lane;
      const int rt = d < R ? s_rt[d] : 0;
      const int lst = wave_incl_scan<int>(rt, lane) - rt;
      if (d < R) {
        if (one_round) {   // the round is the whole super-tile: its counts are the histogram
          s_dig[d] = lst;
          if (s * R + d < nt) tile_starts[s * R + d] = sb + lst;
        }
        s_lst[d] = lst;
        s_gb[d] = s_dig[d];
        s_dig[d] += rt;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (i0 + j * 64 >= se) continue;
      const int d = dg[j];
      const int lpos = s_lst[d] + s_cnt[wv][d] + rank[j];
      s_g[lpos] = gv[j];
      s_q[lpos] = qv[j];
      s_d[lpos] = (unsigned char)d;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n_round; i += kLocalThreads) {
      const int d = s_d[i];
      const int pos = sb + s_gb[d] + (i - s_lst[d]);
      gid_sorted[pos] = s_g[i];
      if (pair_q) pair_q[pos] = s_q[i];
    }
    __syncthreads();
  }
}

// From the sorted tile ids: CSR starts, starts[t] = number of pairs with tile < t (render_triton.py:408).
// Thread = tile: a lower-bound binary search over the sorted keys, so runs of empty tiles cost nothing extra
// (threads of neighbouring tiles walk the same first probes, which stay in cache).
__global__ __launch_bounds__(kBlock) void k_tile_starts(const int* __restrict__ keys, int* __restrict__ gids,
                                                        const long long* __restrict__ info, int cap, int nt,
                                                        int* __restrict__ starts) {
  const int t = blockIdx.x * kBlock + threadIdx.x;
  if (t > nt) return;
  const int tot = pair_count(info, cap);
  if (tot == 0) {   // empty list: all starts 0 and gid_sorted = {0} (render_triton.py:392-394)
    starts[t] = 0;
    if (t == 0) gids[0] = 0;
    return;
  }
  int lo = 0, hi = tot;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (keys[mid] < t) lo = mid + 1; else hi = mid;
  }
  starts[t] = lo;
}

__global__ void k_fill_i32(int* __restrict__ a, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) a[i] = v;
}

// ---------------------------------------------------------------------------------------------- row plan
// Pair phase of the row plan (level tables of at most kMaxRows tile rows). A unit is one splat x one tile row
// of its rect: units are 4-5x fewer than pairs at the benchmark size. The pairs of tile row r in (tile, splat)
// order are the row's units in splat order, expanded column by column; so the sort is a stable partition of
// the units by row (k_scatter_units, from the decode pass's per-block row histogram), and the per-row
// expansion (k_expand_row) writes the pair list, the maps and the CSR starts of the row's tiles.
// Unit arrays (index = position in row-major, splat-ascending order): ug = splat, uq = splat-major index of
// the unit's first pair (offsets[g] + k w for the splat's k-th row), uspan = tx0 | w << 16.

// Stable scatter of the units of block `blockIdx.x` (the decode pass's 256 splats) to their row's range:
// position = first unit of row r (prefix of the row totals) + the block's offset within row r (the scanned
// histogram) + the unit's rank among the block's units of row r in splat order. The block's units are
// walked in splat order, kSortKeys per round: wave w ranks units [512 w, 512 w + 512) of the round 64 at a
// time, equal rows by ballots on top of the wave's running counts; the waves' counts are scanned per row.
__global__ __launch_bounds__(kBlock) void k_scatter_units(const int4* __restrict__ rect, const int* __restrict__ offsets,
                                                          int N, LevelTable L, const long long* __restrict__ info,
                                                          int cap, const int2* __restrict__ rowhist,
                                                          const int2* __restrict__ rtot, int nb, int* __restrict__ ug,
                                                          int* __restrict__ uq, int* __restrict__ uspan) {
  __shared__ int s_own[kSortKeys];
  __shared__ int s_u0[kBlock], s_r0[kBlock], s_q0[kBlock], s_span[kBlock];
  __shared__ int s_cnt[kWaves * kMaxRows];   // [wave][row - rmin]
  __shared__ int s_base[kMaxRows];            // [row]: where the block's next unit of the row goes
  __shared__ int s_w[kWaves];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int blk = blockIdx.x;
  const int t = threadIdx.x;
  const int g = blk * kBlock + t;
  const int nrows = L.rbase[L.n];
  // every global load of the block up front (one round trip): the splat's rect and offsets, and rows
  // [4 t, 4 t + 4) of the row totals and of the block's column of the scanned row histogram
  int4 rc = make_int4(0, 0, 0, 0);
  int q0 = 0, q1 = 0;
  if (g < N) {
    rc = rect[g];
    q0 = offsets[g];
    q1 = offsets[g + 1];
  }
  int rt[4], rh[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = 4 * t + k;
    rt[k] = r < nrows ? rtot[r].x : 0;
    rh[k] = r < nrows ? rowhist[(size_t)r * nb + blk].x : 0;
  }
  const int tot = pair_count(info, cap);
  if (tot == 0) return;   // no pairs, or a speculative launch past its capacity: no units to place
  int h = 0, r0 = nrows, r1 = -1, span = 0, w = 1;
  if (g < N) {
    const int cnt = q1 - q0;
    if (cnt > 0 && rc.z > 0) {
      w = rc.z;
      h = cnt / w;
      r0 = L.rbase[rc.w] + rc.y;
      r1 = r0 + h - 1;
      span = rc.x | (w << 16);
    }
  }
  // one barrier for: the block's row range [rmin, rmax] (block-uniform; a splat without units has r0 = nrows,
  // r1 = -1) and the first unit u0 of splat t within the block (exclusive prefix of h; nu = the block's total)
  int inc = h, mx = r1, mn = r0;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    mx = max(mx, __shfl_xor(mx, m, 64));
    mn = min(mn, __shfl_xor(mn, m, 64));
  }
  __shared__ int s_w3[3][kWaves];
  if (lane == 63) s_w3[0][wv] = inc;
  if (lane == 0) {
    s_w3[1][wv] = mx;
    s_w3[2][wv] = mn;
  }
  __syncthreads();
  int pre = 0, nu = 0, rmax = -1, rmin = nrows;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int x = s_w3[0][w];
    if (w < wv) pre += x;
    nu += x;
    rmax = max(rmax, s_w3[1][w]);
    rmin = min(rmin, s_w3[2][w]);
  }
  int ex = __shfl_up(inc, 1, 64);
  if (lane == 0) ex = 0;
  const int u0 = pre + ex;
  if (rmax < rmin) return;   // the block holds no units
  const int nr = rmax - rmin + 1;
  s_u0[t] = u0;
  s_r0[t] = r0;
  s_q0[t] = q0;
  s_span[t] = span;
  // first unit of every row: exclusive prefix of the row totals (rows [4 t, 4 t + 4) per thread)
  {
    const int sum = rt[0] + rt[1] + rt[2] + rt[3];
    int total;
    int run = block256_excl<false>(sum, s_w, total);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 4 * t + k;
      if (r >= rmin && r <= rmax) s_base[r] = run + rh[k];
      run += rt[k];
    }
  }
  int nbits = 0;
  while ((1 << nbits) < nr) ++nbits;
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int rb = 0; rb < nu; rb += kSortKeys) {
    for (int i = t; i < kSortKeys; i += kBlock) s_own[i] = -1;
    for (int i = t; i < kWaves * nr; i += kBlock) s_cnt[(i / nr) * kMaxRows + i % nr] = 0;
    __syncthreads();
    if (h > 0 && u0 < rb + kSortKeys && u0 + h > rb) s_own[max(u0, rb) - rb] = t;   // one splat per entry
    __syncthreads();
    {   // owner of every unit of the round: inclusive max-scan (thread t: entries [8 t, 8 t + 8))
      int loc[8], run = -1;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        run = max(run, s_own[8 * t + k]);
        loc[k] = run;
      }
      int total;
      const int ex = block256_excl<true>(run, s_w, total);
#pragma unroll
      for (int k = 0; k < 8; ++k) s_own[8 * t + k] = max(loc[k], ex);
    }
    __syncthreads();
    int rk[kItems], rr[kItems], own[kItems], kk[kItems];
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
      const int i = wv * kWaveKeys + j * 64 + lane;
      const bool act = rb + i < nu;
      const int o = act ? s_own[i] : 0;
      const int k = act ? rb + i - s_u0[o] : 0;
      const int r = act ? s_r0[o] + k - rmin : 0;
      unsigned long long peers = __ballot(act);
      for (int b = 0; b < nbits; ++b) {
        const bool bit = (r >> b) & 1;
        const unsigned long long m = __ballot(bit);
        peers &= bit ? m : ~m;
      }
      const int below = __popcll(peers & lt);
      const int before = act ? s_cnt[wv * kMaxRows + r] : 0;
      if (act && below == 0) s_cnt[wv * kMaxRows + r] = before + __popcll(peers);
      rk[j] = before + below;
      rr[j] = act ? r : -1;
      own[j] = o;
      kk[j] = k;
    }
    __syncthreads();
    for (int r = t; r < nr; r += kBlock) {   // per row: the waves' starts, in wave order
      int run = s_base[rmin + r];
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        const int c = s_cnt[ww * kMaxRows + r];
        s_cnt[ww * kMaxRows + r] = run;
        run += c;
      }
      s_base[rmin + r] = run;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
      if (rr[j] < 0) continue;
      const int pos = s_cnt[wv * kMaxRows + rr[j]] + rk[j];
      const int o = own[j];
      const int sp = s_span[o];
      if ((unsigned)pos < (unsigned)cap) {
        ug[pos] = blk * kBlock + o;
        uq[pos] = s_q0[o] + kk[j] * (sp >> 16);
        uspan[pos] = sp;
      }
    }
    __syncthreads();
  }
}

// One workgroup of kRowThreads per tile row and chunk of at most kRowCols tile columns (blockIdx.y = global
// row r, blockIdx.x = chunk of cw columns). Counting: the spans of the row's units (kRowUnits per round) give
// the row's pairs before c0 and a difference array over the chunk's columns (LDS atomics), so the chunk's tile
// starts follow. Writing: the units meeting the chunk are listed in LDS in unit order (their index and span),
// their splat ids and splat-major indices gathered for the listed units only, then each wave owns the columns
// j = wave, wave + 8, ...: it walks the list 64 units at a time and, per column, the units covering it (one
// ballot) are that tile's next pairs in splat order, written by consecutive lanes at the column's running
// position (in registers for chunks of up to 32 columns, else in LDS). Spans are read kRowHold rounds
// at a time. A row of at most kRowHold rounds has its spans read once and held in registers, and the lists of
// all its rounds are gathered together while they fit the list: three dependent global round trips for the
// whole row (row totals, spans, gather). Longer rows read their spans twice (counting, then writing).
constexpr int kRowThreads = 512;
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kRowItems = 4;                          // units per thread and round
constexpr int kRowUnits = kRowThreads * kRowItems;   // 2048 units per round
constexpr int kRowCols = 128;                         // columns per chunk, at most
constexpr int kRowHold = 4;                           // rounds whose spans stay in registers
constexpr int kRowList = 2048;                        // units meeting the chunk listed at once, at most
static_assert(kRowList >= kRowUnits, "a round fits the list");

// CPW > 0 (chunks of at most CPW columns per wave): each wave keeps its columns' running positions in
// registers; CPW = 0: in LDS (s_diff), read and advanced by the owning wave.
template <int CPW>
__global__ __launch_bounds__(kRowThreads) void k_expand_row(LevelTable L, const long long* __restrict__ info, int cap,
                                                            const int2* __restrict__ rtot, int cw,
                                                            const int* __restrict__ ug, const int* __restrict__ uq,
                                                            const int* __restrict__ uspan, int* __restrict__ gid_sorted,
                                                            int* __restrict__ tile_starts, int* __restrict__ pair_splat,
                                                            int* __restrict__ pair_q) {
  __shared__ int s_cu[kRowList], s_cs[kRowList];   // listed units: index (then splat id), span
  __shared__ int s_cq[kRowList];                   // listed units: splat-major index of the first pair
  __shared__ int s_diff[kRowCols + 1];   // difference array, then per column its running position
  __shared__ int s_kc[kRowItems][kRowWaves];
  __shared__ int s_red[3][kRowWaves];
  __shared__ int s_n;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int t = threadIdx.x;
  const int r = blockIdx.y;
  const int l = level_of_row(L, r);
  const int ntx = L.ntx[l];
  const int c0 = blockIdx.x * cw;
  if (c0 >= ntx) return;
  const int c1 = min(c0 + cw, ntx), ncol = c1 - c0;
  const int tile0 = L.tbase[l] + (r - L.rbase[l]) * ntx + c0;
  const int nt = L.tbase[L.n];
  // units and pairs of the rows before r and of row r (loaded before the pair count is known: one round trip)
  int us = 0, pr = 0;
  for (int i = t; i < r; i += kRowThreads) {
    const int2 e = rtot[i];
    us += e.x;
    pr += e.y;
  }
  const int row_units = rtot[r].x;
  const int tot = pair_count(info, cap);
  if (tot == 0) {   // no pairs (or a speculative launch past its capacity): the empty list
    if (t < ncol) tile_starts[tile0 + t] = 0;
    if (r == 0 && c0 == 0 && t == 0) {
      tile_starts[nt] = 0;
      gid_sorted[0] = 0;
    }
    return;
  }
  if (r == 0 && c0 == 0 && t == 0) tile_starts[nt] = tot;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    us += __shfl_xor(us, m, 64);
    pr += __shfl_xor(pr, m, 64);
  }
  if (lane == 0) {
    s_red[0][wv] = us;
    s_red[1][wv] = pr;
  }
  if (t <= kRowCols) s_diff[t] = 0;
  __syncthreads();
  us = 0;
  pr = 0;
#pragma unroll
  for (int w = 0; w < kRowWaves; ++w) {
    us += s_red[0][w];
    pr += s_red[1][w];
  }
  // the row's units (at most one per pair: within the capacity the unit arrays are sized for)
  const int ue = min(us + row_units, cap);
  us = min(us, ue);
  const unsigned long long lt = (1ull << lane) - 1ull;
  const int nround = (ue - us + kRowUnits - 1) / kRowUnits;
  const bool held = nround <= kRowHold;
  // spans of round r0 + h of the current group of kRowHold rounds in slot h; unit rb + 512 k + t of a round
  // sits in item k of thread t: (k, thread) order is unit order; w = 0 (no unit) meets no column
  int sp[kRowHold][kRowItems];
  auto load = [&](int h, int rb) {
#pragma unroll
    for (int k = 0; k < kRowItems; ++k) {
      const int u = rb + kRowThreads * k + t;
      sp[h][k] = u < ue ? uspan[u] : 0;
    }
  };
  auto meets = [&](int s1) {
    const int a = s1 & 0xffff, z = a + (s1 >> 16);
    return z > a && a < c1 && z > c0;
  };
  // counting: the row's pairs before c0 and, per column of the chunk, a difference array of the units meeting it
  int before = 0;
  auto count = [&](int h) {
#pragma unroll
    for (int k = 0; k < kRowItems; ++k) {
      const int a = sp[h][k] & 0xffff, z = a + (sp[h][k] >> 16);
      if (a < c0) before += min(z, c0) - a;
      if (meets(sp[h][k])) {
        atomicAdd(&s_diff[max(a, c0) - c0], 1);
        atomicAdd(&s_diff[min(z, c1) - c0], -1);
      }
    }
  };
  // rounds in groups of kRowHold, a group's spans loaded at once (a held row is one group)
  auto load_group = [&](int r0) {
#pragma unroll
    for (int h = 0; h < kRowHold; ++h)
      if (r0 + h < nround) load(h, us + (r0 + h) * kRowUnits);
  };
  for (int r0 = 0; r0 < nround; r0 += kRowHold) {
    load_group(r0);
#pragma unroll
    for (int h = 0; h < kRowHold; ++h)
      if (r0 + h < nround) count(h);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) before += __shfl_xor(before, m, 64);
  if (lane == 0) s_red[2][wv] = before;
  __syncthreads();
  // tile starts: the prefix of the column counts after the row's pairs before c0 (wave 0; s_diff -> starts)
  if (wv == 0) {
    int run = pr;
#pragma unroll
    for (int w = 0; w < kRowWaves; ++w) run += s_red[2][w];
    int cnt_run = 0;   // the running column count (inclusive scan of the difference array)
    for (int jb = 0; jb < ncol; jb += 64) {
      const int j = jb + lane;
      const int d = j < ncol ? s_diff[j] : 0;
      const int cnt = cnt_run + wave_incl_scan<int>(d, lane);   // pairs of column j
      const int c = j < ncol ? cnt : 0;
      const int inc = wave_incl_scan<int>(c, lane);
      if (j < ncol) {
        s_diff[j] = run + inc - c;
        tile_starts[tile0 + j] = run + inc - c;
      }
      cnt_run = __shfl(cnt, 63, 64);
      run += __shfl(inc, 63, 64);
    }
  }
  // writing. The list holds n units. A round's units meeting the chunk (`mark`: their number, per (k, wave)
  // their first list slot) go to the list in unit order (`place`) once it has room for them; flush() gathers the
  // listed units' ids, writes their pairs and empties the list.
  int n = 0;
  unsigned long long mk[kRowItems];
  auto mark = [&](int h) -> int {
#pragma unroll
    for (int k = 0; k < kRowItems; ++k) {
      mk[k] = __ballot(meets(sp[h][k]));
      if (lane == 0) s_kc[k][wv] = __popcll(mk[k]);
    }
    __syncthreads();
    if (wv == 0) {   // exclusive prefix in (k, wave) order: lane i < kMark takes entry (i / kRowWaves, i % kRowWaves)
      constexpr int kMark = kRowItems * kRowWaves;
      static_assert(kMark <= 64, "one lane per entry");
      int* kc = &s_kc[0][0];
      const int c = lane < kMark ? kc[lane] : 0;
      const int inc = wave_incl_scan<int>(c, lane);
      if (lane < kMark) kc[lane] = inc - c;
      if (lane == kMark - 1) s_n = inc;
    }
    __syncthreads();
    return s_n;
  };
  auto place = [&](int h, int rb) {
#pragma unroll
    for (int k = 0; k < kRowItems; ++k)
      if ((mk[k] >> lane) & 1) {
        const int idx = n + s_kc[k][wv] + __popcll(mk[k] & lt);
        s_cu[idx] = rb + kRowThreads * k + t;
        s_cs[idx] = sp[h][k];
      }
  };
  constexpr bool REG = CPW > 0;
  int rpos[REG ? CPW : 1];   // REG: the wave's columns' running positions
  bool have_pos = false;
  auto flush = [&]() {
    __syncthreads();   // the list is complete (and the column starts written)
    if (REG && !have_pos) {
#pragma unroll
      for (int m = 0; m < (REG ? CPW : 1); ++m) {
        const int j = wv + kRowWaves * m;
        rpos[m] = j < ncol ? s_diff[j] : 0;
      }
      have_pos = true;
    }
    for (int i = t; i < n; i += kRowThreads) {   // gather: unit index -> splat id, splat-major index
      const int u = s_cu[i];
      s_cu[i] = ug[u];
      s_cq[i] = uq[u];
    }
    __syncthreads();
    for (int b = 0; b < n; b += 64) {
      const int i = b + lane;
      const bool act = i < n;
      const int s1 = act ? s_cs[i] : 0;
      const int g = act ? s_cu[i] : 0, q = act ? s_cq[i] : 0;
      const int a = s1 & 0xffff, z = a + (s1 >> 16);
      // column j of the chunk: the units covering it are its next pairs, from its running position pos
      auto column = [&](int j, int pos, unsigned long long msk, bool cov) {
        if (cov) {
          const int p = pos + __popcll(msk & lt);
          const int qc = q + (c0 + j - a);
          if ((unsigned)p < (unsigned)cap) {
            gid_sorted[p] = g;
            if (pair_q) pair_q[p] = qc;
          }
          if (pair_splat && (unsigned)qc < (unsigned)cap) pair_splat[qc] = g;
        }
      };
      // the wave's columns j = wv + 8 m, whose positions only it touches
      if constexpr (REG) {
#pragma unroll
        for (int m = 0; m < CPW; ++m) {
          const int j = wv + kRowWaves * m;
          if (j >= ncol) break;
          const bool cov = act && a <= c0 + j && c0 + j < z;
          const unsigned long long msk = __ballot(cov);
          column(j, rpos[m], msk, cov);
          rpos[m] += __popcll(msk);
        }
      } else {
        for (int j = wv; j < ncol; j += kRowWaves) {
          const bool cov = act && a <= c0 + j && c0 + j < z;
          const unsigned long long msk = __ballot(cov);
          if (msk) {
            const int pos = s_diff[j];
            column(j, pos, msk, cov);
            if (lane == 0) s_diff[j] = pos + __popcll(msk);
          }
        }
      }
    }
    __syncthreads();   // before the list is refilled
    n = 0;
  };
  // kRowList >= kRowUnits: a round always fits an empty list
  for (int r0 = 0; r0 < nround; r0 += kRowHold) {
    if (!held) load_group(r0);   // a held row's spans are still in registers
#pragma unroll
    for (int h = 0; h < kRowHold; ++h) {
      if (r0 + h < nround) {
        const int m = mark(h);
        if (n + m > kRowList) flush();
        place(h, us + (r0 + h) * kRowUnits);
        n += m;
      }
    }
  }
  flush();
}

// ----------------------------------------------------------------------------------------------------
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Pair-phase workspace: two sets of (keys, splat ids, splat-major indices) that the radix passes ping-pong
// between, the per-block digit histograms and the digit totals.
// Two sort plans, both stable on the tile id (so splats keep ascending order within a tile):
//  * two-phase (lb > 0): tile ids of 10 to 14 bits; one radix pass on the super-tile tile >> lb (9 bits), then
//    k_local_sort orders every super-tile's pairs on the low lb bits and writes the tile starts. Taken while
//    the super-tiles average at most kLocalAvgMax pairs (one workgroup sorts each);
//  * LSD (lb = 0): ceil(bits / 9) radix passes of equal digits, then k_tile_starts.
constexpr long long kLocalAvgMax = 16384;

struct PairsPlan {
  int nblk, passes, dbits, radix, lb, nsuper;
  size_t off_set[2][3], off_hist, off_rowtot, total;
};

static PairsPlan plan_pairs(int nt, long long tot) {
  PairsPlan p{};
  p.nblk = tot > 0 ? div_up(tot, kSortKeys) : 0;
  int nbits = 0;
  while (nt > 1 && (1LL << nbits) < nt) ++nbits;   // bits of the largest tile id nt - 1
  const int lb = nbits - kMaxRadixBits;
  if (lb >= 1 && lb <= kLocalMaxBits) {
    const long long nsuper = ((long long)(nt - 1) >> lb) + 1;
    if (tot <= nsuper * kLocalAvgMax) {
      p.lb = lb;
      p.nsuper = (int)nsuper;
    }
  }
  if (p.lb > 0) {
    p.passes = 1;
    p.dbits = kMaxRadixBits;
  } else {
    // at least one pass: it also moves the values into place
    p.passes = nbits > kMaxRadixBits ? (nbits + kMaxRadixBits - 1) / kMaxRadixBits : 1;
    p.dbits = nbits > 0 ? (nbits + p.passes - 1) / p.passes : 1;
  }
  p.radix = 1 << p.dbits;
  const long long nh = (long long)p.radix * p.nblk;
  size_t o = 0;
  for (int s = 0; s < 2; ++s)
    for (int k = 0; k < 3; ++k) { p.off_set[s][k] = o; o += align256(sizeof(int) * (size_t)tot); }
  p.off_hist = o;   o += align256(sizeof(int) * (size_t)(nh > 0 ? nh : 1));
  p.off_rowtot = o; o += align256(sizeof(int) * kMaxRadix);
  p.total = o;
  return p;
}

// Row plan (k_scatter_units + k_expand_row) when the level table has at most kMaxRows tile rows and the row
// histogram (rows x decode blocks) stays below kMaxRowHist entries; else the pair-sort plans of plan_pairs.
// Count workspace: the block sums, then (row plan) the row histogram int2[nrows][nb] and the row totals
// int2[nrows]. Pair workspace of the row plan: the unit arrays ug, uq, uspan for up to `tot` units (a rect
// row holds at least one pair, so units <= pairs).
constexpr long long kMaxRowHist = 1LL << 22;

struct CountPlan {
  int nb, rows, nrows;
  size_t off_rowhist, off_rtot, total;
};

static CountPlan plan_count(const LevelTable& L, int N) {
  CountPlan c{};
  c.nb = N > 0 ? div_up(N, kBlock) : 1;
  c.nrows = L.rbase[L.n];
  c.rows = c.nrows >= 1 && c.nrows <= kMaxRows && (long long)c.nrows * c.nb <= kMaxRowHist;
  size_t o = align256(sizeof(long long) * kSumCols * (size_t)c.nb);
  if (c.rows) {
    c.off_rowhist = o; o += align256(sizeof(int2) * (size_t)c.nrows * c.nb);
    c.off_rtot = o;    o += align256(sizeof(int2) * (size_t)c.nrows);
  }
  c.total = o;
  return c;
}

static size_t unit_bytes(long long tot) { return align256(sizeof(int) * (size_t)(tot > 0 ? tot : 1)); }

// Bytes of the pair workspace for `tot` pairs under the plan the level table takes.
static size_t pairs_ws_bytes(const LevelTable& L, int N, long long tot) {
  return plan_count(L, N).rows ? 3 * unit_bytes(tot) : plan_pairs(L.tbase[L.n], tot).total;
}


}  // namespace splat

using namespace splat;

extern "C" {

size_t splat_bin_count_workspace_bytes(int N, int H, int W, int TILE, const splat_levels* lv) {
  LevelTable L;
  if (N < 0 || H < 1 || W < 1 || TILE < 1 || make_levels(H, W, TILE, lv, &L, nullptr)) return 0;
  return plan_count(L, N).total;
}

int splat_levels_geometry(int H, int W, int TILE, const splat_levels* lv, int* out, int cap) {
  LevelTable L;
  if (H < 1 || W < 1 || TILE < 1 || make_levels(H, W, TILE, lv, &L, nullptr))
    return -set_error(kInvalid, "splat_levels_geometry: bad levels for H=%d W=%d TILE=%d", H, W, TILE);
  if (out) {
    if (cap < 5 * L.n + 2) return -set_error(kInvalid, "splat_levels_geometry: out holds %d < %d ints", cap, 5 * L.n + 2);
    for (int l = 0; l < L.n; ++l) {
      out[5 * l + 0] = L.H[l]; out[5 * l + 1] = L.W[l]; out[5 * l + 2] = L.ntx[l];
      out[5 * l + 3] = L.tbase[l]; out[5 * l + 4] = L.pbase[l];
    }
    out[5 * L.n] = L.tbase[L.n];
    out[5 * L.n + 1] = L.pbase[L.n];
  }
  return L.n;
}

int splat_decode(const float* mu, const float* scale, const float* theta, const float* opacity, const float* color,
                 int C, int N, float* rec, void* stream) {
  if (N < 0 || C < 1 || C > kMaxC) return set_error(kInvalid, "splat_decode: N=%d C=%d (C must be 1..%d)", N, C, kMaxC);
  if (N == 0) return kOk;
  if (!mu || !scale || !opacity || !color || !rec) return set_error(kInvalid, "splat_decode: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const int nb = div_up(N, kBlock);
  LevelTable L{};
  Routing R{};
#define SPLAT_DECODE(CC)                                                                                      \
  k_decode_count<CC><<<nb, kBlock, 0, st>>>(mu, scale, theta, opacity, color, N, L, R, 1.f, 0.f, 0, 0,     \
                                            reinterpret_cast<float4*>(rec), nullptr, nullptr, nullptr, nullptr, 0)
  switch (C) { case 1: SPLAT_DECODE(1); break; case 2: SPLAT_DECODE(2); break;
               case 3: SPLAT_DECODE(3); break; default: SPLAT_DECODE(4); break; }
#undef SPLAT_DECODE
  return check_launch("k_decode_count(decode)");
}

}  // extern "C"

namespace {

// Launches of the count phase (decode + route + count + offsets + info). Arguments already validated.
int bin_count_launch(const float* mu, const float* scale, const float* theta, const float* opacity,
                     const float* color, int C, int N, const LevelTable& L, const Routing& R, int TILE, float cutoff,
                     int flags, float* rec, int* rect, int* offsets, long long* info, long long* mirror, void* ws,
                     hipStream_t st) {
  const CountPlan cp = plan_count(L, N);
  const int nb = cp.nb;
  long long* sums = (long long*)ws;
  int2* rowhist = cp.rows ? (int2*)((char*)ws + cp.off_rowhist) : nullptr;
  int2* rtot = cp.rows ? (int2*)((char*)ws + cp.off_rtot) : nullptr;
#define SPLAT_DC(CC)                                                                                         \
  k_decode_count<CC><<<nb, kBlock, 0, st>>>(mu, scale, theta, opacity, color, N, L, R, (float)TILE, cutoff, 1, \
                                            (flags & kFlagLogScale) ? 1 : 0,                                \
                                            reinterpret_cast<float4*>(rec), reinterpret_cast<int4*>(rect), \
                                            offsets, sums, rowhist, nb)
  switch (C) { case 1: SPLAT_DC(1); break; case 2: SPLAT_DC(2); break;
               case 3: SPLAT_DC(3); break; default: SPLAT_DC(4); break; }
#undef SPLAT_DC
  if (nb <= kFusedScanBlocks) {
    k_offsets_fused<<<nb + (cp.rows ? cp.nrows : 0), kBlock, 0, st>>>(offsets, sums, N, nb, L.n, info, mirror, rowhist,
                                                                      rtot);
  } else {
    k_scan_sums<<<1, 1024, 0, st>>>(sums, nb, L.n, info, mirror);
    k_offsets<<<nb, kBlock, 0, st>>>(offsets, sums, N, info);
    if (cp.rows) k_row_scan<<<cp.nrows, kBlock, 0, st>>>(rowhist, nb, rtot);
  }
  return check_launch("splat_bin_count");
}

// Launches of the pair phase. Exact (dinfo NULL): `t` is the pair count. Speculative (dinfo = the count
// phase's device info): `t` is the capacity the buffers and the grids are sized for, and the kernels take
// the count from dinfo (an empty list when it exceeds t). Arguments already validated; ws holds
// pairs_ws_bytes(L, N, t); ws_count the count phase's workspace (the row plan's histogram).
int bin_pairs_launch(const int* rect, const int* offsets, const void* ws_count, int N, const LevelTable& L, int t,
                     const long long* dinfo, int* gid_sorted, int* tile_starts, int* pair_splat, int* pair_q, void* ws,
                     hipStream_t st) {
  const int nt = L.tbase[L.n];
  if (t == 0) {
    k_fill_i32<<<div_up(nt + 1, 256), 256, 0, st>>>(tile_starts, nt + 1, 0);
    k_fill_i32<<<1, 64, 0, st>>>(gid_sorted, 1, 0);
    return check_launch("splat_bin_pairs(empty)");
  }
  const CountPlan cp = plan_count(L, N);
  if (cp.rows) {
    const int2* rowhist = (const int2*)((const char*)ws_count + cp.off_rowhist);
    const int2* rtot = (const int2*)((const char*)ws_count + cp.off_rtot);
    const size_t ub = unit_bytes(t);
    int* ug = (int*)ws;
    int* uq = (int*)((char*)ws + ub);
    int* uspan = (int*)((char*)ws + 2 * ub);
    k_scatter_units<<<cp.nb, kBlock, 0, st>>>(reinterpret_cast<const int4*>(rect), offsets, N, L, dinfo, t, rowhist, rtot,
                                              cp.nb, ug, uq, uspan);
    int rc = check_launch("k_scatter_units");
    if (rc) return rc;
    int mxtx = 1;
    for (int l = 0; l < L.n; ++l) mxtx = L.ntx[l] > mxtx ? L.ntx[l] : mxtx;
    // chunks of at most kRowCols columns, about 8 per row of the widest level (measured: 4 to 12 chunks, 256 to
    // 1024 threads, 2 to 8 units per thread; this is the fastest at 768 x 768 and 2048 x 2048)
    const int cw = min(kRowCols, max(8, div_up(mxtx, 8)));
    const dim3 grid(div_up(mxtx, cw), cp.nrows);
    if (cw <= 2 * kRowWaves)
      k_expand_row<2><<<grid, kRowThreads, 0, st>>>(L, dinfo, t, rtot, cw, ug, uq, uspan, gid_sorted, tile_starts,
                                                     pair_splat, pair_q);
    else if (cw <= 4 * kRowWaves)
      k_expand_row<4><<<grid, kRowThreads, 0, st>>>(L, dinfo, t, rtot, cw, ug, uq, uspan, gid_sorted, tile_starts,
                                                     pair_splat, pair_q);
    else
      k_expand_row<0><<<grid, kRowThreads, 0, st>>>(L, dinfo, t, rtot, cw, ug, uq, uspan, gid_sorted, tile_starts,
                                                     pair_splat, pair_q);
    return check_launch("k_expand_row");
  }
  const PairsPlan pl = plan_pairs(nt, t);
  char* base = (char*)ws;
  int* S[2][3];   // workspace sets: keys, splat ids, splat-major indices
  for (int s = 0; s < 2; ++s)
    for (int k = 0; k < 3; ++k) S[s][k] = (int*)(base + pl.off_set[s][k]);
  int* hist = (int*)(base + pl.off_hist);
  int* rowtot = (int*)(base + pl.off_rowtot);
  // The scatter writes the splat-major keys and splat ids into set 1 (the splat ids into the caller's
  // pair_splat when given). Pass k < passes - 1 writes set k % 2 and the next pass reads it; the last pass
  // writes its keys into the set it does not read and the values into gid_sorted / pair_q.
  const bool maps = pair_q != nullptr;
  int* psplat = pair_splat ? pair_splat : S[1][1];
  const int dmask = pl.radix - 1;
  const bool two_phase = pl.lb > 0;
  k_scatter_pairs<<<pl.nblk, kBlock, 0, st>>>(reinterpret_cast<const int4*>(rect), offsets, N, L, dinfo, t, pl.lb,
                                              dmask, S[1][0], psplat, hist, pl.nblk);
  int rc = check_launch("k_scatter_pairs");
  if (rc) return rc;
  const int* kin = S[1][0];
  const int* vin = psplat;
  const int* qin = nullptr;
  int* kfin = nullptr;
  for (int pass = 0; pass < pl.passes; ++pass) {
    const int shift = two_phase ? pl.lb : pass * pl.dbits;
    const bool last = pass == pl.passes - 1 && !two_phase;   // writes the final gid_sorted / pair_q
    int* const* D = S[pass & 1];
    int* kout = D[0];
    int* vout = last ? gid_sorted : D[1];
    int* qout = maps ? (last ? pair_q : D[2]) : nullptr;
    if (pass > 0) k_radix_hist<<<pl.nblk, kBlock, 0, st>>>(kin, dinfo, t, shift, dmask, hist, pl.nblk);
    k_hist_row_scan<<<pl.radix, kBlock, 0, st>>>(hist, pl.nblk, rowtot);
    if (pl.dbits > 8)
      k_radix_scatter<2><<<pl.nblk, kBlock, 0, st>>>(kin, vin, qin, dinfo, t, shift, pl.dbits, hist, rowtot, pl.nblk,
                                                     kout, vout, qout);
    else
      k_radix_scatter<1><<<pl.nblk, kBlock, 0, st>>>(kin, vin, qin, dinfo, t, shift, pl.dbits, hist, rowtot, pl.nblk,
                                                     kout, vout, qout);
    rc = check_launch("k_radix_scatter");
    if (rc) return rc;
    kin = kout;
    vin = vout;
    qin = qout;
    kfin = kout;
  }
  if (two_phase) {
    k_local_sort<<<pl.nsuper, kLocalThreads, 0, st>>>(kin, vin, qin, dinfo, t, pl.lb, nt, pl.nsuper, rowtot, gid_sorted,
                                                      maps ? pair_q : nullptr, tile_starts);
    return check_launch("k_local_sort");
  }
  k_tile_starts<<<div_up(nt + 1, kBlock), kBlock, 0, st>>>(kfin, gid_sorted, dinfo, t, nt, tile_starts);
  return check_launch("k_tile_starts");
}

// Device address of the pinned host buffer `h` (hipHostMalloc), or NULL when `h` is not pinned (the count is
// then copied).
constexpr long long kUnsetInfo = LLONG_MIN;   // an info entry not (yet) written
long long* host_mirror(long long* h) {
  hipPointerAttribute_t at{};
  void* d = nullptr;
  if (hipPointerGetAttributes(&at, h) != hipSuccess || at.type != hipMemoryTypeHost ||
      hipHostGetDevicePointer(&d, h, 0) != hipSuccess || !d) {
    (void)hipGetLastError();   // pageable memory: not an error of the render
    return nullptr;
  }
  return (long long*)d;
}

// Scratch of splat_bin_noalloc: the count and pair-phase workspaces of one binning, in a file-scope device
// array. Each GPU the library runs on holds its own copy until the process ends. Host code never uses the
// array's name as an address (in host code it is a host-side stand-in): the device address comes from
// hipGetSymbolAddress, looked up once per device with that device current and kept in g_scratch_dev.
constexpr size_t kNoAllocScratchBytes = 64ull << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of the current device's scratch (looked up on the device's first call), or NULL with the
// error set.
void* noalloc_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error(kHipError, "splat_bin_noalloc: no current device (or device %d >= %d)", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error(kHipError, "splat_bin_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_dev[dev] = ptr;
  }
  return g_scratch_dev[dev];
}

// Ordering of splat_bin_noalloc calls on one device: every call's kernels use the device's one scratch, so each
// call's stream first waits for the event that the previous call recorded behind its last scratch user. The
// mutex makes (wait, launches, record) one step across threads, so the calls run one after another on the GPU
// in the order they took the mutex, whatever streams they are queued on. The event is created on the device's
// first call and kept until the process ends.
struct ScratchOrder {
  std::mutex mu;
  hipEvent_t done = nullptr;
};
ScratchOrder g_scratch_order[kMaxDevices];

// Per-thread read-back events of splat_bin (one per device), destroyed when a thread other than the process's
// first one exits. The first thread's events are left to the end of the process: its thread-local objects are
// destroyed during exit, when the HIP runtime may already be shutting down.
struct ReadbackEvents {
  hipEvent_t ev[kMaxDevices] = {};
  ~ReadbackEvents() {
    if ((pid_t)syscall(SYS_gettid) == getpid()) return;
    for (int d = 0; d < kMaxDevices; ++d)
      if (ev[d]) {
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur != d) (void)hipSetDevice(d);
        (void)hipEventDestroy(ev[d]);
        if (cur >= 0 && cur != d) (void)hipSetDevice(cur);
      }
  }
};

// One event per thread and device, recorded after the read-back of the pair count (splat_bin).
hipEvent_t readback_event() {
  static thread_local ReadbackEvents tls;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  hipEvent_t& ev = tls.ev[dev];
  if (!ev && hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) ev = nullptr;
  return ev;
}

}  // namespace

extern "C" {

int splat_bin_count(const float* mu, const float* scale, const float* theta, const float* opacity, const float* color,
                    int C, int N, int H, int W, int TILE, float cutoff, const splat_levels* lv, int flags, float* rec,
                    int* rect, int* offsets, long long* info, void* ws, size_t ws_bytes, void* stream) {
  if (N < 1 || C < 1 || C > kMaxC || H < 1 || W < 1 || TILE < 1)
    return set_error(kInvalid, "splat_bin_count: N=%d C=%d H=%d W=%d TILE=%d", N, C, H, W, TILE);
  if (flags & ~kFlagLogScale) return set_error(kInvalid, "splat_bin_count: unknown flags 0x%x", flags);
  LevelTable L;
  Routing R;
  if (make_levels(H, W, TILE, lv, &L, &R)) return set_error(kInvalid, "splat_bin_count: bad levels");
  if (!mu || !scale || !opacity || !color || !rec || !rect || !offsets || !info)
    return set_error(kInvalid, "splat_bin_count: null pointer");
  if (ws_bytes < plan_count(L, N).total) return set_error(kWorkspace, "splat_bin_count: workspace too small");
  return bin_count_launch(mu, scale, theta, opacity, color, C, N, L, R, TILE, cutoff, flags, rec, rect, offsets, info, nullptr,
                          ws, (hipStream_t)stream);
}

size_t splat_bin_pairs_workspace_bytes(int N, int H, int W, int TILE, const splat_levels* lv, long long tot) {
  LevelTable L;
  if (N < 0 || H < 1 || W < 1 || TILE < 1 || tot < 0 || make_levels(H, W, TILE, lv, &L, nullptr)) return 0;
  return pairs_ws_bytes(L, N, tot);
}

int splat_bin_pairs(const int* rect, const int* offsets, const void* ws_count, int N, int H, int W, int TILE,
                    const splat_levels* lv, long long tot, int* gid_sorted, int* tile_starts, int* pair_splat,
                    int* pair_q, void* ws, size_t ws_bytes, void* stream) {
  if (N < 1 || H < 1 || W < 1 || TILE < 1 || tot < 0 || tot > 0x7fffffffLL - 64)
    return set_error(kInvalid, "splat_bin_pairs: N=%d H=%d W=%d TILE=%d tot=%lld", N, H, W, TILE, tot);
  if (!rect || !offsets || !ws_count || !gid_sorted || !tile_starts)
    return set_error(kInvalid, "splat_bin_pairs: null pointer");
  LevelTable L;
  if (make_levels(H, W, TILE, lv, &L, nullptr)) return set_error(kInvalid, "splat_bin_pairs: bad levels");
  const size_t need = pairs_ws_bytes(L, N, tot);
  if (ws_bytes < need) return set_error(kWorkspace, "splat_bin_pairs: workspace %zu < %zu bytes", ws_bytes, need);
  return bin_pairs_launch(rect, offsets, ws_count, N, L, (int)tot, nullptr, gid_sorted, tile_starts, pair_splat, pair_q,
                          ws, (hipStream_t)stream);
}

}  // extern "C"

namespace {

// Whether every entry of a pinned totals buffer has been written by the count kernel.
bool totals_seen(const long long* info_host, int ninfo) {
  const volatile long long* ih = info_host;
  for (int i = 0; i < ninfo; ++i)
    if (ih[i] == kUnsetInfo) return false;
  return true;
}

// The one read of a binning's totals (info_host[0, 2 + nlev)) and the checks of splat_bin: error bits, the
// per-level budget, the capacity. Pinned totals (the count kernel stores them into host memory itself, every
// entry preset to kUnsetInfo) are polled until every entry is written, without an event: recording one costs the
// host several microseconds per render. Between polls the stream is queried now and then; once it is idle the
// count kernel has run, and totals still unseen are copied from the device. Pageable totals wait for the
// read-back event recorded behind their copy.
int read_totals(const char* who, long long* info_host, const long long* info, int nlev, long long max_pairs,
                long long pair_cap, hipStream_t st) {
  const int ninfo = 2 + nlev;
  if (host_mirror(info_host)) {
    for (unsigned it = 1; !totals_seen(info_host, ninfo); ++it) {
      __builtin_ia32_pause();
      if ((it & 1023) != 0) continue;
      const hipError_t q = hipStreamQuery(st);
      if (q == hipErrorNotReady) continue;
      if (q != hipSuccess) return set_error(kHipError, "%s: reading the pair totals failed", who);
      if (!totals_seen(info_host, ninfo) &&   // the kernel's stores did not reach the host: copy them
          (hipMemcpyAsync(info_host, info, sizeof(long long) * ninfo, hipMemcpyDeviceToHost, st) != hipSuccess ||
           hipStreamSynchronize(st) != hipSuccess))
        return set_error(kHipError, "%s: reading the pair totals failed", who);
      break;
    }
  } else {
    hipEvent_t ev = readback_event();
    if (!ev || hipEventSynchronize(ev) != hipSuccess)
      return set_error(kHipError, "%s: reading the pair totals failed", who);
  }
  const long long tot = info_host[0];
  if (info_host[1] & 1) return set_error(kInvalid, "%s: a splat has an empty tile rect (negative cutoff or scale)", who);
  if (info_host[1] & 2) return set_error(kOverflow, "%s: %lld pairs exceed the int32 pair index range", who, tot);
  if (max_pairs >= 0)
    for (int l = 0; l < nlev; ++l)
      if (info_host[2 + l] > max_pairs)
        return set_error(kBudget, "%s: %lld pairs on level %d exceed the budget of %lld", who, info_host[2 + l], l,
                         max_pairs);
  if (tot > pair_cap) return set_error(kCapacity, "%s: %lld pairs exceed the capacity %lld", who, tot, pair_cap);
  return kOk;
}

}  // namespace

extern "C" {

int splat_bin(const float* mu, const float* scale, const float* theta, const float* opacity, const float* color, int C,
              int N, int H, int W, int TILE, float cutoff, const splat_levels* lv, int flags, long long max_pairs,
              float* rec, int* rect, int* offsets, long long* info, long long* info_host, void* ws_count, size_t ws_count_bytes,
              long long pair_cap, int* gid_sorted, int* tile_starts, int* pair_splat, int* pair_q, void* ws_pairs,
              size_t ws_pairs_bytes, void* stream) {
  if (N < 1 || C < 1 || C > kMaxC || H < 1 || W < 1 || TILE < 1 || pair_cap < 0)
    return set_error(kInvalid, "splat_bin: N=%d C=%d H=%d W=%d TILE=%d cap=%lld", N, C, H, W, TILE, pair_cap);
  if (flags & ~(kFlagLogScale | kFlagDefer)) return set_error(kInvalid, "splat_bin: unknown flags 0x%x", flags);
  LevelTable L;
  Routing R;
  if (make_levels(H, W, TILE, lv, &L, &R)) return set_error(kInvalid, "splat_bin: bad levels");
  if (!mu || !scale || !opacity || !color || !rec || !rect || !offsets || !info || !info_host)
    return set_error(kInvalid, "splat_bin: null pointer");
  if (ws_count_bytes < plan_count(L, N).total) return set_error(kWorkspace, "splat_bin: count workspace too small");
  // With buffers for pair_cap > 0 pairs the pair phase is queued before the host waits for the count: the GPU
  // goes on with it while the host reads the count (kernels past the count, or past pair_cap, do nothing).
  const bool spec = pair_cap > 0 && pair_cap <= 0x7fffffffLL - 64 && gid_sorted && tile_starts &&
                    ws_pairs_bytes >= pairs_ws_bytes(L, N, pair_cap);
  const bool defer = flags & kFlagDefer;
  if (defer && !spec)
    return set_error(kInvalid, "splat_bin: a deferred read needs pair buffers and workspace for pair_cap > 0 pairs");
  hipStream_t st = (hipStream_t)stream;
  // the one device -> host read of the render (totals and error bits): the offsets kernel writes them into
  // info_host itself when it is pinned memory, else they are copied. Entries the kernel has not written keep
  // the value kUnsetInfo.
  const int ninfo = 2 + L.n;
  long long* mirror = host_mirror(info_host);
  volatile long long* ih = info_host;
  if (mirror)
    for (int i = 0; i < ninfo; ++i) ih[i] = kUnsetInfo;
  int rc = bin_count_launch(mu, scale, theta, opacity, color, C, N, L, R, TILE, cutoff, flags, rec, rect, offsets,
                            info, mirror, ws_count, st);
  if (rc) return rc;
  if (!mirror) {   // pageable totals: a copy and the event read_totals waits for
    hipEvent_t ev = readback_event();
    if (!ev || hipMemcpyAsync(info_host, info, sizeof(long long) * ninfo, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipEventRecord(ev, st) != hipSuccess)
      return set_error(kHipError, "splat_bin: queueing the read of the pair totals failed");
  }
  if (spec) {
    rc = bin_pairs_launch(rect, offsets, ws_count, N, L, (int)pair_cap, info, gid_sorted, tile_starts, pair_splat, pair_q,
                          ws_pairs, st);
    if (rc) return rc;
  }
  if (defer) return kOk;   // splat_bin_finish reads the totals
  rc = read_totals("splat_bin", info_host, info, L.n, max_pairs, pair_cap, st);
  if (rc != kOk || spec) return rc;
  // tot <= pair_cap without a speculative launch (no pairs with pair_cap = 0, or a workspace too small for
  // pair_cap pairs): the pair phase for the count just read
  const long long tot = info_host[0];
  if (!gid_sorted || !tile_starts) return set_error(kInvalid, "splat_bin: null pair buffers");
  if (ws_pairs_bytes < pairs_ws_bytes(L, N, tot)) return set_error(kWorkspace, "splat_bin: pair workspace too small");
  return bin_pairs_launch(rect, offsets, ws_count, N, L, (int)tot, nullptr, gid_sorted, tile_starts, pair_splat, pair_q, ws_pairs,
                          st);
}

int splat_bin_finish(long long* info_host, const long long* info, int nlev, long long max_pairs, long long pair_cap,
                     void* stream) {
  if (!info_host || !info || nlev < 1 || nlev > kMaxLevels || pair_cap < 0)
    return set_error(kInvalid, "splat_bin_finish: nlev=%d cap=%lld", nlev, pair_cap);
  return read_totals("splat_bin_finish", info_host, info, nlev, max_pairs, pair_cap, (hipStream_t)stream);
}

int splat_bin_noalloc(const float* mu, const float* scale, const float* theta, const float* opacity, const float* color,
                      int C, int N, int H, int W, int TILE, float cutoff, const splat_levels* lv, int flags,
                      long long max_pairs, float* rec, int* rect, int* offsets, long long* info, long long* info_host,
                      long long pair_cap, int* gid_sorted, int* tile_starts, int* pair_splat, int* pair_q,
                      void* stream) {
  if (N < 1 || C < 1 || C > kMaxC || H < 1 || W < 1 || TILE < 1)
    return set_error(kInvalid, "splat_bin_noalloc: N=%d C=%d H=%d W=%d TILE=%d", N, C, H, W, TILE);
  if (pair_cap < 1 || pair_cap > 0x7fffffffLL - 64 || !gid_sorted || !tile_starts)
    return set_error(kInvalid, "splat_bin_noalloc: needs pair buffers (pair_cap=%lld)", pair_cap);
  LevelTable L;
  if (make_levels(H, W, TILE, lv, &L, nullptr)) return set_error(kInvalid, "splat_bin_noalloc: bad levels");
  const size_t cbytes = plan_count(L, N).total;
  const size_t pbytes = pairs_ws_bytes(L, N, pair_cap);
  if (cbytes + pbytes > kNoAllocScratchBytes)
    return set_error(kWorkspace,
                     "splat_bin_noalloc: N=%d splats with pair_cap=%lld need %zu bytes of scratch, above its %zu "
                     "(12 bytes per pair at most, 25 past %d tile rows); use splat_bin with a workspace",
                     N, pair_cap, cbytes + pbytes, kNoAllocScratchBytes, kMaxRows);
  char* ws = (char*)noalloc_scratch();
  if (!ws) return kHipError;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(kHipError, "splat_bin_noalloc: no current device");
  ScratchOrder& order = g_scratch_order[dev];
  hipStream_t st = (hipStream_t)stream;
  std::lock_guard<std::mutex> lock(order.mu);
  if (!order.done && hipEventCreateWithFlags(&order.done, hipEventDisableTiming) != hipSuccess) {
    order.done = nullptr;
    return set_error(kHipError, "splat_bin_noalloc: creating the scratch-order event on device %d failed", dev);
  }
  if (hipStreamWaitEvent(st, order.done, 0) != hipSuccess)
    return set_error(kHipError, "splat_bin_noalloc: ordering after the previous scratch user failed");
  const int rc = splat_bin(mu, scale, theta, opacity, color, C, N, H, W, TILE, cutoff, lv, flags, max_pairs, rec, rect,
                           offsets, info, info_host, ws, cbytes, pair_cap, gid_sorted, tile_starts, pair_splat, pair_q,
                           ws + cbytes, pbytes, stream);
  // behind every kernel the call queued (a status after launches still leaves them on the stream)
  if (hipEventRecord(order.done, st) != hipSuccess && rc == kOk)
    return set_error(kHipError, "splat_bin_noalloc: recording the scratch-order event failed");
  return rc;
}

}  // extern "C"
