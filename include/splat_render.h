/* C-ABI of the gfx950 tile-binned Gaussian-splat renderer (libsplat_hip.so).
 *
 * Every entry point takes raw device pointers (fp32 / int32, contiguous), sizes and a hipStream_t passed
 * as `void *stream`; all work is enqueued on that stream. No entry point allocates; only splat_bin and
 * splat_bin_noalloc wait (for the one read-back of the pair totals that sizes the pair buffers and applies
 * the budget).
 * Buffers are owned by the caller; scratch memory comes in as (ws, ws_bytes), sized by the matching
 * *_workspace_bytes query. Every call returns 0 on success or a status code, with a message available
 * from splat_last_error() (thread-local):
 *   1 invalid argument, 2 HIP launch error, 3 unsupported configuration, 4 overflow, 5 workspace too small,
 *   6 pair capacity too small (splat_bin), 7 pair budget exceeded (splat_bin).
 *
 * Layouts (one image; callers loop over the batch like the reference does):
 *   mu[N,2] (y, x) in [0,1];  scale[N,2] (sy, sx) = softplus(log_scale) + 1e-4;  theta[N] or NULL;
 *   opacity[N];  color[N,C] with 1 <= C <= 4;  rec[N,16] the decoded splat record (64 B per splat).
 *   Pixel fields are row-major: [P] or [P,C] with P = H*W, p = y*W + x.
 *
 * The reference (bigwolfeman/gaussian-2d-splat-encoder) is Python + Triton; each function below replaces
 * the cited part of gaussian_splat_encoder/render_triton.py. The package's ctypes binding is
 * gaussian-2d-splat-encoder_amd/gaussian_splat_encoder/_lib.py.
 */
#ifndef SPLAT_RENDER_H
#define SPLAT_RENDER_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPLAT_FLAG_FIELDS 1 /* forward writes raw sums (S_log, S_a, S_ac); backward takes dS_* upstream */
#define SPLAT_FLAG_ODDS 2   /* colour weight a/(1-a) instead of a */
#define SPLAT_FLAG_UPS 4    /* composite adds the coarse levels' upsampled fields; clamp_min gradient of S_a */
#define SPLAT_FLAG_WIDE 8   /* TILE 8: 16 waves share each tile's pair list, instead of 4 in the forward and 1 in
                               the backward (a performance hint for launches of few tiles with long lists; results
                               are identical up to summation order: the forward adds the waves' partial sums in
                               another grouping, and the backward's per-pair sums of the pairs that end a wave's
                               share in a partial pass are split over lanes and combined by xor shuffles) */
#define SPLAT_FLAG_LOG_SCALE 16 /* binning (splat_bin, splat_bin_count): `scale` holds the raw log-scales [N,2]; the
                                   decode pass activates them, softplus(x) + 1e-4 with the bits torch's fp32
                                   F.softplus(x) + 1e-4 gives (params.py:18-28), so callers need no activation
                                   pass of their own; rec holds the activated scale either way */
#define SPLAT_FLAG_DEFER 32 /* splat_bin / splat_bin_noalloc with pair_cap > 0: return as soon as the count, the read-back
                               and the speculative pair phase are queued, without waiting for the read; the
                               caller may queue launches that read the pair list (a count above pair_cap leaves
                               them an empty list) and then calls splat_bin_finish for the statuses */

/* Levels of a render. A NULL splat_levels* (or mode 0) is the single canvas (H, W). Otherwise splats are
 * routed to canvases ("levels"): level 0 is (H, W); coarser levels are rendered into packed fields and
 * bilinearly upsampled (torch upsample_bilinear2d, align_corners=False) onto level 0 before compositing.
 *   mode 1, octaves (render_triton.py:925-980): level o in 0..max_octaves is (max(8, H>>o), max(8, W>>o))
 *     (H, W >= 8); splat goes to o = clamp(ceil(log2(max(max(sy, sx) * min(H, W) / base_texels, 1e-6))),
 *     0, max_octaves), computed in fp32 from the activated scale. Octaves from the first whose canvas is
 *     (8, 8) on share one level (their fields are summed after the same upsample); H, W <= 8 << 11.
 *   mode 2, coarse/fine split (render_triton.py:879-922): splats [0, n_coarse) render on
 *     (coarse_H, coarse_W) as level 1, the rest on (H, W).
 * Level l takes global tile ids [tbase[l], tbase[l+1]) and packed pixel slots [pbase[l], pbase[l+1]) of
 * the FIELDS buffers; splat_levels_geometry reports them. */
typedef struct splat_levels {
  int mode;
  int max_octaves;
  float base_texels;
  int n_coarse;
  int coarse_H, coarse_W;
} splat_levels;

/* Number of levels L (or a negative status). With out != NULL (cap >= 5L+2 ints) writes, per level l,
 * out[5l..5l+4] = (H_l, W_l, tiles per row, tbase[l], pbase[l]) and then total tiles, total pixel slots.
 * Replaces the per-octave canvas sizes of render_triton.py:957-961 and :896-898. */
int splat_levels_geometry(int H, int W, int TILE, const splat_levels *lv, int *out, int cap);

const char *splat_last_error(void);
int splat_abi_version(void);

/* Decoded splat records only (no binning), for the exact path.
 * Replaces the per-launch parameter split of render_triton.py:134-142 and :276-279. */
int splat_decode(const float *mu, const float *scale, const float *theta, const float *opacity,
                 const float *color, int C, int N, float *rec, void *stream);

/* Binning phase 1: decode + level routing + per-splat tile rect and pair count + exclusive scan.
 * Writes rec[N,16], rect[N,4] = (tx0, ty0, w, level) of the splat's tile rect, offsets[N+1]
 * (offsets[N] = total pairs) and info[2 + L] (device int64): info[0] = total pairs, info[1] = error bits
 * (1 empty rect, 2 int32 overflow), info[2 + l] = pairs of level l (L = number of levels).
 * The caller reads info once to size the pair buffers and to apply its pair budget per level.
 * The workspace (sized for N splats on the level table of H, W, TILE, lv) also carries, for level tables of
 * at most 1,024 tile rows, a histogram of the splats' rect rows that phase 2 reads: keep it for phase 2.
 * Replaces render_triton.py:362-391 (_build_tiles up to the tot sync), :520-535 (param gathers) and the
 * octave routing / index_select of :950-962. */
size_t splat_bin_count_workspace_bytes(int N, int H, int W, int TILE, const splat_levels *lv);
int splat_bin_count(const float *mu, const float *scale, const float *theta, const float *opacity,
                    const float *color, int C, int N, int H, int W, int TILE, float cutoff,
                    const splat_levels *lv, int flags, float *rec, int *rect, int *offsets, long long *info, void *ws,
                    size_t ws_bytes, void *stream);

/* Binning phase 2: the stable sort of the (tile, splat) pairs on the global tile id, and CSR tile starts. Level
 * tables of at most 1,024 tile rows: a stable partition of the splats' rect rows ("units", 4-5x fewer than
 * pairs) by tile row, from phase 1's row histogram in ws_count, then each row's units expanded column by
 * column into the row's pairs; larger tables: expansion of the rects into pairs and radix passes on the tile
 * id. ws_count is phase 1's workspace, as phase 1 left it.
 * gid_sorted[max(tot,1)] lists splat ids ordered by (tile, splat id); tile_starts[nt+1] with nt the total
 * tile count over all levels (splat_levels_geometry).
 * tot == 0 gives gid_sorted = {0} and all-zero starts, as the reference does.
 * Optional (NULL skips) maps between the sorted order i and the splat-major pair order q (splat g owns
 * q in [offsets[g], offsets[g+1]), walking its rect row by row), used by the backward:
 * pair_splat[q] = splat of q, pair_q[i] = q of sorted pair i.
 * Replaces render_triton.py:392-409. */
size_t splat_bin_pairs_workspace_bytes(int N, int H, int W, int TILE, const splat_levels *lv, long long tot);
int splat_bin_pairs(const int *rect, const int *offsets, const void *ws_count, int N, int H, int W, int TILE,
                    const splat_levels *lv, long long tot, int *gid_sorted, int *tile_starts,
                    int *pair_splat, int *pair_q, void *ws, size_t ws_bytes, void *stream);

/* Binning in one call: phase 1 (splat_bin_count), one read of info into host memory info_host (2 + L int64),
 * then phase 2 (splat_bin_pairs). When info_host is pinned (hipHostMalloc) the offsets kernel writes the totals
 * into it directly; pageable memory gets a copy. With pair_cap > 0 (buffers for pair_cap pairs, ws_pairs
 * sized by splat_bin_pairs_workspace_bytes(N, H, W, TILE, lv, pair_cap)) phase 2 is queued BEFORE the host waits for
 * the read: its kernels take the pair count from info on the device, so the GPU runs the pair phase while
 * the host checks the count; a count above pair_cap (or an error bit) makes that launch write an empty
 * list (starts 0, gid_sorted[0] = 0) and nothing else. With pair_cap = 0 the host waits first. The call
 * returns after the read has completed; the pair phase may still be running on `stream`. Statuses:
 *   0 the pair phase ran into gid_sorted / tile_starts / pair_splat / pair_q;
 *   6 tot > pair_cap: the caller sizes buffers from info_host[0] and calls splat_bin_pairs (any speculative
 *     launch wrote only its empty list into the given buffers);
 *   7 some level holds more than max_pairs pairs (max_pairs < 0: no budget); no buffer beyond pair_cap
 *     was needed;
 *   1 / 4 the error bits of info (empty rect, int32 overflow).
 * Replaces render_triton.py:351-409 with its one sync (:391) and budget check (:378-385). */
int splat_bin(const float *mu, const float *scale, const float *theta, const float *opacity,
              const float *color, int C, int N, int H, int W, int TILE, float cutoff, const splat_levels *lv,
              int flags, long long max_pairs, float *rec, int *rect, int *offsets, long long *info, long long *info_host,
              void *ws_count, size_t ws_count_bytes, long long pair_cap, int *gid_sorted, int *tile_starts,
              int *pair_splat, int *pair_q, void *ws_pairs, size_t ws_pairs_bytes, void *stream);

/* The read of a binning queued with SPLAT_FLAG_DEFER (no counterpart in the reference: its read is the wait at
 * render_triton.py:391, which splat_bin does inside): waits for the totals to land in info_host[0, 2 + nlev) and
 * returns splat_bin's status for them (0, 6 past pair_cap, 7 over max_pairs, 1 / 4 error bits), with the same
 * info, info_host, max_pairs and pair_cap as that call. Call it on the thread (and current device) that queued the binning,
 * before the next splat_bin into the same info_host: pinned totals are polled (splat_bin presets every entry), pageable
 * ones wait on a read-back event per thread and device. Launches queued in between on the
 * speculative pair list have run on the right list when it returns 0; on status 6 they read an empty list and
 * must be repeated after splat_bin_pairs. */
int splat_bin_finish(long long *info_host, const long long *info, int nlev, long long max_pairs, long long pair_cap,
                     void *stream);

/* No counterpart in the reference: splat_bin for callers that cannot allocate device memory (code in tight
 * serving loops, harnesses that forbid hipMalloc). The same binning as splat_bin with pair_cap > 0, but the
 * count and pair-phase workspaces live in the library's own device scratch, a static array of 64 MiB per
 * GPU, held from the library's load until the process ends. The caller still passes every input and output
 * (rec, rect, offsets, info, info_host and the pair buffers for pair_cap >= 1 pairs). Limit: the workspaces
 * of N splats and pair_cap pairs (splat_bin_count_workspace_bytes + splat_bin_pairs_workspace_bytes) must
 * fit the scratch: 12 bytes per pair plus 8 bytes per tile row and 256 splats for level tables of at most
 * 1,024 tile rows (pair_cap up to ~5M at 768 x 768), about 25 bytes per pair past that; a larger request
 * returns status 5 before any launch. No hipMalloc, hipFree or allocating library call; the first call on a device
 * looks up the scratch address and creates the device's scratch-order event, and the first call of a thread with a
 * pageable info_host creates its read-back event. Statuses as splat_bin. Every call on a GPU shares that GPU's
 * scratch, so calls are serialised on the device: each call's stream waits for the event recorded behind the
 * previous call's last kernel (on whatever stream or thread it was queued), under a per-device mutex. Calls on
 * other streams or threads therefore never overlap on the GPU, and a caller's stream may wait for another
 * caller's binning. Nothing in the scratch needs to start at zero: every region is written before it is read
 * within a call. */
int splat_bin_noalloc(const float *mu, const float *scale, const float *theta, const float *opacity,
                      const float *color, int C, int N, int H, int W, int TILE, float cutoff, const splat_levels *lv,
                      int flags, long long max_pairs, float *rec, int *rect, int *offsets, long long *info,
                      long long *info_host, long long pair_cap, int *gid_sorted, int *tile_starts, int *pair_splat,
                      int *pair_q, void *stream);

/* Measurement only, no counterpart in the reference: the calling thread's next tile-kernel launch (the
 * kernel of splat_render_fwd or splat_render_bwd) records the hipEvent_t events start and stop itself, at the
 * kernel's start and end (hipExtLaunchKernel), so their elapsed time is the kernel's duration without the host's
 * launch latency. The events are then disarmed; NULL, NULL disarms. Returns 1 when a pair armed earlier had not
 * been used by a launch, else 0. For benchmarks that bracket the kernels inside render steps. */
int splat_time_next_launch(void *start, void *stop);

/* Per-tile forward over the binned pairs of levels [lev_begin, lev_end) (TILE in {4, 8, 16}); levels
 * whose bit in levmask is clear are skipped (their pixels are not written).
 * Composite (no FIELDS; levels [0, 1) only): out[P,C], T[P], asum[P], fg[P,C] with background bg[C],
 * P = H*W. With UPS, the masked coarse levels' packed fields slog/sa/sac (inputs, written by an earlier
 * FIELDS call) are upsampled and added before compositing, and asum holds the unclamped S_a.
 * FIELDS: raw sums into the packed fields slog[Pt], sa[Pt] (unclamped), sac[Pt,C] at slot pbase[l] + p.
 * Replaces _render_fwd_cull_kernel, render_triton.py:423-517 (+ launch loops :538-599), and the
 * per-octave render + upsample + sum + composite of render_triton.py:864-876, :900-918, :962-978. */
int splat_render_fwd(const float *rec, const int *gid_sorted, const int *tile_starts, int C, int H, int W,
                     int TILE, int flags, const splat_levels *lv, int lev_begin, int lev_end,
                     unsigned levmask, const float *bg, float *out, float *T, float *asum, float *fg,
                     float *slog, float *sa, float *sac, void *stream);

/* Backward, step 1: per-tile kernel over the pairs of levels [lev_begin, lev_end) (levmask as in the
 * forward). For every pair (sorted position i) it sums over the tile's pixels the terms the parameter
 * gradients need and stores them, 6 + C floats, at pair_sums + pair_q[i] * (6 + C): splat-major order,
 * so the reduction reads them contiguously (splat_pair_sums_bytes sizes the buffer for any C).
 * Composite (levels [0, 1)): upstream gout[P,C] with the forward's T, asum, fg and bg; with bg_part set
 * ([C, ntiles0] floats, ntiles0 = level 0's tiles) it also writes per-tile partials of sum_p gout*T.
 * With UPS the S_a gradient is torch's clamp_min one (zero where S_a < 1e-8) and the pixel upstream
 * dS_log, dS_a, dS_ac is also written to dslog/dsa/dsac[0, P) for splat_upsample_adjoint.
 * FIELDS: upstream from the packed dslog[Pt], dsa[Pt], dsac[Pt,C] (bg_part must be NULL).
 * Replaces _render_bwd_cull_kernel, render_triton.py:602-720 (per-pair grads, :612-614), and the autograd
 * of the octave / coarse-fine composite, render_triton.py:918, :976-978. */
size_t splat_pair_sums_bytes(long long tot);
int splat_render_bwd(const float *rec, const int *gid_sorted, const int *tile_starts, const int *pair_q,
                     long long tot, int C, int H, int W, int TILE, int flags, const splat_levels *lv,
                     int lev_begin, int lev_end, unsigned levmask, const float *bg, const float *T,
                     const float *asum, const float *fg, const float *gout, float *dslog, float *dsa,
                     float *dsac, float *pair_sums, float *bg_part, void *stream);

/* FIELDS forward and backward of the coarse levels [lev_begin, lev_end) of a multi-level render in one
 * launch each, with every tile of level l split into splits[l] (1..1024) contiguous chunks of its pair list,
 * one workgroup per chunk (levels not in levmask take none). Dense coarse levels (few tiles with long
 * pair lists) then occupy every CU. The forward's chunks of a level with splits[l] > 1 write partial sums into
 * the workspace (splat_fields_split_workspace_bytes; 0 when no level is split) and a second kernel adds them
 * in chunk order: deterministic, the same fields as splat_render_fwd with FIELDS up to summation order. The
 * backward's chunks write the per-pair sums as splat_render_bwd with FIELDS does. flags: SPLAT_FLAG_ODDS or 0.
 * Replace the per-octave-group launches of _render_fwd_cull_kernel / _render_bwd_cull_kernel over the coarse
 * groups, render_triton.py:962-978 (forward, per octave) and :768-810 (their backward). */
size_t splat_fields_split_workspace_bytes(int C, int H, int W, int TILE, const splat_levels *lv, int lev_begin,
                                          int lev_end, unsigned levmask, const int *splits);
int splat_render_fields_split(const float *rec, const int *gid_sorted, const int *tile_starts, int C, int H, int W,
                              int TILE, int flags, const splat_levels *lv, int lev_begin, int lev_end,
                              unsigned levmask, const int *splits, float *slog, float *sa, float *sac, void *ws,
                              size_t ws_bytes, void *stream);
int splat_render_fields_split_bwd(const float *rec, const int *gid_sorted, const int *tile_starts, const int *pair_q,
                                  long long tot, int C, int H, int W, int TILE, int flags, const splat_levels *lv,
                                  int lev_begin, int lev_end, unsigned levmask, const int *splits, float *dslog,
                                  float *dsa, float *dsac, float *pair_sums, void *stream);

/* Backward of the upsample: the exact adjoint of the bilinear upsample of every masked coarse level,
 * from the level-0 upstream dslog/dsa/dsac[0, P) into the coarse levels' packed slots, deterministic
 * (two gather passes, no atomics). Replaces the autograd of F.interpolate at render_triton.py:864-876. */
size_t splat_upsample_adjoint_workspace_bytes(int C, int H, int W, int TILE, const splat_levels *lv);
int splat_upsample_adjoint(int C, int H, int W, int TILE, const splat_levels *lv, unsigned levmask,
                           float *dslog, float *dsa, float *dsac, void *ws, size_t ws_bytes, void *stream);

/* Backward, step 2: per-splat reduction of the pair sums into parameter gradients, written (not
 * accumulated), deterministic, no global atomics, one launch. Takes the binning's offsets (splat g owns the
 * sums records [offsets[g], offsets[g+1])); pair_splat is not read and may be NULL.
 * g_mu[N,2], g_scale[N,2] (w.r.t. the activated scale; with log_scale[N,2] given, the raw log-scales of a
 * SPLAT_FLAG_LOG_SCALE binning, w.r.t. those, chained as torch's softplus backward evaluates it),
 * g_theta[N] (NULL when there is no theta),
 * g_op[N], g_color[N,C]; g_bg[C] (NULL skips) from the nparts = ntiles0 per-tile partials of step 1.
 * One call covers the pairs of every level.
 * Replaces the index_add_ scatter and the g_bg reduction, render_triton.py:723-810. */
int splat_reduce_pairs(const float *rec, const int *offsets, const int *pair_splat, long long tot, int N,
                       int C, const float *pair_sums, const float *bg_part, int nparts, const float *log_scale,
                       float *g_mu, float *g_scale, float *g_theta, float *g_op, float *g_color, float *g_bg, void *stream);

/* Exact (unculled) path: every pixel sums every splat; pixel centres py[P], px[P] supplied by the caller.
 * Replaces _render_fwd_kernel / _render_bwd_kernel and their wrappers, render_triton.py:58-303. */
int splat_exact_fwd(const float *rec, int N, int C, const float *py, const float *px, int P, const float *bg,
                    float *out, float *T, float *asum, float *fg, void *stream);
size_t splat_exact_bwd_workspace_bytes(int N, int C, int P);
int splat_exact_bwd(const float *rec, int N, int C, const float *py, const float *px, int P, const float *bg,
                    const float *T, const float *asum, const float *fg, const float *gout, float *g_mu,
                    float *g_scale, float *g_theta, float *g_op, float *g_color, float *g_bg, void *ws,
                    size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SPLAT_RENDER_H */
