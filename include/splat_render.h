/* C-ABI of the gfx950 tile-binned Gaussian-splat renderer (libsplat_hip.so).
 *
 * Every entry point takes raw device pointers (fp32 / int32, contiguous), sizes and a hipStream_t passed
 * as `void *stream`; all work is enqueued on that stream and no entry point synchronises or allocates.
 * Buffers are owned by the caller; scratch memory comes in as (ws, ws_bytes), sized by the matching
 * *_workspace_bytes query. Every call returns 0 on success or a status code, with a message available
 * from splat_last_error() (thread-local):
 *   1 invalid argument, 2 HIP launch error, 3 unsupported configuration, 4 overflow, 5 workspace too small.
 *
 * Layouts (one image; callers loop over the batch like the reference does):
 *   mu[N,2] (y, x) in [0,1];  scale[N,2] (sy, sx) = softplus(log_scale) + 1e-4;  theta[N] or NULL;
 *   opacity[N];  color[N,C] with 1 <= C <= 4;  rec[N,16] the decoded splat record (64 B per splat).
 *   Pixel fields are row-major: [P] or [P,C] with P = H*W, p = y*W + x.
 *
 * The reference (bigwolfeman/gaussian-2d-splat-encoder) is Python + Triton; each function below replaces
 * the cited part of gaussian_splat_encoder/render_triton.py. A ctypes binding is in INTEGRATION.md.
 */
#ifndef SPLAT_RENDER_H
#define SPLAT_RENDER_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPLAT_FLAG_FIELDS 1 /* forward writes raw sums (S_log, S_a, S_ac); backward takes dS_* upstream */
#define SPLAT_FLAG_ODDS 2   /* colour weight a/(1-a) instead of a */

const char *splat_last_error(void);
int splat_abi_version(void);

/* Decoded splat records only (no binning), for the exact path.
 * Replaces the per-launch parameter split of render_triton.py:134-142 and :276-279. */
int splat_decode(const float *mu, const float *scale, const float *theta, const float *opacity,
                 const float *color, int C, int N, float *rec, void *stream);

/* Binning phase 1: decode + per-splat tile rect and pair count + exclusive scan of the counts.
 * Writes rec[N,16], rect[N,4] = (tx0, ty0, w, h), offsets[N+1] (offsets[N] = total pairs) and
 * info[2] (device int64): info[0] = total pairs, info[1] = error bits (1 empty rect, 2 int32 overflow).
 * The caller reads info once to size the pair buffers and to apply its pair budget.
 * Replaces render_triton.py:362-391 (_build_tiles up to the tot sync) and :520-535 (param gathers). */
size_t splat_bin_count_workspace_bytes(int N);
int splat_bin_count(const float *mu, const float *scale, const float *theta, const float *opacity,
                    const float *color, int C, int N, int H, int W, int TILE, float cutoff, float *rec,
                    int *rect, int *offsets, long long *info, void *ws, size_t ws_bytes, void *stream);

/* Binning phase 2: expand rects into pairs, stable radix sort on the tile id, CSR tile starts.
 * gid_sorted[max(tot,1)] lists splat ids ordered by (tile, splat id); tile_starts[nt+1].
 * tot == 0 gives gid_sorted = {0} and all-zero starts, as the reference does.
 * Optional (NULL skips) maps over the splat-major pair order q (splat g owns q in [offsets[g], offsets[g+1])),
 * used by the backward's per-splat reduction: pair_splat[tot] = splat of q, pair_inv[tot] = sorted position
 * of q.
 * Replaces render_triton.py:392-409. */
size_t splat_bin_pairs_workspace_bytes(int N, int nt, long long tot);
int splat_bin_pairs(const int *rect, const int *offsets, int N, int H, int W, int TILE, long long tot,
                    int *gid_sorted, int *tile_starts, int *pair_splat, int *pair_inv, void *ws,
                    size_t ws_bytes, void *stream);

/* Per-tile forward compositing over the binned pairs (TILE in {4, 8, 16}).
 * Composite (flags without FIELDS): out[P,C], T[P], asum[P], fg[P,C] with background bg[C].
 * FIELDS: slog[P], sa[P] (unclamped), sac[P,C]; every pixel is written, empty tiles get zeros.
 * Replaces _render_fwd_cull_kernel, render_triton.py:423-517 (+ launch loops :538-599). */
int splat_render_fwd(const float *rec, const int *gid_sorted, const int *tile_starts, int C, int H, int W,
                     int TILE, int flags, const float *bg, float *out, float *T, float *asum, float *fg,
                     float *slog, float *sa, float *sac, void *stream);

/* Backward, step 1: per-tile kernel over the same pairs. For every pair (sorted position i) it sums over
 * the tile's pixels the terms the parameter gradients need and stores them in pair_sums[i] (12 floats,
 * splat_pair_sums_bytes). Composite: upstream gout[P,C] with the forward's T, asum, fg and bg; with
 * bg_part set ([C, nt] floats) it also writes per-tile partials of sum_p gout*T. FIELDS: upstream
 * dslog[P], dsa[P], dsac[P,C] (bg_part must be NULL).
 * Replaces _render_bwd_cull_kernel, render_triton.py:602-720 (per-pair grads, :612-614). */
size_t splat_pair_sums_bytes(long long tot);
int splat_render_bwd(const float *rec, const int *gid_sorted, const int *tile_starts, long long tot, int C,
                     int H, int W, int TILE, int flags, const float *bg, const float *T, const float *asum,
                     const float *fg, const float *gout, const float *dslog, const float *dsa,
                     const float *dsac, float *pair_sums, float *bg_part, void *stream);

/* Backward, step 2: per-splat reduction of the pair sums into parameter gradients, written (not
 * accumulated), deterministic, no global atomics. Takes the binning's offsets, pair_splat and pair_inv.
 * g_mu[N,2], g_scale[N,2] (w.r.t. the activated scale), g_theta[N] (NULL when there is no theta),
 * g_op[N], g_color[N,C]; g_bg[C] (NULL skips) from the nparts = nt per-tile partials of step 1.
 * Replaces the index_add_ scatter and the g_bg reduction, render_triton.py:723-810. */
size_t splat_reduce_workspace_bytes(long long tot);
int splat_reduce_pairs(const float *rec, const int *offsets, const int *pair_splat, const int *pair_inv,
                       long long tot, int N, int C, const float *pair_sums, const float *bg_part, int nparts,
                       float *g_mu, float *g_scale, float *g_theta, float *g_op, float *g_color,
                       float *g_bg, void *ws, size_t ws_bytes, void *stream);

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
