/* CPU oracle in C. TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library, and only as the checker.
 *
 * Compiled with -ffp-contract=off (see Makefile) so every float32 operation of the binning is rounded
 * separately, as the reference's elementwise torch ops are.
 *
 *   orc_rects     render_triton.py:364-377   fp32 rect + count per splat
 *   orc_pairs     render_triton.py:386-409   pairs ordered by (tile, splat), CSR tile starts
 *                                             (a stable counting sort; independent of binning.py's
 *                                              repeat/argsort formulation)
 *   orc_fwd_cull  render_triton.py:423-517   cull forward, float64 arithmetic over the fp32 pair list;
 *                                             fields or composite, alpha or odds weights
 *   orc_bwd_cull  render_triton.py:602-720   cull backward: the reference's per-pair analytic gradient
 *                 render_triton.py:723-810   formulas in float64, summed per splat; g_bg (:764)
 *
 * The per-tile loops run on OpenMP threads (tiles are independent; the backward sums per-thread
 * accumulators in thread order), so full-size frames (2048 x 2048, 31M pairs) check in seconds.
 */
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float clampf_(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

void orc_rects(const float* mu, const float* scale, int N, int H, int W, int TILE, float cutoff,
               int* tx0, int* tx1, int* ty0, int* ty1, int* counts) {
    const int ntx = (W + TILE - 1) / TILE, nty = (H + TILE - 1) / TILE;
    const float fW = (float)W, fH = (float)H, fT = (float)TILE;
    for (int g = 0; g < N; ++g) {
        const float my = mu[2 * g + 0], mx = mu[2 * g + 1];
        const float sy = scale[2 * g + 0], sx = scale[2 * g + 1];
        const float cx = mx * fW;
        const float cy = my * fH;
        const float smax = sy >= sx ? sy : sx;
        const float r = cutoff * smax;
        const float rx = r * fW;
        const float ry = r * fH;
        const float a = cx - rx, b = cx + rx, c = cy - ry, d = cy + ry;
        tx0[g] = (int)clampf_(floorf(a / fT), 0.0f, (float)(ntx - 1));
        tx1[g] = (int)clampf_(floorf(b / fT), 0.0f, (float)(ntx - 1));
        ty0[g] = (int)clampf_(floorf(c / fT), 0.0f, (float)(nty - 1));
        ty1[g] = (int)clampf_(floorf(d / fT), 0.0f, (float)(nty - 1));
        counts[g] = (tx1[g] - tx0[g] + 1) * (ty1[g] - ty0[g] + 1);
    }
}

/* Counting sort by tile, visiting splats in ascending order: within a tile, splats come out ascending,
 * which is the stable order of render_triton.py:405-407. gid_sorted must hold sum(counts) entries. */
int64_t orc_pairs(const int* tx0, const int* tx1, const int* ty0, const int* ty1, int N, int ntx, int nt,
                  int* gid_sorted, int* tile_starts) {
    int64_t* cnt = (int64_t*)calloc((size_t)nt + 1, sizeof(int64_t));
    for (int g = 0; g < N; ++g)
        for (int ty = ty0[g]; ty <= ty1[g]; ++ty)
            for (int tx = tx0[g]; tx <= tx1[g]; ++tx) cnt[ty * ntx + tx + 1]++;
    for (int t = 0; t < nt; ++t) cnt[t + 1] += cnt[t];
    for (int t = 0; t <= nt; ++t) tile_starts[t] = (int)cnt[t];
    const int64_t tot = cnt[nt];
    for (int g = 0; g < N; ++g)
        for (int ty = ty0[g]; ty <= ty1[g]; ++ty)
            for (int tx = tx0[g]; tx <= tx1[g]; ++tx) gid_sorted[cnt[ty * ntx + tx]++] = g;
    free(cnt);
    return tot;
}

/* Splat parameters of one batch, as the kernels receive them (activated scale). */
typedef struct {
    const float* mu;      /* [N,2] (y,x) */
    const float* scale;   /* [N,2] (sy,sx) */
    const float* theta;   /* [N] or NULL */
    const float* opacity; /* [N] */
    const float* color;   /* [N,C] */
    double* cs;           /* [N] cos(theta), filled by trig_tables */
    double* sn;           /* [N] sin(theta) */
} orc_splats;

/* The splats' rotation: cos and sin of the float32 angle in float64 (the default), or, after orc_set_rot32(1), each
 * rounded to the nearest float32 value: the precision in which the reference holds its rotation (cos and sin of a
 * float32 angle in float32 arithmetic, render_triton.py:95-96, :480-481) and in which the HIP decode stores it. */
static int g_rot32 = 0;
void orc_set_rot32(int on) { g_rot32 = on; }

static void trig_tables(orc_splats* s, int N) {
    s->cs = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
    s->sn = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
    for (int g = 0; g < N; ++g) {
        const double th = s->theta ? (double)s->theta[g] : 0.0;
        double c = s->theta ? cos(th) : 1.0, sn = s->theta ? sin(th) : 0.0;
        if (g_rot32) {
            c = (double)(float)c;
            sn = (double)(float)sn;
        }
        s->cs[g] = c;
        s->sn[g] = sn;
    }
}
static void trig_free(orc_splats* s) { free(s->cs); free(s->sn); }

/* The offsets of a pixel centre from a splat centre: the exact difference of the two float32 values (the default),
 * or, after orc_set_off32(1), that difference rounded to float32, as the reference's float32 arithmetic and the HIP
 * kernels form it. */
static int g_off32 = 0;
void orc_set_off32(int on) { g_off32 = on; }

/* The alpha clamp 1 - 1e-4 as the reference applies it to float32 alphas (render_triton.py:106, :235, :491, :684):
 * the float32 value nearest 0.9999, so 1 - a on the clamp is 1.00017e-4 there, not 1e-4. */
#define ORC_CLAMP 0.99989998340606689453125

/* Pixel centre of the cull kernels: fp32 (i + 0.5) / size (render_triton.py:455-456). */
static inline double centre(int i, int size) { return (double)(((float)i + 0.5f) / (float)size); }

static inline void splat_alpha(const orc_splats* s, int g, double py, double px, double* ry_o, double* rx_o,
                               double* f_o, double* fo_o, double* a_o) {
    double dy = py - (double)s->mu[2 * g], dx = px - (double)s->mu[2 * g + 1];
    if (g_off32) {
        dy = (double)((float)py - s->mu[2 * g]);
        dx = (double)((float)px - s->mu[2 * g + 1]);
    }
    double ry = dy, rx = dx;
    if (s->theta) {
        const double c = s->cs[g], sn = s->sn[g];
        ry = c * dy + sn * dx;
        rx = -sn * dy + c * dx;
    }
    const double sy = (double)s->scale[2 * g], sx = (double)s->scale[2 * g + 1];
    const double maha = ry * ry / (sy * sy) + rx * rx / (sx * sx);
    const double f = exp(-0.5 * maha);
    const double fo = f * (double)s->opacity[g];
    *ry_o = ry; *rx_o = rx; *f_o = f; *fo_o = fo;
    *a_o = fo < ORC_CLAMP ? fo : ORC_CLAMP;
}

/* Forward over one batch. fields != 0: write S_log[P], S_a[P] (unclamped), S_ac[P*C], and into T[P], asum[P] and
 * fg[P*C] the fields' sensitivities to a relative change of every unclamped alpha, d/de at a -> a (1 + e):
 * sum a / (1 - a), sum a dw/da and sum |c| a dw/da over the pixel's pairs (dw/da = 1, or 1 / (1 - a)^2 for odds
 * weights; 0 for a pair on the clamp), the condition of each field under float32 falloff rounding; else
 * composite into out[P*C], T[P], asum[P], fg[P*C] with bg[C]. */
void orc_fwd_cull(const float* mu, const float* scale, const float* theta, const float* opacity,
                  const float* color, int C, const int* gid_sorted, const int* tile_starts, int H, int W,
                  int TILE, int odds, int fields, const float* bg, double* out, double* T, double* asum,
                  double* fg, double* slog, double* sa, double* sac) {
    const int ntx = (W + TILE - 1) / TILE, nty = (H + TILE - 1) / TILE;
    int N = 0;
    for (int i = 0; i < tile_starts[ntx * nty]; ++i) if (gid_sorted[i] + 1 > N) N = gid_sorted[i] + 1;
    orc_splats s = {mu, scale, theta, opacity, color, NULL, NULL};
    trig_tables(&s, N);
    /* tiles are independent: one thread per tile at a time */
#pragma omp parallel for schedule(dynamic, 4)
    for (int t = 0; t < ntx * nty; ++t) {
            const int ty = t / ntx, tx = t % ntx;
            double acc[16];
            for (int ly = 0; ly < TILE; ++ly)
                for (int lx = 0; lx < TILE; ++lx) {
                    const int yp = ty * TILE + ly, xp = tx * TILE + lx;
                    if (yp >= H || xp >= W) continue;
                    const double py = centre(yp, H), px = centre(xp, W);
                    double S_log = 0.0, S_a = 0.0, K_log = 0.0, K_a = 0.0, K_ac[16];
                    for (int c = 0; c < C; ++c) acc[c] = K_ac[c] = 0.0;
                    for (int i = tile_starts[t]; i < tile_starts[t + 1]; ++i) {
                        const int g = gid_sorted[i];
                        double ry, rx, f, fo, a;
                        splat_alpha(&s, g, py, px, &ry, &rx, &f, &fo, &a);
                        S_log += log(1.0 - a);
                        const double w = odds ? a / (1.0 - a) : a;
                        S_a += w;
                        for (int c = 0; c < C; ++c) acc[c] += w * (double)color[g * C + c];
                        if (fields && fo < ORC_CLAMP) {
                            const double k = odds ? a / ((1.0 - a) * (1.0 - a)) : a;
                            K_log += a / (1.0 - a);
                            K_a += k;
                            for (int c = 0; c < C; ++c) K_ac[c] += k * fabs((double)color[g * C + c]);
                        }
                    }
                    const int p = yp * W + xp;
                    if (fields) {
                        slog[p] = S_log; sa[p] = S_a;
                        for (int c = 0; c < C; ++c) sac[p * C + c] = acc[c];
                        T[p] = K_log; asum[p] = K_a;
                        for (int c = 0; c < C; ++c) fg[p * C + c] = K_ac[c];
                    } else {
                        const double Tp = exp(S_log), as = S_a > 1e-8 ? S_a : 1e-8;
                        T[p] = Tp; asum[p] = as;
                        for (int c = 0; c < C; ++c) {
                            const double f = acc[c] / as;
                            fg[p * C + c] = f;
                            out[p * C + c] = (1.0 - Tp) * f + Tp * (double)bg[c];
                        }
                    }
                }
        }
    trig_free(&s);
}

/* Backward over one batch. fields != 0: upstream dS_log[P], dS_a[P], dS_ac[P*C]; else upstream gout[P*C]
 * with the saved T, asum, fg and bg. Per-splat outputs are zeroed here and summed over pairs.
 * g_mag (optional, [N, 6 + C]): per splat and gradient component (mu_y, mu_x, s_y, s_x, theta, opacity,
 * colour[C]) the sum over the splat's pixel-pairs of the magnitudes of every term that enters that component:
 * the scale against which a per-splat relative error of the component is meaningful. Each pixel-pair's term is
 * the reference's product of factors (render_triton.py:688-710) with every sum in it replaced by the sum of its
 * terms' magnitudes: da by m_da = |dS_log| |u| + (|dS_a| + sum_c |dS_ac[c] col[c]|) u^k (k = 2 for odds, 0 for
 * alpha), and the two summands of each of g_mu and g_theta taken apart (|gry c| + |grx s|, |gry rx| + |grx ry|).
 * In composite mode |dS_log| and |dS_a| are themselves the composite's per-channel terms summed in magnitude
 * (T sum_c |gout[c] (bg[c] - fg[c])| and sum_c |gout[c] (1 - T) fg[c]| / asum, render_triton.py:650-654).
 * Tiles run in parallel (OpenMP), each thread into accumulators of its own, summed in thread order. */
enum { ACC_MU = 0, ACC_SC = 2, ACC_TH = 4, ACC_OP = 5, ACC_COL = 6 };

void orc_bwd_cull(const float* mu, const float* scale, const float* theta, const float* opacity,
                  const float* color, int C, int N, const int* gid_sorted, const int* tile_starts, int H,
                  int W, int TILE, int odds, int fields, const float* bg, const double* T,
                  const double* asum, const double* fg, const double* gout, const double* dslog_in,
                  const double* dsa_in, const double* dsac_in, double* g_mu, double* g_scale,
                  double* g_theta, double* g_op, double* g_col, double* g_bg, double* g_mag) {
    orc_splats s = {mu, scale, theta, opacity, color, NULL, NULL};
    trig_tables(&s, N);
    const int ntx = (W + TILE - 1) / TILE, nty = (H + TILE - 1) / TILE;
    const int KG = ACC_COL + C;   /* gradient components; their magnitude sums follow at KG + k */
    const int K = 2 * KG;
    int nth = 1;
#ifdef _OPENMP
    nth = omp_get_max_threads();
#endif
    double* acc = (double*)calloc((size_t)nth * (size_t)(N > 0 ? N : 1) * K, sizeof(double));
    double* bgacc = (double*)calloc((size_t)nth * 16, sizeof(double));
#pragma omp parallel num_threads(nth)
    {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        double* A = acc + (size_t)tid * (size_t)(N > 0 ? N : 1) * K;
        double* gb = bgacc + (size_t)tid * 16;
        double dS_ac[16];
        double dS_log_m, dS_a_m;   /* magnitudes: the composite's per-channel terms summed in absolute value */
#pragma omp for schedule(dynamic, 4)
        for (int t = 0; t < ntx * nty; ++t) {
            const int ty = t / ntx, tx = t % ntx;
            for (int ly = 0; ly < TILE; ++ly)
                for (int lx = 0; lx < TILE; ++lx) {
                    const int yp = ty * TILE + ly, xp = tx * TILE + lx;
                    if (yp >= H || xp >= W) continue;
                    const int p = yp * W + xp;
                    const double py = centre(yp, H), px = centre(xp, W);
                    double dS_log, dS_a;
                    if (fields) {
                        dS_log = dslog_in[p]; dS_a = dsa_in[p];
                        for (int c = 0; c < C; ++c) dS_ac[c] = dsac_in[p * C + c];
                        dS_log_m = fabs(dS_log); dS_a_m = fabs(dS_a);
                    } else {
                        /* render_triton.py:650-654 */
                        double dTp = 0.0, sfg = 0.0, dTp_m = 0.0, sfg_m = 0.0;
                        for (int c = 0; c < C; ++c) {
                            const double go = gout[p * C + c], dfg = go * (1.0 - T[p]);
                            dTp += go * ((double)bg[c] - fg[p * C + c]);
                            sfg += dfg * fg[p * C + c];
                            dTp_m += fabs(go * ((double)bg[c] - fg[p * C + c]));
                            sfg_m += fabs(dfg * fg[p * C + c]);
                            dS_ac[c] = dfg / asum[p];
                            gb[c] += go * T[p];
                        }
                        dS_log = dTp * T[p];
                        dS_a = -sfg / asum[p];
                        dS_log_m = dTp_m * fabs(T[p]);
                        dS_a_m = sfg_m / fabs(asum[p]);
                    }
                    for (int i = tile_starts[t]; i < tile_starts[t + 1]; ++i) {
                        const int g = gid_sorted[i];
                        double* a_g = A + (size_t)g * K;
                        double ry, rx, f, fo, a;
                        splat_alpha(&s, g, py, px, &ry, &rx, &f, &fo, &a);
                        /* render_triton.py:688-710 */
                        const double u = 1.0 / (1.0 - a);
                        double col_term = 0.0, col_abs = 0.0;
                        for (int c = 0; c < C; ++c) {
                            col_term += dS_ac[c] * (double)color[g * C + c];
                            col_abs += fabs(dS_ac[c] * (double)color[g * C + c]);
                        }
                        double da, cw, mag;
                        if (odds) {
                            da = -dS_log * u + (dS_a + col_term) * u * u; cw = a * u;
                            mag = dS_log_m * fabs(u) + (dS_a_m + col_abs) * u * u;
                        } else {
                            da = -dS_log * u + dS_a + col_term; cw = a;
                            mag = dS_log_m * fabs(u) + dS_a_m + col_abs;
                        }
                        double* m_g = a_g + KG;
                        for (int c = 0; c < C; ++c) {
                            a_g[ACC_COL + c] += cw * dS_ac[c];
                            m_g[ACC_COL + c] += fabs(cw * dS_ac[c]);
                        }
                        const double da_fo = fo < ORC_CLAMP ? da : 0.0;
                        const double mag_fo = fo < ORC_CLAMP ? mag : 0.0;
                        const double op = (double)opacity[g];
                        const double sy = (double)scale[2 * g], sx = (double)scale[2 * g + 1];
                        a_g[ACC_OP] += da_fo * f;
                        m_g[ACC_OP] += mag_fo * f;
                        const double gm = (da_fo * op) * (-0.5 * f), gmm = (mag_fo * op) * (0.5 * f);
                        a_g[ACC_SC + 0] += gm * (-2.0 * ry * ry) / (sy * sy * sy);
                        a_g[ACC_SC + 1] += gm * (-2.0 * rx * rx) / (sx * sx * sx);
                        m_g[ACC_SC + 0] += gmm * (2.0 * ry * ry) / (sy * sy * sy);
                        m_g[ACC_SC + 1] += gmm * (2.0 * rx * rx) / (sx * sx * sx);
                        const double gry = gm * 2.0 * ry / (sy * sy), grx = gm * 2.0 * rx / (sx * sx);
                        const double grym = gmm * 2.0 * fabs(ry) / (sy * sy), grxm = gmm * 2.0 * fabs(rx) / (sx * sx);
                        if (theta) {
                            const double cth = s.cs[g], sth = s.sn[g];
                            a_g[ACC_TH] += gry * rx - grx * ry;
                            a_g[ACC_MU + 0] += -(gry * cth - grx * sth);
                            a_g[ACC_MU + 1] += -(gry * sth + grx * cth);
                            m_g[ACC_TH] += grym * fabs(rx) + grxm * fabs(ry);
                            m_g[ACC_MU + 0] += grym * fabs(cth) + grxm * fabs(sth);
                            m_g[ACC_MU + 1] += grym * fabs(sth) + grxm * fabs(cth);
                        } else {
                            a_g[ACC_MU + 0] += -gry;
                            a_g[ACC_MU + 1] += -grx;
                            m_g[ACC_MU + 0] += grym;
                            m_g[ACC_MU + 1] += grxm;
                        }
                    }
                }
        }
    }
    for (int g = 0; g < N; ++g) {
        double v[2 * (ACC_COL + 16)];
        for (int k = 0; k < K; ++k) v[k] = 0.0;
        for (int th = 0; th < nth; ++th) {
            const double* a_g = acc + ((size_t)th * (size_t)N + (size_t)g) * K;
            for (int k = 0; k < K; ++k) v[k] += a_g[k];
        }
        g_mu[2 * g] = v[ACC_MU]; g_mu[2 * g + 1] = v[ACC_MU + 1];
        g_scale[2 * g] = v[ACC_SC]; g_scale[2 * g + 1] = v[ACC_SC + 1];
        if (g_theta) g_theta[g] = v[ACC_TH];
        g_op[g] = v[ACC_OP];
        if (g_mag)
            for (int k = 0; k < KG; ++k) g_mag[(size_t)g * KG + k] = v[KG + k];
        for (int c = 0; c < C; ++c) g_col[g * C + c] = v[ACC_COL + c];
    }
    if (g_bg)
        for (int c = 0; c < C; ++c) {
            double x = 0.0;
            for (int th = 0; th < nth; ++th) x += bgacc[th * 16 + c];
            g_bg[c] = x;
        }
    free(acc);
    free(bgacc);
    trig_free(&s);
}

/* The reference's own CPU renderer restated in C (render.py:34-58, 90-110): exact, every pixel sums
 * every splat, float32 arithmetic, linspace pixel centres passed in. Used for the CPU baseline timing of
 * a bounded band of rows. out[(row - row0) * W * C + x * C + c]. */
void orc_exact_rows_f32(const float* mu, const float* scale, const float* theta, const float* opacity,
                        const float* color, int C, int N, const float* ys, const float* xs, int row0,
                        int row1, int W, const float* bg, float* out) {
    float acc[16];
    for (int yy = row0; yy < row1; ++yy)
        for (int xx = 0; xx < W; ++xx) {
            const float py = ys[yy], px = xs[xx];
            float S_log = 0.0f, S_a = 0.0f;
            for (int c = 0; c < C; ++c) acc[c] = 0.0f;
            for (int g = 0; g < N; ++g) {
                const float dy = py - mu[2 * g], dx = px - mu[2 * g + 1];
                float ry = dy, rx = dx;
                if (theta) {
                    const float c = cosf(theta[g]), sn = sinf(theta[g]);
                    ry = c * dy + sn * dx;
                    rx = -sn * dy + c * dx;
                }
                const float sy = scale[2 * g], sx = scale[2 * g + 1];
                const float maha = ry * ry / (sy * sy) + rx * rx / (sx * sx);
                float a = expf(-0.5f * maha) * opacity[g];
                if (a > (float)ORC_CLAMP) a = (float)ORC_CLAMP;
                S_log += log1pf(-a);
                S_a += a;
                for (int c = 0; c < C; ++c) acc[c] += a * color[g * C + c];
            }
            const float T = expf(S_log), as = S_a > 1e-8f ? S_a : 1e-8f;
            for (int c = 0; c < C; ++c)
                out[((yy - row0) * W + xx) * C + c] = (1.0f - T) * (acc[c] / as) + T * bg[c];
        }
}
