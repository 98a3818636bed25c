/* s2s_oracle.c - CPU restatement of the swin2sr crate's CPU path (f32).
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT: the checker for the HIP backend's parity
 * tests and the CPU baseline bench.py times. Nothing in the HIP library calls
 * this code, and the library has no CPU fallback.
 *
 * Built with `-ffp-contract=off`: the reference is Rust, which never fuses a
 * multiply and an add, so every `acc += w * x` below is a rounded multiply
 * followed by a rounded add, in the order the reference's loop performs them.
 * The parallel splits (OpenMP) are always over independent outputs, as the
 * reference's rayon splits are (src/cpu.rs:46-77), so results do not depend on
 * the thread count.
 *
 * Pinning - how each function is checked by tests/test_oracle.py against
 * something other than its own formula:
 *   plan/index/region/pad_reflect : torch.roll/window_partition/calculate_mask and
 *       torch.cat(flip) restated with numpy slicing (independent route), bit-exact.
 *   conv3x3, conv1x1, linear       : float64 definitions (numpy einsum), 1e-5.
 *   conv3x3_shuffle2               : conv3x3 followed by pixel_shuffle2 (as the
 *       reference's own selftest does, src/cpu.rs:2064-2098) and numpy
 *       depth-to-space, 1e-5.
 *   channel_layer_norm             : float64 two-pass LayerNorm, 1e-5.
 *   fast_exp                       : sqrt(2)*exp(x) (what the reference's series
 *       computes, see below) within 2e-5 relative over [-88, 0].
 *   gelu                           : scipy.special.erf form in float64, 1e-6.
 *   gather/scatter                 : numpy roll + window_partition; inverse pair.
 *   attention                      : float64 F.normalize/softmax transcription
 *       (src/cpu.rs:2242-2314), 2e-5.
 *   cpb table                      : float64 numpy restatement of
 *       tools/convert.py:141-167 + network_swin2sr.py:109-136, 1e-5.
 *   bicubic_resize                 : the reference's torch KAT
 *       (tests/data/bicubic_{in_40x32,out_148x116}.npy), < 2e-5.
 *   forward composition            : golden vectors written by
 *       tests/golden/make_golden.py from the reference's PyTorch network.
 */
#include "s2s_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#ifdef __AVX2__
#include <immintrin.h>
#endif

#define LN_EPS 1e-5f
/* reference src/cpu.rs:68: below this many outputs an op stays on one thread */
#define PAR_MIN (1L << 14)

static __thread char g_err[512];

const char *orc_last_error(void) { return g_err; }

int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

static void *xalloc(size_t bytes) {
    void *p = NULL;
    if (posix_memalign(&p, 64, bytes ? bytes : 64) != 0) {
        fprintf(stderr, "oracle: out of memory (%zu bytes)\n", bytes);
        abort();
    }
    return p;
}

static float *falloc(long n) { return (float *)xalloc((size_t)n * sizeof(float)); }
static float *fzeros(long n) {
    float *p = falloc(n);
    memset(p, 0, (size_t)n * sizeof(float));
    return p;
}

/* ------------------------------------------------------------------------- */
/* Plan: reference src/plan.rs                                              */
/* ------------------------------------------------------------------------- */

/* src/plan.rs:39-47: pad to the NEXT window multiple, always >= one window. */
void orc_plan_new(int h, int w, int win, int c, orc_plan *p) {
    p->h = h;
    p->w = w;
    p->hp = (h / win + 1) * win;
    p->wp = (w / win + 1) * win;
    p->win = win;
    p->nwh = p->hp / win;
    p->nww = p->wp / win;
    p->nw = p->nwh * p->nww;
    p->n = win * win;
    p->c = c;
}

void orc_plan_explicit(int hp, int wp, int win, int c, orc_plan *p) {
    p->h = hp;
    p->w = wp;
    p->hp = hp;
    p->wp = wp;
    p->win = win;
    p->nwh = hp / win;
    p->nww = wp / win;
    p->nw = p->nwh * p->nww;
    p->n = win * win;
    p->c = c;
}

/* src/plan.rs:59-65 */
int orc_shift_for(const orc_plan *p, int b) { return (b % 2 == 1) ? p->win / 2 : 0; }

/* src/plan.rs:72-78: token (wi, t) reads ((wh*win+i+shift) % hp, (ww*win+j+shift) % wp). */
void orc_index(const orc_plan *p, int wi, int t, int shift, int *y, int *x) {
    int wh = wi / p->nww, ww = wi % p->nww;
    int i = t / p->win, j = t % p->win;
    *y = (wh * p->win + i + shift) % p->hp;
    *x = (ww * p->win + j + shift) % p->wp;
}

/* src/plan.rs:100-108 */
int orc_region_of(int a, int len, int win, int shift) {
    if (a + win < len) return 0;
    if (a + shift < len) return 1;
    return 2;
}

/* src/plan.rs:84-89: the band on the UNWRAPPED (rolled-plane) coordinate. */
void orc_region(const orc_plan *p, int wi, int t, int shift, uint8_t *ry, uint8_t *rx) {
    int wh = wi / p->nww, ww = wi % p->nww;
    int i = t / p->win, j = t % p->win;
    *ry = (uint8_t)orc_region_of(wh * p->win + i, p->hp, p->win, shift);
    *rx = (uint8_t)orc_region_of(ww * p->win + j, p->wp, p->win, shift);
}

void orc_window_map(const orc_plan *p, int shift, int32_t *yx, uint8_t *reg) {
    for (int wi = 0; wi < p->nw; ++wi)
        for (int t = 0; t < p->n; ++t) {
            long k = (long)wi * p->n + t;
            int y, x;
            orc_index(p, wi, t, shift, &y, &x);
            yx[2 * k] = y;
            yx[2 * k + 1] = x;
            orc_region(p, wi, t, shift, &reg[2 * k], &reg[2 * k + 1]);
        }
}

/* src/plan.rs:116-140: rows first (full width), then columns (padded height);
 * the pad is the mirror of the whole plane, sy = 2h-1-y. */
void orc_pad_reflect(const float *x, int c, int h, int w, int hp, int wp, float *out) {
    float *rows = falloc((long)c * hp * w);
    for (int ch = 0; ch < c; ++ch)
        for (int y = 0; y < hp; ++y) {
            int ym = y < 2 * h - 1 ? y : 2 * h - 1;
            int sy = y < h ? y : 2 * h - 1 - ym;
            memcpy(&rows[((long)ch * hp + y) * w], &x[((long)ch * h + sy) * w],
                   (size_t)w * sizeof(float));
        }
    for (int ch = 0; ch < c; ++ch)
        for (int y = 0; y < hp; ++y)
            for (int bx = 0; bx < wp; ++bx) {
                int xm = bx < 2 * w - 1 ? bx : 2 * w - 1;
                int sx = bx < w ? bx : 2 * w - 1 - xm;
                out[((long)ch * hp + y) * wp + bx] = rows[((long)ch * hp + y) * w + sx];
            }
    free(rows);
}

/* ------------------------------------------------------------------------- */
/* Convolutions: reference src/cpu.rs:400-577                               */
/* ------------------------------------------------------------------------- */

/* cpu::conv3x3 -> lg::conv3x3s1p1 (src/cpu.rs:400-414). The toolkit's exact
 * summation order is not in the reference tree (lightgpu is an un-vendored git
 * dependency); this follows the DEFINITION order the reference's selftest
 * holds it to (src/cpu.rs:2029-2062): bias first, then ci, ky, kx ascending,
 * taps outside the plane skipped. Four output channels share each input row
 * pass; every output element still accumulates in that order. */
void orc_conv3x3(const float *in, int cin, int h, int w, const float *wgt, int cout,
                 const float *bias, float *out) {
    long hw = (long)h * w;
    int ngrp = (cout + 3) / 4;
    long tasks = (long)ngrp * h;
#pragma omp parallel for schedule(dynamic, 4) if (hw * cout >= PAR_MIN)
    for (long task = 0; task < tasks; ++task) {
        int g = (int)(task / h), y = (int)(task % h);
        int co0 = g * 4, nco = cout - co0 < 4 ? cout - co0 : 4;
        float *dd[4];
        for (int j = 0; j < 4; ++j) dd[j] = out + ((long)(co0 + (j < nco ? j : 0)) * h + y) * w;
        for (int j = 0; j < nco; ++j)
            for (int x = 0; x < w; ++x) dd[j][x] = bias[co0 + j];
        for (int ci = 0; ci < cin; ++ci) {
            const float *ip = in + (long)ci * hw;
            for (int ky = 0; ky < 3; ++ky) {
                int sy = y + ky - 1;
                if (sy < 0 || sy >= h) continue;
                const float *row = ip + (long)sy * w;
                for (int kx = 0; kx < 3; ++kx) {
                    int x0 = kx == 0 ? 1 : 0;
                    int x1 = kx == 2 ? w - 1 : w;
                    const float *s = row + (kx - 1);
                    if (nco == 4) {
                        float w0 = wgt[(((long)(co0 + 0) * cin + ci) * 3 + ky) * 3 + kx];
                        float w1 = wgt[(((long)(co0 + 1) * cin + ci) * 3 + ky) * 3 + kx];
                        float w2 = wgt[(((long)(co0 + 2) * cin + ci) * 3 + ky) * 3 + kx];
                        float w3 = wgt[(((long)(co0 + 3) * cin + ci) * 3 + ky) * 3 + kx];
                        float *a0 = dd[0], *a1 = dd[1], *a2 = dd[2], *a3 = dd[3];
                        for (int x = x0; x < x1; ++x) {
                            float v = s[x];
                            a0[x] += w0 * v;
                            a1[x] += w1 * v;
                            a2[x] += w2 * v;
                            a3[x] += w3 * v;
                        }
                    } else {
                        for (int j = 0; j < nco; ++j) {
                            float wv = wgt[(((long)(co0 + j) * cin + ci) * 3 + ky) * 3 + kx];
                            float *a = dd[j];
                            for (int x = x0; x < x1; ++x) a[x] += wv * s[x];
                        }
                    }
                }
            }
        }
    }
}

/* cpu::conv_row + row_accumulate (src/cpu.rs:432-483): one output row of one
 * channel, bias first, then ci outer, ky over the rows inside the plane, and
 * per input row the three kx taps (edges peeled). */
static void conv_row(const float *in, int cin, int h, int w, const float *wc, float b, int y,
                     float *dest) {
    for (int x = 0; x < w; ++x) dest[x] = b;
    int ky0 = (y == 0) ? 1 : 0;
    int ky1 = (y + 1 == h) ? 1 : 2;
    long hw = (long)h * w;
    for (int ci = 0; ci < cin; ++ci) {
        const float *ic = in + ci * hw;
        const float *k = wc + ci * 9;
        for (int ky = ky0; ky <= ky1; ++ky) {
            const float *srow = ic + (long)(y + ky - 1) * w;
            const float *krow = k + ky * 3;
            if (w == 1) {
                dest[0] += krow[1] * srow[0];
                continue;
            }
            dest[0] += krow[1] * srow[0];
            dest[0] += krow[2] * srow[1];
            for (int x = 1; x < w - 1; ++x) {
                dest[x] += krow[0] * srow[x - 1];
                dest[x] += krow[1] * srow[x];
                dest[x] += krow[2] * srow[x + 1];
            }
            dest[w - 1] += krow[0] * srow[w - 2];
            dest[w - 1] += krow[1] * srow[w - 1];
        }
    }
}

/* cpu::conv3x3_shuffle2 (src/cpu.rs:502-542): output row y2 of channel ch is
 * conv rows co0 = 4ch + 2(y2%2) and co0+1 at y = y2/2, interleaved. */
void orc_conv3x3_shuffle2(const float *in, int cin, int h, int w, const float *wgt, int feat,
                          const float *bias, float *out) {
    int h2 = 2 * h, w2 = 2 * w;
    long nrows = (long)feat * h2;
#pragma omp parallel if ((long)feat * h2 * w2 >= PAR_MIN)
    {
        float *t0 = falloc(w), *t1 = falloc(w);
#pragma omp for schedule(dynamic, 8)
        for (long i = 0; i < nrows; ++i) {
            int ch = (int)(i / h2), y2 = (int)(i % h2);
            int dy = y2 % 2, y = y2 / 2;
            int co0 = 4 * ch + 2 * dy;
            conv_row(in, cin, h, w, wgt + (long)co0 * cin * 9, bias[co0], y, t0);
            int co1 = co0 + 1;
            conv_row(in, cin, h, w, wgt + (long)co1 * cin * 9, bias[co1], y, t1);
            float *dest = out + i * w2;
            for (int x = 0; x < w; ++x) {
                dest[2 * x] = t0[x];
                dest[2 * x + 1] = t1[x];
            }
        }
        free(t0);
        free(t1);
    }
}

/* cpu::conv1x1 -> lg::conv1x1 (src/cpu.rs:560-577): NCHW, out[co][p] =
 * b[co] + sum_ci w[co][ci] in[ci][p], bias folded first, ci ascending. */
void orc_conv1x1(const float *in, int cin, long hw, const float *wgt, int cout,
                 const float *bias, float *out) {
    const long PB = 256;
    long nblk = (hw + PB - 1) / PB;
    long tasks = nblk * ((cout + 3) / 4);
#pragma omp parallel for schedule(static) if (hw * cout >= PAR_MIN)
    for (long task = 0; task < tasks; ++task) {
        long pb = task % nblk;
        int co0 = (int)(task / nblk) * 4;
        long p0 = pb * PB, np = hw - p0 < PB ? hw - p0 : PB;
        int nco = cout - co0 < 4 ? cout - co0 : 4;
        float acc[4][256];
        for (int j = 0; j < nco; ++j)
            for (long i = 0; i < np; ++i) acc[j][i] = bias[co0 + j];
        for (int ci = 0; ci < cin; ++ci) {
            const float *s = in + (long)ci * hw + p0;
            for (int j = 0; j < nco; ++j) {
                float wv = wgt[(long)(co0 + j) * cin + ci];
                float *a = acc[j];
                for (long i = 0; i < np; ++i) a[i] += wv * s[i];
            }
        }
        for (int j = 0; j < nco; ++j)
            memcpy(out + (long)(co0 + j) * hw + p0, acc[j], (size_t)np * sizeof(float));
    }
}

/* cpu::linear -> matmul_rows -> matmul_tile! (src/cpu.rs:607-775):
 * out[r][co] = bias[co] + sum_ci w[co][ci] x[r][ci], bias first, ci ascending,
 * on a transposed operand xt[ci][rows] and a packed weight wp[ci][co], with an
 * 8-row x 10-channel register tile (the reference's AVX2 tile) and peeled
 * ragged edges in the same order. */
#define MR 8
#define NR 10
void orc_linear(const float *x, long rows, int cin, const float *wgt, int cout,
                const float *bias, float *out) {
    float *wp = falloc((long)cin * cout);
    for (int co = 0; co < cout; ++co)
        for (int ci = 0; ci < cin; ++ci) wp[(long)ci * cout + co] = wgt[(long)co * cin + ci];
    const long RB = 64; /* rows per task: transposed locally, MR-aligned */
    long nblk = (rows + RB - 1) / RB;
#pragma omp parallel if (rows * cout >= PAR_MIN)
    {
        float *xt = falloc((long)cin * RB);
#pragma omp for schedule(static)
        for (long b = 0; b < nblk; ++b) {
            long r0 = b * RB, nr = rows - r0 < RB ? rows - r0 : RB;
            for (int ci = 0; ci < cin; ++ci)
                for (long i = 0; i < nr; ++i) xt[ci * RB + i] = x[(r0 + i) * cin + ci];
            long rb = 0;
            for (; rb + MR <= nr; rb += MR) {
                int co0 = 0;
#ifdef __AVX2__
                /* The same tile with the accumulators pinned in ten YMM
                 * registers: per ci, one load of 8 rows, then per channel a
                 * broadcast, a multiply and an add (separately rounded, no
                 * FMA), exactly the scalar tile's arithmetic. */
                for (; co0 + NR <= cout; co0 += NR) {
                    __m256 a[NR];
                    for (int j = 0; j < NR; ++j) a[j] = _mm256_set1_ps(bias[co0 + j]);
                    for (int ci = 0; ci < cin; ++ci) {
                        const __m256 xv = _mm256_loadu_ps(xt + ci * RB + rb);
                        const float *wv = wp + (long)ci * cout + co0;
                        for (int j = 0; j < NR; ++j)
                            a[j] = _mm256_add_ps(a[j], _mm256_mul_ps(_mm256_set1_ps(wv[j]), xv));
                    }
                    for (int j = 0; j < NR; ++j) {
                        float tmp[MR];
                        _mm256_storeu_ps(tmp, a[j]);
                        for (int i = 0; i < MR; ++i) out[(r0 + rb + i) * cout + co0 + j] = tmp[i];
                    }
                }
#endif
                for (; co0 + NR <= cout; co0 += NR) {
                    float acc[NR][MR];
                    for (int j = 0; j < NR; ++j)
                        for (int i = 0; i < MR; ++i) acc[j][i] = bias[co0 + j];
                    for (int ci = 0; ci < cin; ++ci) {
                        const float *xv = xt + ci * RB + rb;
                        const float *wv = wp + (long)ci * cout + co0;
                        for (int j = 0; j < NR; ++j) {
                            float wj = wv[j];
                            for (int i = 0; i < MR; ++i) acc[j][i] += wj * xv[i];
                        }
                    }
                    for (int j = 0; j < NR; ++j)
                        for (int i = 0; i < MR; ++i)
                            out[(r0 + rb + i) * cout + co0 + j] = acc[j][i];
                }
                for (int j = co0; j < cout; ++j)
                    for (int i = 0; i < MR; ++i) {
                        float a = bias[j];
                        for (int ci = 0; ci < cin; ++ci)
                            a += wp[(long)ci * cout + j] * xt[ci * RB + rb + i];
                        out[(r0 + rb + i) * cout + j] = a;
                    }
            }
            for (long i = rb; i < nr; ++i)
                for (int j = 0; j < cout; ++j) {
                    float a = bias[j];
                    for (int ci = 0; ci < cin; ++ci) a += wp[(long)ci * cout + j] * xt[ci * RB + i];
                    out[(r0 + i) * cout + j] = a;
                }
        }
        free(xt);
    }
    free(wp);
}

/* ------------------------------------------------------------------------- */
/* Resampling: reference src/cpu.rs:795-966                                 */
/* ------------------------------------------------------------------------- */

/* src/cpu.rs:795-821: [4C][H][W] -> [C][2H][2W] */
void orc_pixel_shuffle2(const float *in, int c4, int h, int w, float *out) {
    int c = c4 / 4, oh = 2 * h, ow = 2 * w;
    for (long r = 0; r < (long)c * oh; ++r) {
        int ch = (int)(r / oh), rem = (int)(r % oh);
        int dy = rem & 1, y = rem >> 1;
        const float *s0 = in + (((long)ch * 4 + dy * 2) * h + y) * w;
        const float *s1 = in + (((long)ch * 4 + dy * 2 + 1) * h + y) * w;
        float *dst = out + r * ow;
        for (int x = 0; x < w; ++x) {
            dst[2 * x] = s0[x];
            dst[2 * x + 1] = s1[x];
        }
    }
}

/* src/cpu.rs:824-847: [C*s^2][H][W] -> [C][H*s][W*s] */
void orc_pixel_shuffle(const float *in, int c, int h, int w, int scale, float *out) {
    int oh = h * scale, ow = w * scale;
    for (long r = 0; r < (long)c * oh; ++r) {
        int ch = (int)(r / oh), rem = (int)(r % oh);
        int dy = rem % scale, y = rem / scale;
        float *dst = out + r * ow;
        for (int dx = 0; dx < scale; ++dx) {
            const float *src = in + (((long)ch * scale * scale + dy * scale + dx) * h + y) * w;
            for (int x = 0; x < w; ++x) dst[x * scale + dx] = src[x];
        }
    }
}

/* src/cpu.rs:875-935: torch's bicubic (a = -0.75, align_corners=False, edge clamp). */
static float cubic_w(float t) {
    const float A = -0.75f;
    t = fabsf(t);
    if (t <= 1.0f) return ((A + 2.0f) * t - (A + 3.0f)) * t * t + 1.0f;
    if (t < 2.0f) return (((t - 5.0f) * t + 8.0f) * t - 4.0f) * A;
    return 0.0f;
}

typedef struct { int idx[4]; float wt[4]; } tap4;

static tap4 *bicubic_taps(int n_in, int n_out) {
    tap4 *t = (tap4 *)xalloc(sizeof(tap4) * (size_t)n_out);
    for (int i = 0; i < n_out; ++i) {
        float src = ((float)i + 0.5f) * ((float)n_in / (float)n_out) - 0.5f;
        float base = floorf(src);
        for (int m = 0; m < 4; ++m) {
            int idx = (int)base - 1 + m;
            if (idx < 0) idx = 0;
            if (idx > n_in - 1) idx = n_in - 1;
            t[i].idx[m] = idx;
            t[i].wt[m] = cubic_w(src - (base + (float)m - 1.0f));
        }
    }
    return t;
}

void orc_bicubic_resize(const float *in, int c, int h, int w, int oh, int ow, float *out) {
    tap4 *ty = bicubic_taps(h, oh), *tx = bicubic_taps(w, ow);
#pragma omp parallel for schedule(static) if ((long)c * oh * ow >= PAR_MIN)
    for (long i = 0; i < (long)c * oh; ++i) {
        int ch = (int)(i / oh), y = (int)(i % oh);
        const float *src = in + (long)ch * h * w;
        float *dst = out + i * ow;
        for (int x = 0; x < ow; ++x) {
            float acc = 0.0f;
            for (int m = 0; m < 4; ++m) {
                const float *r = src + (long)ty[y].idx[m] * w;
                float a0 = tx[x].wt[0] * r[tx[x].idx[0]];
                float a1 = tx[x].wt[1] * r[tx[x].idx[1]];
                float a2 = tx[x].wt[2] * r[tx[x].idx[2]];
                float a3 = tx[x].wt[3] * r[tx[x].idx[3]];
                acc += ty[y].wt[m] * ((a0 + a1) + (a2 + a3));
            }
            dst[x] = acc;
        }
    }
    free(ty);
    free(tx);
}

/* src/cpu.rs:938-966 */
void orc_upsample2x_nearest(const float *in, int c, int h, int w, float *out) {
    int oh = 2 * h, ow = 2 * w;
    (void)oh;
    for (long i = 0; i < (long)c * h; ++i) {
        const float *src = in + i * w;
        float *a = out + i * 2 * ow, *b = a + ow;
        for (int x = 0; x < w; ++x) {
            float v = src[x];
            a[2 * x] = v;
            a[2 * x + 1] = v;
            b[2 * x] = v;
            b[2 * x + 1] = v;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Elementwise and normalisation: reference src/cpu.rs:970-1132             */
/* ------------------------------------------------------------------------- */

/* src/cpu.rs:970-983 */
void orc_leaky_relu(float *x, long n, float slope) {
#pragma omp parallel for schedule(static) if (n >= PAR_MIN)
    for (long i = 0; i < n; ++i)
        if (x[i] < 0.0f) x[i] *= slope;
}

/* src/cpu.rs:993-1002: y += a */
void orc_add_into(const float *a, float *y, long n) {
#pragma omp parallel for schedule(static) if (n >= PAR_MIN)
    for (long i = 0; i < n; ++i) y[i] += a[i];
}

/* src/cpu.rs:1019-1073: per position, s1 and s2 summed over ascending
 * channels, mean = s1/c, var = max(s2/c - mean^2, 0), then
 * y = (x - mean) * rstd * w + b with rstd = 1/sqrt(var + eps). */
void orc_channel_layer_norm(const float *x, const float *w, const float *b, float *y, int c,
                            long hw, float eps) {
    const long BLK = 64;
    long nblk = (hw + BLK - 1) / BLK;
#pragma omp parallel for schedule(static) if (hw >= PAR_MIN)
    for (long bi = 0; bi < nblk; ++bi) {
        long p0 = bi * BLK, np = hw - p0 < BLK ? hw - p0 : BLK;
        float s1[64], s2[64], mean[64], rstd[64];
        for (long j = 0; j < np; ++j) s1[j] = s2[j] = 0.0f;
        for (int ch = 0; ch < c; ++ch) {
            const float *pl = x + (long)ch * hw + p0;
            for (long j = 0; j < np; ++j) {
                float v = pl[j];
                s1[j] += v;
                s2[j] += v * v;
            }
        }
        float n = (float)c;
        for (long j = 0; j < np; ++j) {
            float m = s1[j] / n;
            float var = s2[j] / n - m * m;
            mean[j] = m;
            rstd[j] = 1.0f / sqrtf((var > 0.0f ? var : 0.0f) + eps);
        }
        for (int ch = 0; ch < c; ++ch) {
            const float *pl = x + (long)ch * hw + p0;
            float *dst = y + (long)ch * hw + p0;
            float wv = w[ch], bv = b[ch];
            for (long j = 0; j < np; ++j) dst[j] = (pl[j] - mean[j]) * rstd[j] * wv + bv;
        }
    }
}

/* src/cpu.rs:1095-1120, statement for statement. NOTE what it computes: with
 * n = floor(t + 0.5) - 0.5 a half-integer, `f = t - n` lies in [0, 1) and the
 * integer scale is trunc(n), which is floor(t+0.5) for every t < 0.5 - so the
 * result is 2^(t + 0.5) = sqrt(2) * e^x to the series' accuracy (<= 1.6e-5
 * relative at f -> 1), not e^x. The softmax only ever feeds it x <= 0 and
 * normalises, so the constant sqrt(2) cancels; tests pin both facts. */
float orc_fast_exp(float x) {
    const float LOG2_E = 1.4426950408889634f;
    float t = x * LOG2_E;
    float n = floorf(t + 0.5f) - 0.5f;
    if (n < -126.0f) return 0.0f;
    float f = t - n;
    float p = 1.0f +
              f * (0.69314718f +
                   f * (0.24022651f +
                        f * (0.05550411f +
                             f * (0.009618129f + f * (0.0013333558f + f * 0.0001540353f)))));
    uint32_t bits = ((uint32_t)((int32_t)n + 127)) << 23;
    float scale;
    memcpy(&scale, &bits, 4);
    return scale * p;
}

/* src/cpu.rs:1125-1132: 0.5 x (1 + erf(x / sqrt 2)). The toolkit's `lg::erf`
 * is not in the reference tree; libm's erff stands in (ulp-level). */
void orc_gelu_erf_inplace(float *x, long n) {
#pragma omp parallel for schedule(static) if (n >= PAR_MIN)
    for (long i = 0; i < n; ++i) {
        float v = x[i];
        x[i] = 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
    }
}

/* ------------------------------------------------------------------------- */
/* The window pair and attention: reference src/cpu.rs:1148-1402            */
/* ------------------------------------------------------------------------- */

/* src/cpu.rs:1148-1197 (norm = None, the only mode the graph uses). */
void orc_gather(const orc_plan *p, const float *x, int shift, float *tok) {
    int c = p->c;
    long hw = (long)p->hp * p->wp;
#pragma omp parallel for schedule(static) if ((long)p->nw * p->n * c >= PAR_MIN)
    for (int wi = 0; wi < p->nw; ++wi)
        for (int t = 0; t < p->n; ++t) {
            int y, xx;
            orc_index(p, wi, t, shift, &y, &xx);
            long pos = (long)y * p->wp + xx;
            float *dst = tok + ((long)wi * p->n + t) * c;
            for (int i = 0; i < c; ++i) dst[i] = x[(long)i * hw + pos];
        }
}

/* src/cpu.rs:1200-1222 */
void orc_scatter(const orc_plan *p, const float *tok, int shift, float *x) {
    int c = p->c;
    long hw = (long)p->hp * p->wp;
#pragma omp parallel for schedule(static) if ((long)p->nw * p->n * c >= PAR_MIN)
    for (int i = 0; i < c; ++i) {
        float *dst = x + (long)i * hw;
        for (int wi = 0; wi < p->nw; ++wi)
            for (int t = 0; t < p->n; ++t) {
                int y, xx;
                orc_index(p, wi, t, shift, &y, &xx);
                dst[(long)y * p->wp + xx] = tok[((long)wi * p->n + t) * c + i];
            }
    }
}

/* src/cpu.rs:1244-1402: cosine attention, cpb bias, -100 shift mask,
 * max-subtracted softmax with fast_exp, AV with four accumulators (d outer). */
void orc_attention(const orc_plan *p, int heads, int head_dim, const float *logit_scale,
                   const float *cpb, const float *qkv, int shift, float *out) {
    int c = p->c, n = p->n;
    long tok_c = (long)p->nw * n * c;
    int masked = shift != 0;
    float ls[64];
    for (int hd = 0; hd < heads; ++hd) {
        float v = logit_scale[hd];
        float cap = logf(100.0f);
        ls[hd] = expf(v < cap ? v : cap);
    }
    float *cpbt = falloc((long)heads * n * n);
    for (int q = 0; q < n; ++q)
        for (int k = 0; k < n; ++k)
            for (int hd = 0; hd < heads; ++hd)
                cpbt[((long)hd * n + q) * n + k] = cpb[((long)q * n + k) * heads + hd];
#pragma omp parallel if ((long)p->nw * n * c >= PAR_MIN)
    {
        float *scores = falloc(n), *kn = falloc(n);
        long *ktok = (long *)xalloc(sizeof(long) * (size_t)n);
        uint8_t *kry = (uint8_t *)xalloc((size_t)n), *krx = (uint8_t *)xalloc((size_t)n);
#pragma omp for schedule(static)
        for (int wi = 0; wi < p->nw; ++wi) {
            float *outw = out + (long)wi * n * c;
            for (int k = 0; k < n; ++k) {
                ktok[k] = (long)wi * n + k;
                if (masked) orc_region(p, wi, k, shift, &kry[k], &krx[k]);
            }
            for (int hd = 0; hd < heads; ++hd) {
                int off = hd * head_dim;
                for (int k = 0; k < n; ++k) {
                    long kbase = tok_c + ktok[k] * c + off;
                    float s = 0.0f;
                    for (int d = 0; d < head_dim; ++d) {
                        float v = qkv[kbase + d];
                        s += v * v;
                    }
                    float r = sqrtf(s);
                    kn[k] = r > 1e-12f ? r : 1e-12f;
                }
                for (int q = 0; q < n; ++q) {
                    uint8_t rqy = masked ? kry[q] : 0, rqx = masked ? krx[q] : 0;
                    float *orow = outw + (long)q * c;
                    const float *qv = qkv + ktok[q] * c + off;
                    float qs = 0.0f;
                    for (int d = 0; d < head_dim; ++d) qs += qv[d] * qv[d];
                    float qn = sqrtf(qs);
                    qn = qn > 1e-12f ? qn : 1e-12f;
                    for (int k = 0; k < n; ++k) {
                        const float *kv = qkv + tok_c + ktok[k] * c + off;
                        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
                        int d = 0;
                        for (; d + 4 <= head_dim; d += 4) {
                            a0 += qv[d] * kv[d];
                            a1 += qv[d + 1] * kv[d + 1];
                            a2 += qv[d + 2] * kv[d + 2];
                            a3 += qv[d + 3] * kv[d + 3];
                        }
                        float tail = 0.0f;
                        for (; d < head_dim; ++d) tail += qv[d] * kv[d];
                        float dot = ((a0 + a1) + (a2 + a3) + tail) / (qn * kn[k]);
                        float s = dot * ls[hd] + cpbt[((long)hd * n + q) * n + k];
                        if (masked && (rqy != kry[k] || rqx != krx[k])) s -= 100.0f;
                        scores[k] = s;
                    }
                    float mx = -INFINITY;
                    for (int k = 0; k < n; ++k) mx = fmaxf(mx, scores[k]);
                    float sum = 0.0f;
                    for (int k = 0; k < n; ++k) {
                        scores[k] = orc_fast_exp(scores[k] - mx);
                        sum += scores[k];
                    }
                    float inv = 1.0f / sum;
                    const float *V = qkv + 2 * tok_c;
                    for (int d = 0; d < head_dim; ++d) {
                        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
                        int k = 0;
                        for (; k + 4 <= n; k += 4) {
                            a0 += scores[k] * V[ktok[k] * c + off + d];
                            a1 += scores[k + 1] * V[ktok[k + 1] * c + off + d];
                            a2 += scores[k + 2] * V[ktok[k + 2] * c + off + d];
                            a3 += scores[k + 3] * V[ktok[k + 3] * c + off + d];
                        }
                        float tail = 0.0f;
                        for (; k < n; ++k) tail += scores[k] * V[ktok[k] * c + off + d];
                        orow[off + d] = ((a0 + a1) + (a2 + a3) + tail) * inv;
                    }
                }
            }
        }
        free(scores);
        free(kn);
        free(ktok);
        free(kry);
        free(krx);
    }
    free(cpbt);
}

/* tools/convert.py:141-167 with network_swin2sr.py:101-136: the log-spaced
 * coordinate table t = sign(v) log2(|v|+1)/log2(8), v = 8 d/(win-1), through
 * Linear(2,512)+ReLU+Linear(512,heads), gathered by the relative position
 * index and mapped by 16 sigmoid. out is [n*n][heads] (the checkpoint's
 * cpb_pre layout). f32 arithmetic in numpy's order (matmul sums ascending). */
void orc_cpb_table(int win, int heads, const float *w0, const float *b0, const float *w2,
                   float *out) {
    int side = 2 * win - 1, nt = side * side, n = win * win;
    float *tab = falloc((long)nt * heads);
    float *hid = falloc(512);
    for (int a = 0; a < side; ++a)
        for (int b = 0; b < side; ++b) {
            float co[2] = {(float)(a - (win - 1)), (float)(b - (win - 1))};
            for (int k = 0; k < 2; ++k) {
                float v = co[k] / (float)(win - 1);
                v = v * 8.0f;
                float s = (v > 0.0f) ? 1.0f : (v < 0.0f ? -1.0f : 0.0f);
                co[k] = s * log2f(fabsf(v) + 1.0f) / (float)log2(8.0);
            }
            for (int j = 0; j < 512; ++j) {
                float hv = co[0] * w0[j * 2 + 0] + co[1] * w0[j * 2 + 1] + b0[j];
                hid[j] = hv > 0.0f ? hv : 0.0f;
            }
            for (int h = 0; h < heads; ++h) {
                float acc = 0.0f;
                for (int j = 0; j < 512; ++j) acc += hid[j] * w2[(long)h * 512 + j];
                tab[(long)(a * side + b) * heads + h] = acc;
            }
        }
    for (int q = 0; q < n; ++q)
        for (int k = 0; k < n; ++k) {
            int yq = q / win, xq = q % win, yk = k / win, xk = k % win;
            int idx = (yq - yk + win - 1) * side + (xq - xk + win - 1);
            for (int h = 0; h < heads; ++h) {
                float v = tab[(long)idx * heads + h];
                out[((long)q * n + k) * heads + h] = 16.0f / (1.0f + expf(-v));
            }
        }
    free(tab);
    free(hid);
}

/* ------------------------------------------------------------------------- */
/* Epilogues: reference src/cpu.rs:1890-1941, src/image.rs:29-39            */
/* ------------------------------------------------------------------------- */

void orc_finish(const s2s_arch *a, const orc_plan *p, const float *planes, int src_w,
                float *out) {
    int s = a->scale, h = p->h * s, w = p->w * s;
    int ow = src_w, oh = p->hp * s;
    for (int ci = 0; ci < 3; ++ci)
        for (int y = 0; y < h; ++y)
            for (int x = 0; x < w; ++x)
                out[((long)ci * h + y) * w + x] =
                    planes[((long)ci * oh + y) * ow + x] / a->img_range + a->mean[ci];
}

void orc_finish_aux(const s2s_arch *a, const orc_plan *p, const float *aux, float *out) {
    long hw = (long)p->hp * p->wp;
    for (int ci = 0; ci < 3; ++ci)
        for (long i = 0; i < hw; ++i)
            out[ci * hw + i] = aux[ci * hw + i] / a->img_range + a->mean[ci];
}

/* src/image.rs:29-39: floor(clamp01(v) * 255 + 0.5) */
void orc_to_rgb8(const float *x, long n, uint8_t *out) {
    for (long i = 0; i < n; ++i) {
        float v = x[i];
        v = v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
        out[i] = (uint8_t)floorf(v * 255.0f + 0.5f);
    }
}

/* ------------------------------------------------------------------------- */
/* The graph: reference src/cpu.rs:1437-1880                                */
/* ------------------------------------------------------------------------- */

static const float *tget(const s2s_tensor *t, size_t nt, const char *name) {
    for (size_t i = 0; i < nt; ++i)
        if (strcmp(t[i].name, name) == 0) return t[i].data;
    snprintf(g_err, sizeof g_err, "weight `%s` is missing", name);
    return NULL;
}

#define NEED(var, ...)                                                     \
    const float *var;                                                      \
    do {                                                                   \
        char nm_[160];                                                     \
        snprintf(nm_, sizeof nm_, __VA_ARGS__);                            \
        var = tget(t, nt, nm_);                                            \
        if (!var) goto fail;                                               \
    } while (0)

typedef struct {
    float *tok, *tok2, *attn, *qkv, *mlp, *acc, *res, *zero_bias;
} blk_scratch;

/* One post-norm Swin V2 block (src/cpu.rs:1516-1575), in place on `cur`
 * (which is also `res` after the block). */
static int run_block(const s2s_arch *a, const s2s_tensor *t, size_t nt, const orc_plan *p,
                     int s, int b, float *cur, blk_scratch *sc) {
    int c = p->c;
    long tokens = (long)p->nw * p->n, tok = tokens * c, hw = (long)p->hp * p->wp;
    int hidden = a->mlp_ratio * c;
    int shift = orc_shift_for(p, b);
    const char *pf = "layers.%d.residual_group.blocks.%d.";
    NEED(wq, "layers.%d.residual_group.blocks.%d.attn.qkv.wq", s, b);
    NEED(wk, "layers.%d.residual_group.blocks.%d.attn.qkv.wk", s, b);
    NEED(wv, "layers.%d.residual_group.blocks.%d.attn.qkv.wv", s, b);
    NEED(qb, "layers.%d.residual_group.blocks.%d.attn.qkv.q_bias", s, b);
    NEED(vb, "layers.%d.residual_group.blocks.%d.attn.qkv.v_bias", s, b);
    NEED(ls, "layers.%d.residual_group.blocks.%d.attn.logit_scale", s, b);
    NEED(cpb, "layers.%d.residual_group.blocks.%d.attn.cpb_pre", s, b);
    NEED(pw, "layers.%d.residual_group.blocks.%d.attn.proj.weight", s, b);
    NEED(pb, "layers.%d.residual_group.blocks.%d.attn.proj.bias", s, b);
    NEED(n1w, "layers.%d.residual_group.blocks.%d.norm1.weight", s, b);
    NEED(n1b, "layers.%d.residual_group.blocks.%d.norm1.bias", s, b);
    NEED(n2w, "layers.%d.residual_group.blocks.%d.norm2.weight", s, b);
    NEED(n2b, "layers.%d.residual_group.blocks.%d.norm2.bias", s, b);
    NEED(f1w, "layers.%d.residual_group.blocks.%d.mlp.fc1.weight", s, b);
    NEED(f1b, "layers.%d.residual_group.blocks.%d.mlp.fc1.bias", s, b);
    NEED(f2w, "layers.%d.residual_group.blocks.%d.mlp.fc2.weight", s, b);
    NEED(f2b, "layers.%d.residual_group.blocks.%d.mlp.fc2.bias", s, b);
    (void)pf;
    /* res == cur on entry (the reference copies res into cur after every block
     * and starts each stage with res = cur). */
    orc_gather(p, cur, shift, sc->tok);
    orc_linear(sc->tok, tokens, c, wq, c, qb, sc->qkv);
    orc_linear(sc->tok, tokens, c, wk, c, sc->zero_bias, sc->qkv + tok);
    orc_linear(sc->tok, tokens, c, wv, c, vb, sc->qkv + 2 * tok);
    orc_attention(p, a->heads, c / a->heads, ls, cpb, sc->qkv, shift, sc->attn);
    orc_linear(sc->attn, tokens, c, pw, c, pb, sc->tok2);
    orc_scatter(p, sc->tok2, shift, sc->acc);
    orc_channel_layer_norm(sc->acc, n1w, n1b, sc->tok2, c, hw, LN_EPS);
    orc_add_into(sc->tok2, cur, hw * c);
    orc_gather(p, cur, shift, sc->tok);
    orc_linear(sc->tok, tokens, c, f1w, hidden, f1b, sc->mlp);
    orc_gelu_erf_inplace(sc->mlp, tokens * hidden);
    orc_linear(sc->mlp, tokens, hidden, f2w, c, f2b, sc->attn);
    orc_scatter(p, sc->attn, shift, sc->acc);
    orc_channel_layer_norm(sc->acc, n2w, n2b, sc->tok2, c, hw, LN_EPS);
    orc_add_into(sc->tok2, cur, hw * c);
    return 0;
fail:
    return -1;
}

static void scratch_new(const s2s_arch *a, const orc_plan *p, blk_scratch *sc) {
    long tok = (long)p->nw * p->n * p->c, plane = (long)p->hp * p->wp * p->c;
    sc->tok = falloc(tok);
    sc->tok2 = falloc(tok > plane ? tok : plane);
    sc->attn = falloc(tok);
    sc->qkv = falloc(3 * tok);
    sc->mlp = falloc(tok * a->mlp_ratio);
    sc->acc = falloc(plane);
    sc->res = NULL;
    sc->zero_bias = fzeros(p->c);
}

static void scratch_free(blk_scratch *sc) {
    free(sc->tok);
    free(sc->tok2);
    free(sc->attn);
    free(sc->qkv);
    free(sc->mlp);
    free(sc->acc);
    free(sc->zero_bias);
}

/* The RSTB stage (src/cpu.rs:1505-1583): blocks in place, then conv3x3 ->
 * conv1x1 -> + stage input. */
static int run_stage(const s2s_arch *a, const s2s_tensor *t, size_t nt, const orc_plan *p,
                     int s, float *cur, blk_scratch *sc) {
    int c = p->c;
    long hw = (long)p->hp * p->wp;
    float *stage = falloc(hw * c);
    memcpy(stage, cur, sizeof(float) * (size_t)(hw * c));
    for (int b = 0; b < a->depths[s]; ++b)
        if (run_block(a, t, nt, p, s, b, cur, sc) != 0) {
            free(stage);
            return -1;
        }
    NEED(cw, "layers.%d.conv.weight", s);
    NEED(cb, "layers.%d.conv.bias", s);
    NEED(pw, "layers.%d.patch_embed.proj.weight", s);
    NEED(pb, "layers.%d.patch_embed.proj.bias", s);
    orc_conv3x3(cur, c, p->hp, p->wp, cw, c, cb, sc->acc);
    orc_conv1x1(sc->acc, c, hw, pw, c, pb, cur);
    orc_add_into(stage, cur, hw * c);
    free(stage);
    return 0;
fail:
    free(stage);
    return -1;
}

int orc_rstb(const s2s_arch *a, const s2s_tensor *t, size_t nt, const orc_plan *p, int stage,
             float *x) {
    blk_scratch sc;
    scratch_new(a, p, &sc);
    int rc = run_stage(a, t, nt, p, stage, x, &sc);
    scratch_free(&sc);
    return rc;
}

static int log2i(int v) {
    int o = 0;
    while ((1 << o) < v) ++o;
    return o;
}

int orc_forward(const s2s_arch *a, const s2s_tensor *t, size_t nt, int h, int w,
                const float *in_adjusted, float *out, float *aux_out) {
    orc_plan P;
    orc_plan_new(h, w, a->window, a->embed, &P);
    const orc_plan *p = &P;
    int c = a->embed, s = a->scale;
    long hw = (long)p->hp * p->wp;
    float *padded = falloc(3 * hw);
    float *cur = falloc(hw * c), *body = falloc(hw * c), *nbuf = NULL;
    float *planes = NULL, *aux = NULL;
    float *bic = NULL;
    blk_scratch sc;
    int rc = -1;
    scratch_new(a, p, &sc);

    orc_pad_reflect(in_adjusted, 3, h, w, p->hp, p->wp, padded);
    {
        NEED(cfw, "conv_first.weight");
        NEED(cfb, "conv_first.bias");
        orc_conv3x3(padded, 3, p->hp, p->wp, cfw, c, cfb, cur);
    }
    memcpy(body, cur, sizeof(float) * (size_t)(hw * c));
    {
        NEED(pw, "patch_embed.proj.weight");
        NEED(pb, "patch_embed.proj.bias");
        NEED(nw_, "patch_embed.norm.weight");
        NEED(nb_, "patch_embed.norm.bias");
        orc_conv1x1(cur, c, hw, pw, c, pb, sc.acc);
        orc_channel_layer_norm(sc.acc, nw_, nb_, cur, c, hw, LN_EPS);
    }
    for (int st = 0; st < a->n_stages; ++st)
        if (run_stage(a, t, nt, p, st, cur, &sc) != 0) goto fail;
    nbuf = falloc(hw * c);
    {
        NEED(nw_, "norm.weight");
        NEED(nb_, "norm.bias");
        NEED(cw, "conv_after_body.weight");
        NEED(cb, "conv_after_body.bias");
        orc_channel_layer_norm(cur, nw_, nb_, nbuf, c, hw, LN_EPS);
        orc_conv3x3(nbuf, c, p->hp, p->wp, cw, c, cb, sc.acc);
        orc_add_into(body, sc.acc, hw * c);
        memcpy(cur, sc.acc, sizeof(float) * (size_t)(hw * c));
    }
    free(nbuf);
    nbuf = NULL;
    scratch_free(&sc);
    sc.tok = NULL;

    int oh = p->hp * s, ow = p->wp * s;
    if (a->upsampler == S2S_PIXELSHUFFLE || a->upsampler == S2S_PIXELSHUFFLE_AUX) {
        NEED(bw, "conv_before_upsample.0.weight");
        NEED(bb, "conv_before_upsample.0.bias");
        NEED(lw, "conv_last.weight");
        NEED(lb, "conv_last.bias");
        /* feat = len / (c * 9) */
        int feat = 0;
        for (size_t i = 0; i < nt; ++i)
            if (strcmp(t[i].name, "conv_before_upsample.0.weight") == 0) feat = (int)t[i].shape[0];
        int octaves = log2i(s);
        float *xa = falloc((long)feat * hw);
        orc_conv3x3(cur, c, p->hp, p->wp, bw, feat, bb, xa);
        orc_leaky_relu(xa, (long)feat * hw, 0.01f);
        if (a->upsampler == S2S_PIXELSHUFFLE_AUX) {
            NEED(bcw, "conv_bicubic.weight");
            NEED(bcb, "conv_bicubic.bias");
            NEED(aw, "conv_aux.weight");
            NEED(ab, "conv_aux.bias");
            NEED(caw, "conv_after_aux.0.weight");
            NEED(cab, "conv_after_aux.0.bias");
            float *resized = falloc(3L * oh * ow);
            orc_bicubic_resize(padded, 3, p->hp, p->wp, oh, ow, resized);
            bic = falloc((long)feat * oh * ow);
            orc_conv3x3(resized, 3, oh, ow, bcw, feat, bcb, bic);
            free(resized);
            aux = falloc(3 * hw);
            orc_conv3x3(xa, feat, p->hp, p->wp, aw, 3, ab, aux);
            float *xb = falloc((long)feat * hw);
            orc_conv3x3(aux, 3, p->hp, p->wp, caw, feat, cab, xb);
            orc_leaky_relu(xb, (long)feat * hw, 0.01f);
            free(xa);
            xa = xb;
        }
        int h2 = p->hp, w2 = p->wp;
        for (int o = 0; o < octaves; ++o) {
            NEED(uw, "upsample.%d.weight", 2 * o);
            NEED(ub, "upsample.%d.bias", 2 * o);
            float *shuf = falloc((long)feat * 4 * h2 * w2);
            orc_conv3x3_shuffle2(xa, feat, h2, w2, uw, feat, ub, shuf);
            free(xa);
            xa = shuf;
            h2 *= 2;
            w2 *= 2;
        }
        if (bic) {
            orc_add_into(bic, xa, (long)feat * h2 * w2);
        }
        planes = falloc(3L * h2 * w2);
        orc_conv3x3(xa, feat, h2, w2, lw, 3, lb, planes);
        free(xa);
    } else if (a->upsampler == S2S_PIXELSHUFFLE_DIRECT) {
        NEED(uw, "upsample.0.weight");
        NEED(ub, "upsample.0.bias");
        int och = 3 * s * s;
        float *up = falloc((long)och * hw);
        orc_conv3x3(cur, c, p->hp, p->wp, uw, och, ub, up);
        planes = falloc(3L * oh * ow);
        orc_pixel_shuffle(up, 3, p->hp, p->wp, s, planes);
        free(up);
    } else if (a->upsampler == S2S_NEAREST_CONV) {
        NEED(bw, "conv_before_upsample.0.weight");
        NEED(bb, "conv_before_upsample.0.bias");
        NEED(u1w, "conv_up1.weight");
        NEED(u1b, "conv_up1.bias");
        NEED(u2w, "conv_up2.weight");
        NEED(u2b, "conv_up2.bias");
        NEED(hrw, "conv_hr.weight");
        NEED(hrb, "conv_hr.bias");
        NEED(lw, "conv_last.weight");
        NEED(lb, "conv_last.bias");
        int feat = 0;
        for (size_t i = 0; i < nt; ++i)
            if (strcmp(t[i].name, "conv_before_upsample.0.weight") == 0) feat = (int)t[i].shape[0];
        int h2 = p->hp, w2 = p->wp;
        float *xa = falloc((long)feat * hw);
        orc_conv3x3(cur, c, h2, w2, bw, feat, bb, xa);
        orc_leaky_relu(xa, (long)feat * hw, 0.01f);
        for (int step = 0; step < 2; ++step) {
            float *up = falloc((long)feat * 4 * h2 * w2);
            orc_upsample2x_nearest(xa, feat, h2, w2, up);
            free(xa);
            h2 *= 2;
            w2 *= 2;
            xa = falloc((long)feat * h2 * w2);
            orc_conv3x3(up, feat, h2, w2, step == 0 ? u1w : u2w, feat, step == 0 ? u1b : u2b, xa);
            orc_leaky_relu(xa, (long)feat * h2 * w2, 0.2f);
            free(up);
        }
        float *hr = falloc((long)feat * h2 * w2);
        orc_conv3x3(xa, feat, h2, w2, hrw, feat, hrb, hr);
        orc_leaky_relu(hr, (long)feat * h2 * w2, 0.2f);
        free(xa);
        planes = falloc(3L * h2 * w2);
        orc_conv3x3(hr, feat, h2, w2, lw, 3, lb, planes);
        free(hr);
    } else {
        snprintf(g_err, sizeof g_err, "unknown upsampler %d", a->upsampler);
        goto fail;
    }
    orc_finish(a, p, planes, ow, out);
    if (aux && aux_out) orc_finish_aux(a, p, aux, aux_out);
    rc = 0;
fail:
    if (sc.tok) scratch_free(&sc);
    free(padded);
    free(cur);
    free(body);
    free(nbuf);
    free(planes);
    free(aux);
    free(bic);
    return rc;
}
