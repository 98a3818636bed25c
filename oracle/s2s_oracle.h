/* s2s_oracle.h - CPU restatement of the swin2sr crate's CPU path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker or
 * as the timed CPU baseline. The HIP backend never calls it.
 *
 * Every function follows one function of the reference (paths relative to the
 * reference repository) in its operation order and its f32 summation order, so
 * that the oracle computes what `src/cpu.rs` computes, not merely the same
 * mathematics. Layouts are the reference's: image planes NCHW `[c][h][w]`,
 * window tokens `[nw*n][c]` window-major.
 *
 * Pinning (how each function is checked independently of its own formula) is
 * listed per function in the header comment of s2s_oracle.c.
 */
#ifndef S2S_ORACLE_H
#define S2S_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/swin2sr_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference src/plan.rs:20-36 */
typedef struct orc_plan {
    int h, w, hp, wp, win, nwh, nww, nw, n, c;
} orc_plan;

void orc_plan_new(int h, int w, int win, int c, orc_plan *p);
/* An explicit, unpadded plane (the config-1 micro-bench builds Plan{hp,wp}
 * directly rather than through Plan::new). */
void orc_plan_explicit(int hp, int wp, int win, int c, orc_plan *p);
int orc_shift_for(const orc_plan *p, int b);
void orc_index(const orc_plan *p, int wi, int t, int shift, int *y, int *x);
int orc_region_of(int a, int len, int win, int shift);
void orc_region(const orc_plan *p, int wi, int t, int shift, uint8_t *ry, uint8_t *rx);
void orc_window_map(const orc_plan *p, int shift, int32_t *yx, uint8_t *reg);
void orc_pad_reflect(const float *x, int c, int h, int w, int hp, int wp, float *out);

void orc_conv3x3(const float *in, int cin, int h, int w, const float *wgt, int cout,
                 const float *bias, float *out);
void orc_conv3x3_shuffle2(const float *in, int cin, int h, int w, const float *wgt, int feat,
                          const float *bias, float *out);
void orc_conv1x1(const float *in, int cin, long hw, const float *wgt, int cout,
                 const float *bias, float *out);
void orc_linear(const float *x, long rows, int cin, const float *wgt, int cout,
                const float *bias, float *out);
void orc_pixel_shuffle2(const float *in, int c4, int h, int w, float *out);
void orc_pixel_shuffle(const float *in, int c, int h, int w, int scale, float *out);
void orc_bicubic_resize(const float *in, int c, int h, int w, int oh, int ow, float *out);
void orc_upsample2x_nearest(const float *in, int c, int h, int w, float *out);
void orc_leaky_relu(float *x, long n, float slope);
void orc_add_into(const float *a, float *y, long n);
void orc_channel_layer_norm(const float *x, const float *w, const float *b, float *y, int c,
                            long hw, float eps);
float orc_fast_exp(float x);
void orc_gelu_erf_inplace(float *x, long n);
void orc_gather(const orc_plan *p, const float *x, int shift, float *tok);
void orc_scatter(const orc_plan *p, const float *tok, int shift, float *x);
void orc_attention(const orc_plan *p, int heads, int head_dim, const float *logit_scale,
                   const float *cpb, const float *qkv, int shift, float *out);
void orc_cpb_table(int win, int heads, const float *w0, const float *b0, const float *w2,
                   float *out);
void orc_finish(const s2s_arch *a, const orc_plan *p, const float *planes, int src_w,
                float *out);
void orc_finish_aux(const s2s_arch *a, const orc_plan *p, const float *aux, float *out);
void orc_to_rgb8(const float *x, long n, uint8_t *out);

/* One RSTB stage (blocks + conv3x3 + conv1x1 + residual) on an NCHW plane of
 * `p`, in place on `x`. Returns 0 or -1 (missing tensor; see orc_last_error). */
int orc_rstb(const s2s_arch *a, const s2s_tensor *t, size_t nt, const orc_plan *p, int stage,
             float *x);

/* The whole-image forward, reference cpu::forward (src/cpu.rs:1437-1685) + head
 * + finish. `in_adjusted` [3][h][w]; `out` [3][h*s][w*s]; `aux` (may be NULL)
 * receives [3][hp][wp] for the compressed head. Returns 0 or -1. */
int orc_forward(const s2s_arch *a, const s2s_tensor *t, size_t nt, int h, int w,
                const float *in_adjusted, float *out, float *aux);

const char *orc_last_error(void);
int orc_threads(void);
void orc_set_threads(int n);

#ifdef __cplusplus
}
#endif

#endif
