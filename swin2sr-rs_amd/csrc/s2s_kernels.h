// s2s_kernels.h - argument blocks and launchers of the gfx950 kernels
// (s2s_kernels.hip). Host code in s2s_api.cpp plans buffers and calls these.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

enum {
    ALOAD_ROWS = 0,       // A[m*lda + k]
    ALOAD_IM2COL = 1,     // 3x3 im2col of the channel-last H x W plane A[H*W][cin]
    ALOAD_IM2COL5 = 3,    // 5x5 im2col of the channel-last H x W plane (k = tap*cin + ci)
    ALOAD_SUB2 = 4        // a 3x3 conv of the nearest-2x upsampling of the H x W plane A,
                          // as four 2x2 convs of A, one per output phase (a, b): row m =
                          // (y, x) of A, k = tap*cin + ci with tap (i, j) reading A at
                          // (y + a - 1 + i, x + b - 1 + j); B = [4 phases][N][ldb]; the
                          // epilogue stores output pixel (2y + a, 2x + b) of the 2H x 2W
                          // plane. One launch covers the four phases.
};
enum {
    EPI_STORE = 0,   // out = acc + bias
    EPI_GELU = 1,    // out = gelu_erf(acc + bias)
    EPI_RES = 2,     // out = acc + bias + res
    EPI_LN = 3,      // out = LayerNorm(acc + bias)             (N <= 192)
    EPI_LN_RES = 4,  // out = res + LayerNorm(acc + bias)       (N <= 192)
    EPI_LRELU = 5,   // out = leaky_relu(acc + bias, slope)
    EPI_SHUFFLE = 6,  // pixel_shuffle(2) store into a 2H x 2W channel-last plane (+ res
                      // in that layout when res is set)
    EPI_SHUFFLE_FINISH = 7,  // pixel_shuffle(scale) of a 3*scale^2-channel conv, denormalised
                             // and cropped into the planar [3][oh][ow] output
    EPI_QKV_WIN = 8  // out = acc + bias, A rows read window by window in the shifted-window
                     // order and stored in the attention unit layout (attn_unit_stride)
};

// The window-attention unit layout of qkv (written by the qkv GEMM under
// EPI_QKV_WIN, read by the window attention): one unit per (window, head
// pair) of the shifted plane, units in (window, pair) order, each 64 token
// rows of attn_unit_stride(hd) floats - the pair's q columns (2*hd), then its
// k and v columns, then 2 padding floats. Token t of window (wh, ww) is plane
// pixel ((8wh + t/8 + shift) mod hp, (8ww + t%8 + shift) mod wp). A lone last
// head (odd head count) leaves its pair's second-head columns unwritten.
__host__ __device__ constexpr int attn_unit_stride(int hd) { return 6 * hd + 2; }
inline size_t attn_unit_floats(int hp, int wp, int heads, int hd) {
    return (size_t)(hp / 8) * (wp / 8) * ((heads + 1) / 2) * 64 * attn_unit_stride(hd);
}
// The window attention that reads the unit layout takes these head shapes.
bool attn_unit_eligible(int heads, int hd, int c);
// The forward writes qkv in the unit layout (one GEMM, then the unit
// attention) for these shapes, in the plane layout [P][3c] otherwise.
bool qkv_unit_layout(int heads, int hd, int c);

struct GemmArgs {
    // A operand: ALOAD_ROWS -> A[m*lda + k]; ALOAD_IM2COL -> the 3x3 im2col
    // view of the channel-last plane A[H*W][cin], k = tap*cin + ci.
    const float *A;
    int lda;
    int H, W, cin;
    // B operand: weight rows B[n*ldb + k].
    const float *B;
    int ldb;
    const float *bias;  // [N] or null
    float *out;
    int ldo;
    const float *res;  // residual [M][ldr]
    int ldr;
    const float *ln_w, *ln_b;
    float slope;
    int feat;  // EPI_SHUFFLE: output channels (N = 4*feat)
    // EPI_QKV_WIN: the plane is H x W, the block's shift, heads of head_dim
    // hd (N = 3 * heads * hd)
    int shift, heads, hd;
    // EPI_SHUFFLE_FINISH: scale, output crop, img_range and the RGB mean
    int scale, oh, ow;
    float img_range, mean[3];
    int M, N, K;
    // A batch of nb independent row GEMMs (0 or 1 = one; ALOAD_ROWS, store
    // epilogue, no bias): A, B and out advance by a_bstride, b_bstride and
    // o_bstride floats per batch (out may be A: each row's output is stored
    // after that row has been read)
    int nb;
    size_t a_bstride, b_bstride, o_bstride;
    // B in k_bsgemm's register order (bs_pack_weights, b_bstride counting that
    // layout's floats) instead of rows [N][ldb]: only k_bsgemm reads that
    // layout (it reads both)
    int b_packed;
};

// k_bsgemm's weight layout, "register order": for each column group, K half,
// column wave and 16-column MFMA tile, one block holding, for every k group of
// 16, the 64 lanes' float4s lane after lane (1 KiB), then for the K tail of R
// steps R dwords per lane, lane after lane; columns past the group are zeros.
// Each weight load of the kernel then reads 1 KiB contiguous, where the rows
// [N][K] layout has it read 64 bytes of each of 16 rows. bs_weight_floats is a
// weight's size in that layout (0: no k_bsgemm shape; it depends on N, K and
// the epilogue only); bs_pack_weights writes it from host rows w [N][ldb].
size_t bs_weight_floats(int N, int K, int epi);
void bs_pack_weights(const float *w, int ldb, int N, int K, int epi, float *dst);
// the GEMM's shape is one k_bsgemm runs (with B packed)
bool bs_takes(const GemmArgs &g, int aload, int epi);

// The weight-stationary token GEMM (k_bsgemm): out = epi(A B^T + bias) with A
// [M][lda] rows, B [N][ldb] rows. Set by the launcher: P (workgroups per
// column group) and ngw (columns per group).
struct BsArgs {
    const float *A;
    int lda;
    const float *B;
    int ldb;
    const float *bias;
    float *out;
    int ldo;
    const float *res;
    int ldr;
    const float *ln_w, *ln_b;
    float slope;
    int M, N, K;
    int P, ngw;
    // EPI_QKV_WIN: plane hp x wp (nww windows per row), shift, head shape
    int hp, wp, nww, shift, heads, hd;
    // batches (nb >= 1) and their strides in floats
    int nb;
    size_t a_bs, b_bs, o_bs;
    int bpk;  // B in register order (bs_pack_weights), else rows [N][ldb]
};

// The attention kernels run the softmax in base 2: logits scaled by log2(e)
// (the CPB table cpbt is stored scaled, the logit scale and the mask constant
// carry the factor), so each probability is one v_exp_f32 of (s - max)
// instead of a multiply and the exp. exp(s - m) = 2^((s - m) log2 e), and the
// maximum is unchanged by the positive factor.
#define ATTN_LOG2E 1.4426950408889634f

struct AttnArgs {
    const float *qkv;          // unit ? the unit layout : [hp*wp][3c] plane order q | k | v
    int unit;                  // qkv is in the unit layout (needs attn_unit_eligible)
    const float *cpbt;         // [heads][64][64], CPB bias x ATTN_LOG2E
    const float *logit_scale;  // [heads]
    float *out;                // [hp*wp][c]
    int hp, wp, nww, nw;
    int heads, head_dim, c;
    int shift;
    int nws;                   // k_wattn: window lanes per XCD (set by launch_attention)
};

// A block's qkv projection and window attention in one kernel (k_qkv_wattn)
// for 6 heads of 30: x [hp*wp][180], the q|k|v weight rows of each head pair
// in the attention unit's column order w [3][180][180] and bias [3][180]
// (qkv_pair_weights), the CPB table and logit scales as for AttnArgs; out
// [hp*wp][180].
struct QkvAttnArgs {
    const float *x;
    const float *w;
    const float *bias;
    const float *cpbt;         // [6][64][64], CPB bias x ATTN_LOG2E
    const float *logit_scale;  // [6]
    float *out;
    int hp, wp, nww, nw;
    int shift;
    int nws;                   // window lanes per XCD (set by launch_qkv_attention)
};
inline bool qkv_attn_fused(int heads, int hd) { return heads == 6 && hd == 30; }
// The fused [3c][c] qkv weight (rows q, k, v) and bias [3c] re-laid out per
// head pair: w_out [heads/2][6 hd][c] with rows [q_2p | q_2p+1 | k_2p |
// k_2p+1 | v_2p | v_2p+1], b_out [heads/2][6 hd] alike.
void qkv_pair_weights(const float *w, const float *b, int heads, int hd, float *w_out,
                      float *b_out);
hipError_t launch_qkv_attention(const QkvAttnArgs &g, hipStream_t st, unsigned *grid_out);
unsigned qkv_attention_grid(int hp, int wp);

// A block's qkv projection as the forward launches it: x [hp*wp][c] times
// the fused [3c][c] weight plus [q_bias | 0 | v_bias], written in the window
// attention's unit layout (EPI_QKV_WIN; A rows read in the block's
// shifted-window order) when the head shape takes it, else in the plane
// layout [hp*wp][3c] (EPI_STORE). Returns the epilogue to launch with.
inline int qkv_gemm_args(const float *x, const float *wqkv, const float *bqkv, float *qkv,
                         int hp, int wp, int shift, int heads, int hd, GemmArgs *g) {
    const int c = heads * hd;
    *g = GemmArgs{};
    g->A = x;
    g->lda = c;
    g->B = wqkv;
    g->ldb = c;
    g->bias = bqkv;
    g->out = qkv;
    g->ldo = 3 * c;
    g->M = hp * wp;
    g->N = 3 * c;
    g->K = c;
    g->H = hp;
    g->W = wp;
    g->shift = shift;
    g->heads = heads;
    g->hd = hd;
    return qkv_unit_layout(heads, hd, c) ? EPI_QKV_WIN : EPI_STORE;
}

// The window attention over that qkv buffer, output scattered back to the
// plane [hp*wp][c] (cpbt [heads][64][64] x log2(e), logit_scale [heads]).
inline AttnArgs window_attn_args(const float *qkv, const float *cpbt, const float *logit_scale,
                                 float *out, int hp, int wp, int shift, int heads, int hd) {
    AttnArgs a{};
    a.qkv = qkv;
    a.unit = qkv_unit_layout(heads, hd, heads * hd);
    a.cpbt = cpbt;
    a.logit_scale = logit_scale;
    a.out = out;
    a.hp = hp;
    a.wp = wp;
    a.nww = wp / 8;
    a.nw = (hp / 8) * a.nww;
    a.heads = heads;
    a.head_dim = hd;
    a.c = heads * hd;
    a.shift = shift;
    return a;
}

#define GEMM_NVARIANTS 6
hipError_t launch_gemm(const GemmArgs &g, int aload, int epi, hipStream_t st);
hipError_t launch_gemm_variant(const GemmArgs &g, int aload, int epi, int variant,
                               hipStream_t st);
int gemm_pick(const GemmArgs &g, int aload, int epi);
void gemm_grid(const GemmArgs &g, int aload, int epi, unsigned *gx, unsigned *gy);
void gemm_variant_grid(const GemmArgs &g, int variant, unsigned *gx, unsigned *gy);
const char *gemm_kernel_name(const GemmArgs &g, int aload, int epi);
// The launch geometry launch_gemm will use for these arguments (for the
// profiler's rows), and the kernel family name it picks.
void gemm_geometry(const GemmArgs &g, int aload, int epi, dim3 *grid, dim3 *block);
hipError_t launch_attention(const AttnArgs &g, hipStream_t st, unsigned *grid_out);
// Winograd F(4x4,3x3) for a 3x3 stride-1 zero-pad-1 conv on a channel-last
// H x W plane (C % 4 == 0): wino_weights transforms the [co][ci][3][3]
// weights to U = G g G^T, the GEMM's B [36][co][round4(ci)] (double
// accumulation, rounded once); launch_wino_in writes V = B^T d B of every 4x4
// output tile's 6x6 input patch (zero outside the plane) as [36][T][C] for the
// T = wino_tiles(H, W) tiles; a batch of 36 row GEMMs M[b] = V[b] U[b]^T (over
// M's own buffer); launch_wino_out transforms M back (Y = A^T M A), adds the
// bias, then the residual `res` [H*W][ldr] if set, then LeakyReLU(slope) if
// `lrelu`, into out [H*W][ldo] (the tiles' pixels inside the plane).
constexpr int WINO_POS = 36;
inline size_t wino_tiles(int H, int W) { return (size_t)((H + 3) / 4) * ((W + 3) / 4); }
// Winograd F(2x2,5x5) for the x4 head's composed 5x5 conv (F = 64 -> 48, the
// pixel_shuffle(4) finish): the same six points and B^T; the 2x2 output
// tiles covering Ho x Wo pixels of an H x W plane, the patch origin 2t - 2.
// wino5_weights: U = G5 g G5^T from the composed weights [48][25][F] (double,
// rounded once) as [36][48][F]; launch_wino5_in writes V [36][T][F];
// launch_wino5_finish takes M [36][T][ldm] (48 used) to Y = A5^T M A5 + bias,
// pixel_shuffle(4), denormalised (v / img_range + mean) and cropped to oh x ow
// into out [3][oh][ow].
inline size_t wino5_tiles(int Ho, int Wo) { return (size_t)((Ho + 1) / 2) * ((Wo + 1) / 2); }
inline bool wino_up2(int octaves, int feat) { return octaves == 2 && feat == 64; }
void wino5_weights(const double *w, int co, int ci, float *out);
hipError_t launch_wino5_in(const float *in, int ldi, float *v, int H, int W, int Ho, int Wo, int C,
                           hipStream_t st);
unsigned wino5_in_grid(int Ho, int Wo, int C);
hipError_t launch_wino5_finish(const float *m, int ldm, const float *bias, float *out, int Ho,
                               int Wo, int oh, int ow, float img_range, const float *mean,
                               hipStream_t st);
unsigned wino5_finish_grid(int Ho, int Wo);
void wino_weights(const float *w, int co, int ci, float *out);
// The body's C -> C convs take the Winograd path when the batched GEMM runs on
// the weight-stationary kernel with every column in one workgroup (so it may
// write M over V in place): C in {60, 120, 180}, every released width.
inline bool wino_body(int c) { return c == 60 || c == 120 || c == 180; }
// conv_before_upsample (C -> F, then LeakyReLU) takes the Winograd path when C
// is a body width above and F fits one narrow (64-column) group of the
// weight-stationary kernel; its products go to a buffer of their own.
inline bool wino_head(int c, int f) { return wino_body(c) && f % 4 == 0 && f <= 64; }
hipError_t launch_wino_in(const float *in, int ldi, float *v, int H, int W, int C, hipStream_t st);
unsigned wino_in_grid(int H, int W, int C);   // the launches' 1-D grids of 256 threads
unsigned wino_out_grid(int H, int W, int C);
hipError_t launch_wino_out(const float *m, const float *bias, const float *res, int ldr,
                           float *out, int ldo, int H, int W, int C, int lrelu, float slope,
                           hipStream_t st);
unsigned attention_grid(const AttnArgs &g);
hipError_t launch_pad_input(const float *in, float *out, int h, int w, int hp, int wp,
                            hipStream_t st);
hipError_t launch_layernorm(const float *x, const float *w, const float *b, const float *res,
                            float *out, int P, int C, hipStream_t st);
// conv_first and the folded patch_embed + LayerNorm in one pass over the padded
// input in4 [H*W][4] (channel 3 zero): wts [2][9][4][C] (set 0 conv_first, set
// 1 patch_embed folded in; tap-major, then input channel, channels fastest),
// biases b0, b1 [C], LayerNorm lnw, lnb [C]; body and cur are [H*W][C].
hipError_t launch_embed(const float *in4, const float *wts, const float *b0, const float *b1,
                        const float *lnw, const float *lnb, float *body, float *cur, int H, int W,
                        int C, hipStream_t st);
dim3 conv_last_grid(int oh, int ow);
// `in` is the H x W x feat plane, channel-last.
hipError_t launch_conv_last_finish(const float *in, const float *wt, const float *bias,
                                   float *out, int H, int W, int feat, int oh, int ow,
                                   float img_range, const float *mean, hipStream_t st);
// The classical head's last pixel-shuffle octave + conv_last + finish, composed:
// `in` is the octave's H x W x feat input plane (channel-last), `wt` the
// composed interior weights [25][feat][12] and `bias` [12], `wedge` the four
// edge variants [4][12][25][feat] and `bedge` [4][12]; out is [3][oh][ow].
// Two launches (the interior, then the top row and left column).
dim3 up_last_grid(int oh, int ow);
hipError_t launch_up_last(const float *in, const float *wt, const float *bias, const float *wedge,
                          const float *bedge, float *out, int H, int W, int feat, int oh, int ow,
                          float img_range, const float *mean, hipStream_t st);
// The two-octave composition's edge outputs (input row 0 and column 0), after
// the ALOAD_IM2COL5 / EPI_SHUFFLE_FINISH GEMM (feat = 64): weights [4][48][25][feat],
// biases [4][48].
hipError_t launch_up2_last_edge(const float *in, const float *wedge, const float *bedge, float *out,
                               int H, int W, int feat, int oh, int ow, float img_range,
                               const float *mean, hipStream_t st);
// The four phases' 2x2 weights of a 3x3 conv w [co][ci][3][3] applied to a
// nearest-2x upsampling (ALOAD_SUB2's B): [4][co][4][ci_pad4] at out.
void subpixel_weights(const float *w, int co, int ci, float *out);
// torch's bicubic resize (a = -0.75, align_corners = False, edge clamp) of a
// channel-last [h*w][4] plane to [oh*ow][4] (channel 3 stays 0).
hipError_t launch_bicubic4(const float *in, float *out, int h, int w, int oh, int ow,
                           hipStream_t st);
// The compressed head's bicubic branch through conv_last, added into the
// finished output: out[k][Y][X] += (bias[v][k] + sum over the 5x5 taps t and
// the 3 channels c of w[v][t][k][c] * bic[Y + t/5 - 2][X + t%5 - 2][c]) /
// img_range over the cropped oh x ow image, bic the [qh*qw][4] bicubic plane
// (zero outside), v = 2 (Y == 0) + (X == 0) the edge variant; weights
// [4][25][3][4] (c = 3 unused), biases [4][3].
hipError_t launch_bic_last_add(const float *bic, int qh, int qw, const float *w, const float *bias,
                               float *out, int oh, int ow, float img_range, hipStream_t st);
// The compressed head's conv_aux (feat -> 3, 3x3, zero pad; weights [tap][ci][3]
// as conv_last's) over the H x W plane with cpu::finish_aux: the conv's output
// to aux4 [H*W][4] (channel 3 zero) and the aux image v / img_range + mean to
// auxp [3][H][W].
hipError_t launch_conv_aux(const float *in, const float *wt, const float *bias, float *aux4,
                           float *auxp, int H, int W, int feat, float img_range, const float *mean,
                           hipStream_t st);
hipError_t launch_cpb(const float *w0, const float *b0, const float *w2, float *tab, float *cpbt,
                      int win, int heads, hipStream_t st);
hipError_t launch_window_map(int hp, int wp, int shift, int32_t *yx, uint8_t *reg,
                             hipStream_t st);
// The fp32 MFMA peak probe: `blocks` workgroups of 512 threads, each wave
// issuing 4 * iters independent v_mfma_f32_16x16x4f32; one float per thread
// to `out` (blocks * 512 floats).
hipError_t launch_mfma_peak(float *out, int blocks, int iters, hipStream_t st);

// The ABI's thread-local error slot (defined in s2s_api.cpp): records `msg`
// for s2s_last_error() and returns -1. Internal to the library.
__attribute__((visibility("hidden"))) int s2s_fail(const char *msg);
// A context's embed width (channels of its planes); 0 for a null context.
struct s2s_ctx;
__attribute__((visibility("hidden"))) int s2s_ctx_embed(struct s2s_ctx *ctx);
