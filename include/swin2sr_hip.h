/* swin2sr_hip.h - the C ABI of the MI355X (gfx950) swin2sr backend.
 *
 * This is the drop-in boundary for the device half of the swin2sr crate: every
 * entry point below replaces one thing the crate's CUDA backend does today
 * (`src/gpu.rs` over `src/cuda.rs` over `lightgpu::vm`), and each declaration
 * names the reference interface it stands in for. The Rust side binds these
 * with `extern "C"` (the binding a maintainer adds is shown in INTEGRATION.md
 * at the repository root); the C++ harnesses and the Python tests bind the same
 * symbols.
 *
 * Conventions, all of them inherited from the crate's `Backend` contract:
 *  - Every call that can fail returns int: 0 = ok, non-zero = error, and
 *    `s2s_last_error()` holds the message (thread-local, owned by the library).
 *    An allocation failure's message contains "out of memory", which is what
 *    `run_with_fallback`'s `is_out_of_memory` keys its tile-halving retry on
 *    (reference src/main.rs:655-662).
 *  - Images at the boundary are planar `[3][h][w]` f32. The forward input is
 *    MEAN-ADJUSTED by the caller (`Pre::adjust`, reference src/backend.rs:76-86)
 *    and the output is denormalised and cropped, `[3][h*scale][w*scale]`.
 *  - One context = one HIP stream = one host thread at a time (the reference's
 *    `Backend` takes `&mut self`, src/backend.rs:29-49). No internal threads.
 *  - Weights are borrowed for the duration of `s2s_create` only; they are
 *    copied (and re-laid-out) onto the device there.
 */
#ifndef SWIN2SR_HIP_H
#define SWIN2SR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Every symbol below is exported even when the library is built with hidden
 * default visibility. */
#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility push(default)
#endif

/* The reconstruction head (reference src/weights.rs:19-29, `Upsampler`). */
enum s2s_upsampler {
    S2S_PIXELSHUFFLE = 0,        /* classical SR: conv+lrelu, (conv3x3 + shuffle2) per octave, conv_last */
    S2S_PIXELSHUFFLE_DIRECT = 1, /* lightweight SR: one conv to 3*s^2 + pixel_shuffle(s) */
    S2S_NEAREST_CONV = 2,        /* real-world SR: two nearest x2 + conv + lrelu(0.2) */
    S2S_PIXELSHUFFLE_AUX = 3     /* compressed SR: pixelshuffle + bicubic branch + aux image */
};

#define S2S_MAX_STAGES 16

/* The architecture the checkpoint's `__metadata__` describes
 * (reference src/weights.rs:66-137: task, upsampler, scale, window_size,
 * embed_dim, num_heads, mlp_ratio, depths, img_range, rgb_mean). */
typedef struct s2s_arch {
    int upsampler;              /* enum s2s_upsampler */
    int scale;
    int window;
    int embed;
    int heads;                  /* head_dim = embed / heads */
    int mlp_ratio;
    int n_stages;
    int depths[S2S_MAX_STAGES]; /* blocks per RSTB stage */
    float img_range;
    float mean[3];
} s2s_arch;

/* One named f32 tensor of the crate's checkpoint (tensor names and shapes as
 * `Weights::validate` checks them, reference src/weights.rs:142-235).
 * `data` is row-major in the checkpoint's (torch) layout. */
typedef struct s2s_tensor {
    const char *name;
    const float *data;
    int ndim;
    int64_t shape[4];
} s2s_tensor;

typedef struct s2s_ctx s2s_ctx;

/* ---- construction ------------------------------------------------------ */

/* Replaces `Gpu::new(&Weights)` (reference src/gpu.rs:101-125): opens the
 * device, creates the context's stream, validates the tensor set against
 * `arch` and uploads it once, re-laid-out for the kernels. */
int s2s_create(const s2s_arch *arch, const s2s_tensor *tensors, size_t n_tensors,
               s2s_ctx **out);

/* Frees every device allocation the context owns (the reference frees on
 * `Drop` of `Gpu`/`Acts`, src/gpu.rs:41-81). NULL is ignored. */
void s2s_destroy(s2s_ctx *ctx);

/* `Backend::name` (reference src/gpu.rs:737-739 returns "cuda"): "hip". */
const char *s2s_name(void);

/* `gpu::uploaded_bytes` (reference src/gpu.rs:792-799): the bytes the
 * context holds on the device for the weights. */
uint64_t s2s_uploaded_bytes(const s2s_ctx *ctx);

/* `gpu::uploaded_bytes(&Weights)` (reference src/gpu.rs:792-799) as the crate
 * calls it: from the checkpoint alone, before any backend exists
 * (`memory_budget`, reference src/main.rs:459-471). `*bytes` is exactly what
 * `s2s_create` will upload for this architecture and tensor set (the weights
 * as the kernels read them - re-laid-out, folded, composed - and the CPB
 * tables), so `s2s_uploaded_bytes` of the context it makes equals it. */
int s2s_uploaded_bytes_for(const s2s_arch *arch, const s2s_tensor *tensors, size_t n_tensors,
                           uint64_t *bytes);

/* The device bytes a forward of an h x w image allocates in this context
 * (the body plan and the image plan, the host path's device copies of the
 * input and output included): this backend's exact counterpart of the figure
 * the crate models as `activation_bytes` / `per_pixel_floats(gpu = true)`
 * (reference src/backend.rs:205-212, 300-383), which it never exceeds. */
int s2s_plan_bytes(s2s_ctx *ctx, int h, int w, uint64_t *bytes);

/* A cap on the bytes of the per-image plans (`s2s_plan_bytes`); 0 = none, the
 * default, or the value of SWIN2SR_HIP_ALLOC_LIMIT (bytes) at `s2s_create`. A
 * forward whose plan would pass it fails like a failed allocation, with
 * "out of memory" in the message - the error the crate's tile-halving retry
 * keys on (`run_with_fallback` / `is_out_of_memory`, reference
 * src/main.rs:579-662). No counterpart in the reference (the CUDA driver's
 * own limit is the only one there): it lets a caller reserve device memory,
 * and a test drive that retry. */
int s2s_set_alloc_limit(s2s_ctx *ctx, uint64_t bytes);

/* ---- the forward pass ---------------------------------------------------- */

/* `Backend::forward` for the device (reference src/gpu.rs:741-754 and
 * `forward_plan`, :462-583). `in_adjusted` is host `[3][h][w]`, mean-adjusted;
 * `out` is caller-owned host `[3][h*scale][w*scale]`. Buffers are planned per
 * (h, w) and reused while the size repeats. Synchronous: returns when the
 * download has completed. */
int s2s_forward(s2s_ctx *ctx, int h, int w, const float *in_adjusted, float *out);

/* `n` host images through `s2s_forward`'s path (sizes may differ: a tiled
 * image's crops), alternating between the context and the second lane of
 * `s2s_forward_device_batch` and pipelined, so that one lane computes while
 * the other's image is downloaded and copied out. `in_adjusted[i]`, `out[i]`
 * as for `s2s_forward` with `h[i]`, `w[i]`; `aux_out` may be NULL, or hold per
 * image a NULL or a caller-owned `[3][hp][wp]` buffer that receives that
 * image's aux image (the compressed head's; `s2s_aux` afterwards returns the
 * last image's). No reference counterpart: it is what a tile loop calls with a
 * whole image's tiles (reference `run_tiled`, src/backend.rs:92-165, calls
 * `Backend::forward` once per tile); each result equals `s2s_forward`'s for
 * its input bit for bit. Synchronous: returns when every output is written. */
int s2s_forward_batch(s2s_ctx *ctx, int n, const int *h, const int *w, const float *const *in_adjusted,
                      float *const *out, float *const *aux_out);

/* The same pass on device-resident buffers (no host copies): `d_in` is a
 * device `[3][h][w]` mean-adjusted plane, `d_out` a device
 * `[3][h*scale][w*scale]` buffer. Enqueued on the context's stream and NOT
 * synchronised; `s2s_stream` / `s2s_sync` order it. No reference counterpart:
 * the crate always hands over host slices; this is the entry a caller with
 * inputs already in HBM (the throughput harness) uses. The second call in a
 * row with the same (h, w, d_in, d_out) and buffer plan captures the pass's
 * launches into a HIP graph, which later such calls replay (the same kernels;
 * SWIN2SR_HIP_GRAPHS=0 at `s2s_create` turns this off; profiling launches
 * eagerly). A caller may capture the context's stream around this call: the
 * launches are then recorded in the caller's graph, provided the buffers for
 * (h, w) are already planned (one call of that size before the capture);
 * otherwise the call is refused with an error, since planning allocates and
 * synchronises the stream, and the context is left as it was.
 * `s2s_forward` runs this pass on its own device copies. */
int s2s_forward_device(s2s_ctx *ctx, int h, int w, const float *d_in, float *d_out);

/* `n` images of one size on device-resident buffers (`d_in[i]`, `d_out[i]` as
 * for `s2s_forward_device`), alternating between the context's stream and a
 * second lane the context makes on first use: a stream of its own, buffer
 * plans of its own (a second `s2s_plan_bytes` worth of device memory, kept
 * until `s2s_destroy`) and graphs of its own, over the same uploaded weights.
 * One image's kernel boundaries (each launch's start and its last, partial
 * round, where CUs idle) then overlap the other's kernels. No reference
 * counterpart (the crate forwards one image at a time): it is the serving
 * entry, for callers with several images in HBM. The lane starts after the
 * work already on the context's stream, and the context's stream waits for
 * the lane, so `s2s_stream` / `s2s_sync` order the whole batch; not
 * synchronised on return. Each output equals `s2s_forward_device`'s for its
 * input bit for bit. */
int s2s_forward_device_batch(s2s_ctx *ctx, int n, int h, int w, const float *const *d_in,
                             float *const *d_out);

/* `s2s_forward_device` without allocating anything: every intermediate
 * buffer is carved out of a static device workspace of 256 MiB per GPU
 * (a file-scope array the library holds on each GPU it runs on until the
 * process ends), and the call makes no hipMalloc, hipFree or other allocating
 * call (no profiler events either). No counterpart in the reference: it is
 * for callers that cannot allocate - code under HIP graph capture, tight
 * serving loops, harnesses that forbid it. The caller passes the device input
 * and output as for `s2s_forward_device`; enqueued on the context's stream,
 * not synchronised. Planes whose buffers do not fit the workspace are refused
 * with an error (classical x4 at C = 180: padded planes up to ~38,900 pixels,
 * i.e. images up to 191 x 191; `s2s_plan_bytes` less the two host-path copies
 * is the figure). Every call on one GPU shares that GPU's workspace, which
 * keeps the last call's contents. Eager calls are ordered on the device: each
 * makes its stream wait for the workspace's previous user (an event the
 * library creates per GPU at `s2s_create`) and records itself as the last, so
 * contexts on different streams take the workspace in the order their calls
 * were made. A call captured into a caller's graph is not ordered that way:
 * its replays run when the caller launches them, so a replay that overlaps
 * another call or replay on the same GPU races on the workspace. */
int s2s_forward_device_noalloc(s2s_ctx *ctx, int h, int w, const float *d_in, float *d_out);

/* `Backend::aux` (reference src/gpu.rs:756-758): the last forward's secondary
 * image, denormalised, at the PADDED plane's geometry `[3][hp][wp]`. `*n` is 0
 * (and `*ptr` NULL) when the head makes none. Valid until the next forward. */
int s2s_aux(s2s_ctx *ctx, const float **ptr, size_t *n);

/* ---- errors and device queries ------------------------------------------ */

/* The message of the last failed call on this thread ("" if none). */
const char *s2s_last_error(void);

/* `vm::device()` (reference src/main.rs:169,516-517): the device name and its
 * architecture string ("gfx950..." here, where the crate prints sm_xx). */
int s2s_device_info(char *name, size_t name_cap, char *arch, size_t arch_cap);

/* `vm::vram()` (reference src/main.rs:461): free and total device bytes. */
int s2s_vram(uint64_t *free_bytes, uint64_t *total_bytes);

/* `vm::sync()` (reference src/main.rs:342): waits for all device work. */
int s2s_sync(void);

/* The context's hipStream_t, as an opaque pointer (for callers that enqueue
 * their own work or timing events around `s2s_forward_device`). */
void *s2s_stream(s2s_ctx *ctx);

/* ---- profiling ----------------------------------------------------------- */

/* The per-launch event profiler of reference src/cuda.rs:109-140,156-259,
 * switched on by SWIN2SR_PROFILE_GPU at `s2s_create` or by this call. While on,
 * every kernel launch is bracketed by a hipEvent pair on the context stream. */
int s2s_profile_enable(s2s_ctx *ctx, int on);

/* Clears the accumulated profile rows. */
int s2s_profile_reset(s2s_ctx *ctx);

/* `Profile::report(total_wall_ms)` (reference src/cuda.rs:239-259): prints one
 * row per (kernel, grid, block) to stderr, after synchronising the stream. */
int s2s_profile_report(s2s_ctx *ctx, float wall_ms);

/* Totals for one kernel name over all its rows: summed device milliseconds and
 * launch count (after synchronising). Unknown names give 0 and 0. */
int s2s_profile_query(s2s_ctx *ctx, const char *kernel, double *total_ms, int *launches);

/* Restricts the profiler's event pairs to launches of one kernel name (NULL or
 * "" = every launch, the default), so a timed run can carry the events of the
 * kernel it reports without bracketing the others. No counterpart in the
 * reference (its profiler always brackets every launch); a measurement aid. */
int s2s_profile_only(s2s_ctx *ctx, const char *kernel);

/* ---- the single-RSTB path (config 1 micro-bench) -------------------------- */

/* One residual Swin transformer block group (stage `stage` of the checkpoint:
 * its blocks, then conv3x3, 1x1 and the stage residual), on an explicit
 * `hp x wp` plane (both multiples of the window; NOT re-padded), channel-last
 * `[hp*wp][embed]` device buffers. In place is allowed (d_in == d_out).
 * Reference: the stage loop of src/gpu.rs:481-529 / src/cpu.rs:1516-1581. */
int s2s_rstb_device(s2s_ctx *ctx, int stage, int hp, int wp, const float *d_in, float *d_out);

/* ---- self-test ------------------------------------------------------------ */

/* `gpu::selftest(&Weights)` behind `--cuda-selftest` (reference
 * src/gpu.rs:889-1265, src/main.rs:180-192): every kernel of the forward on a
 * small deterministic input (x[i] = sin(0.7 i + phase), the reference's
 * generator) against the operation's definition evaluated on the host in
 * double precision, at the reference selftest's shapes and at the
 * checkpoint's own width and head shape; plus the checkpoint's CPB tables
 * (the device MLP against `cpb_pre`, where the set carries both). Prints
 * "hip selftest: N kernel/shape pairs checked ..." to stdout on success;
 * otherwise fails naming the check, the worst element and both values.
 * `tensors` may be NULL (no CPB check). */
int s2s_selftest(const s2s_arch *arch, const s2s_tensor *tensors, size_t n_tensors);

/* ---- per-op test entry points -------------------------------------------- */
/* The device half of `gpu::selftest` (reference src/gpu.rs:889-1265): each runs
 * one kernel on host buffers (uploads, launches, downloads, synchronises) so a
 * harness can hold it against the CPU definition. Planes here are CHANNEL-LAST
 * `[h*w][c]` (the layout this backend keeps activations in); token tables are
 * in plane order. */

/* `Plan::index` / `Plan::region` (reference src/plan.rs:72-108) as the device
 * computes them: for every (window wi, token t) of a `hp x wp` plane,
 * `yx[(wi*n+t)*2+{0,1}]` = plane (y, x) read at `shift`, and
 * `reg[(wi*n+t)*2+{0,1}]` = the mask band (row, column). */
int s2s_test_window_map(int hp, int wp, int win, int shift, int32_t *yx, uint8_t *reg);

/* The production shifted-window gather (`Plan::index`, reference
 * src/plan.rs:72-78; the CUDA build's `ss_window_gather`, cuda/swin2sr.cu:
 * 99-135): a block's qkv GEMM exactly as the forward launches it, whose A rows
 * are read window by window in the shifted order and stored in the window
 * attention's unit layout - one unit per (window, head pair), 64 token rows of
 * 6*head_dim + 2 floats: [q_h0 | q_h1 | k_h0 | k_h1 | v_h0 | v_h1 | 2 pad].
 * `x` is `[hp*wp][c]`, `wqkv` `[3c][c]`, `bqkv` `[3c]`; `unit` receives the raw
 * buffer (`unit_cap` >= its size in floats; unwritten padding reads NaN).
 * Only for the head shapes that use the unit layout. */
int s2s_test_qkv_windows(int hp, int wp, int heads, int head_dim, int shift, const float *x,
                         const float *wqkv, const float *bqkv, float *unit, size_t unit_cap);

/* The production attention half of a block: the qkv GEMM above, then the
 * window attention with the shift mask (`Plan::region`, reference
 * src/plan.rs:84-108) and the scatter back to the plane (`cpu::scatter`,
 * src/cpu.rs:1200-1222), exactly as the forward launches them - for 6 heads
 * of 30 as the forward's one fused kernel (the qkv projection and the
 * attention together, the projection's shifted-window gather inside it).
 * `x` is `[hp*wp][c]`, `wqkv` the fused `[3c][c]` (rows q, k, v), `cpb`
 * `[n*n][heads]` (the checkpoint's cpb_pre layout), `out` `[hp*wp][c]`. */
int s2s_test_block_attention(int hp, int wp, int heads, int head_dim, int shift, const float *x,
                             const float *wqkv, const float *bqkv, const float *logit_scale,
                             const float *cpb, float *out);

/* Window attention (reference cpu::attention, src/cpu.rs:1244-1402): `qkv` is
 * `[hp*wp][3*c]` in plane order (q | k | v per pixel), `cpb` the `[n*n][heads]`
 * table in the checkpoint's layout, `logit_scale` `[heads]`. `out` is
 * `[hp*wp][c]`. Window must be 8 (n = 64), head_dim <= 32. */
int s2s_test_attention(int hp, int wp, int win, int heads, int head_dim, int shift,
                       const float *qkv, const float *logit_scale, const float *cpb,
                       float *out);

/* The device CPB table from the MLP weights (reference tools/convert.py:141-167):
 * `out` is `[n*n][heads]`, 16*sigmoid(MLP(log-spaced coords)) gathered. */
int s2s_test_cpb_table(int win, int heads, const float *w0 /*[512][2]*/,
                       const float *b0 /*[512]*/, const float *w2 /*[heads][512]*/,
                       float *out);

/* Token GEMM with an epilogue (reference cpu::linear, src/cpu.rs:607-625, and
 * the ops the build fuses behind it). `x` is `[rows][c_in]`, `w` `[c_out][c_in]`,
 * `bias` `[c_out]` (NULL = zero). `res` `[rows][c_out]` is read by the
 * residual epilogues; `ln_w`/`ln_b` `[c_out]` by the LayerNorm ones.
 * epilogue: 0 store, 1 erf-GELU, 2 += res, 3 LayerNorm, 4 res + LayerNorm,
 * 5 LeakyReLU(slope). LayerNorm epilogues need c_out <= 192. */
int s2s_test_linear(int rows, int c_in, int c_out, const float *x, const float *w,
                    const float *bias, int epilogue, const float *res, const float *ln_w,
                    const float *ln_b, float slope, float *out);

/* Channel LayerNorm over `[hw][c]` (reference cpu::channel_layer_norm,
 * src/cpu.rs:1019-1073), optionally `y = res + LN(x)` when `res` is non-NULL. */
int s2s_test_ln_residual(int hw, int c, const float *x, const float *ln_w, const float *ln_b,
                         const float *res, float *out);

/* The forward's first kernel as it runs it (reference src/gpu.rs:474-478):
 * conv_first (3 -> c, 3x3, zero pad) of a channel-last `[h*w][3]` image, and
 * the same image through a second set of 3x3 weights (patch_embed's 1x1 conv
 * folded into conv_first, as s2s_create forms it) followed by the channel
 * LayerNorm (reference cpu::channel_layer_norm, src/cpu.rs:1019-1073).
 * Weights `[c][3][3][3]`, biases and LayerNorm parameters `[c]`; outputs
 * `body` (conv_first) and `cur` (the LayerNorm's), both `[h*w][c]`.
 * c % 4 == 0, c <= 192. */
int s2s_test_embed(int h, int w, int c, const float *x, const float *w_first, const float *b_first,
                   const float *w_fold, const float *b_fold, const float *ln_w, const float *ln_b,
                   float *body, float *cur);

/* 3x3 stride-1 zero-pad-1 convolution (reference cpu::conv3x3, src/cpu.rs:
 * 400-414) on a channel-last `[h*w][c_in]` plane, weights `[c_out][c_in][3][3]`,
 * output `[h*w][c_out]`. epilogue: 0 store, 2 += res, 5 LeakyReLU(slope). */
int s2s_test_conv3x3(int h, int w, int c_in, int c_out, const float *x, const float *wgt,
                     const float *bias, int epilogue, const float *res, float slope, float *out);

/* The body's C -> C 3x3 convs as the forward runs them for the released
 * widths (the stage close, conv_after_body): Winograd F(4x4,3x3) - the
 * weights transformed as at upload, the input transform, the 36
 * transform-position GEMMs on the weight-stationary kernel, the output
 * transform with the bias and the epilogue (0 store, 2 += res, 5
 * LeakyReLU(slope)) - against the reference's direct cpu::conv3x3
 * (src/cpu.rs:400-414; the reference's own CUDA backend runs these convs as
 * Winograd with 6x6 tiles, src/gpu.rs:161-181). Also conv_before_upsample's
 * C -> F conv, which the head runs the same way (F <= 64, a multiple of 4,
 * on the narrow build of the GEMM, its products in a buffer of their own).
 * Channel-last `[h*w][c_in]` in, `[h*w][c_out]` out; any h, w >= 1;
 * c_in == c_out == C in {60, 120, 180}, or c_in = C and c_out = F. */
int s2s_test_conv3x3_winograd(int h, int w, int c_in, int c_out, const float *x, const float *wgt,
                              const float *bias, int epilogue, const float *res, float slope,
                              float *out);

/* The real-world head's conv_up1 / conv_up2 (reference src/gpu.rs:641-669:
 * nearest-2x upsampling, conv3x3 c -> c, LeakyReLU(slope)) as the forward
 * runs them: the four 2x2 convs of the plane itself, one per output phase,
 * whose weights are sums of the 3x3 taps that land on the same plane pixel.
 * Channel-last `[h*w][c]` in, weights `[c][c][3][3]`, channel-last
 * `[(2h)*(2w)][c]` out; c a multiple of 4. */
int s2s_test_conv3x3_nearest2(int h, int w, int c, const float *x, const float *wgt,
                              const float *bias, float slope, float *out);

/* The head's fused conv3x3 + pixel_shuffle(2) (reference cpu::conv3x3_shuffle2,
 * src/cpu.rs:502-542): weights `[4*feat][c_in][3][3]`, output channel-last
 * `[(2h)*(2w)][feat]`. */
int s2s_test_conv3x3_shuffle2(int h, int w, int c_in, int feat, const float *x,
                              const float *wgt, const float *bias, float *out);

/* One RSTB stage of a context on host buffers (the config-1 micro-bench's op
 * sequence: the stage's Swin blocks with shifts 0/4 alternating, the 3x3 close
 * with its folded 1x1, the stage residual; reference src/cpu.rs:1516-1581):
 * `s2s_rstb_device` between an upload of `x` and a download into `out`, both
 * channel-last `[hp*wp][embed]` on an explicit (not re-padded) plane whose
 * sides are multiples of the window. Synchronous. */
int s2s_test_rstb(s2s_ctx *ctx, int stage, int hp, int wp, const float *x, float *out);

/* The device's fp32 matrix rate under pure MFMA load, measured (no reference
 * counterpart: the reference quotes no device ceiling; the roofline fractions
 * are read against it beside the spec figure): one 512-thread workgroup per CU,
 * every wave issuing 4 * iters independent v_mfma_f32_16x16x4f32 and nothing
 * else, `reps` launches timed with events after one warm-up. `*ms` is the time
 * per launch, `*tflops` 2048 FLOPs per MFMA over it, `*ghz` the shader clock
 * that rate implies at 64 fp32 matrix FLOPs per cycle per SIMD. */
int s2s_test_mfma_peak(int iters, int reps, double *ms, double *tflops, double *ghz);

#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* SWIN2SR_HIP_H */
