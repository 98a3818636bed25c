// s2s_kernels.hip - the swin2sr hot path as CDNA4 (gfx950) kernels.
//
// ACTIVATIONS ARE CHANNEL-LAST: a plane is `[hp*wp][c]`, one token per pixel,
// row-major in the plane. That one choice removes the reference's window
// gather and scatter copies (reference cuda/swin2sr.cu:99-154): every per-token
// op (the projections, LayerNorm, the MLP, the residuals) runs on the plane in
// raster order, and only window attention needs the cyclic-shift window map
// (reference src/plan.rs:72-108): the qkv GEMM reads its rows through it, the
// attention writes its output back through it.
//
// Dense contractions run on fp32 MFMA (fp32 in, fp32 accumulate):
//   - k_qkv_wattn: a Swin block's qkv projection and window attention in one
//     kernel for 6 heads of 30 (every released 180-wide checkpoint): a
//     workgroup per (window, head pair) multiplies the window's 64 gathered
//     token rows by the pair's q|k|v weights held in registers, and runs the
//     scaled-cosine attention of both heads on the products in LDS;
//   - k_bsgemm: the other token GEMMs (proj, fc1, fc2, and qkv for other head
//     shapes), weights stationary in registers, with the elementwise work
//     fused into the epilogue: bias, erf-GELU, residual, LeakyReLU, LayerNorm
//     (+ residual) over the full row, and the qkv store in the attention's
//     unit layout; batched, the transform-domain products of the Winograd
//     convolutions;
//   - k_wino_in / k_wino_out: the Winograd F(4x4,3x3) input and output
//     transforms of the body's 3x3 convolutions (bias, residual or LeakyReLU
//     in the output pass), and, with k_wino5_finish, the F(2x2,5x5) form of the
//     x4 head's composed last stage;
//   - k_gemm: 3x3 convolutions as implicit GEMMs (im2col done by the operand
//     loader) for the widths the Winograd path does not take, with the same
//     epilogues and the pixel-shuffle store of the head's octaves;
//   - k_wattn (k_attention for other head shapes): S^T = K Q^T and
//     O^T = V^T P^T per (window, head) with the softmax in registers between;
//   - k_embed: conv_first and the folded patch_embed with its LayerNorm.
// The x2 head's last octave and conv_last run composed on the VALU
// (k_up_last), and the composed heads' padded edge outputs in their own small
// kernels; the memory-bound leftovers (input padding, the standalone final
// LayerNorm, the other heads' 64->3 conv_last with the crop/denormalisation)
// are plain streaming kernels.
//
// MFMA 32x32x2 f32 lane layout (checked on the device): lane l supplies
// A[l%32][l/32] and B[l/32][l%32]; accumulator register r of lane l holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32].
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "s2s_kernels.h"

typedef float f16v __attribute__((ext_vector_type(16)));

#define MFMA32(a, b, c) __builtin_amdgcn_mfma_f32_32x32x2f32((a), (b), (c), 0, 0, 0)

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// Raw buffer access: a load whose byte offset lies past the resource's size
// returns zero and such a store is dropped, so tile edges (rows past M, columns
// past the group) need no branches, and every wave issues the same number of
// memory instructions on every path - which lets the compiler count them
// exactly in its s_waitcnt instead of draining the queue.
#define BUF_OOB 0x7ffffff0
// The size is capped below BUF_OOB, so that offset stays out of range even
// for a resource based inside a larger buffer (whose own offsets stay small).
#define BUF_MAX_BYTES 0x7fff0000u
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes < BUF_MAX_BYTES ? bytes : BUF_MAX_BYTES),
                                             0x00020000);
}
__device__ __forceinline__ float4 buf_load4(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float buf_load1(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ void buf_store1(__amdgpu_buffer_rsrc_t r, int off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, off, 0, 0);
}
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, int off, float4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), r, off, 0, 0);
}
// The same with a wave-uniform part of the offset in the instruction's SGPR
// offset (only for accesses known to be in range: the bounds check is not
// meant to be relied on for that part).
__device__ __forceinline__ float4 buf_load4s(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ void buf_store1s(__amdgpu_buffer_rsrc_t r, int voff, int soff, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, voff, soff, 0);
}
__device__ __forceinline__ void buf_store4s(__amdgpu_buffer_rsrc_t r, int voff, int soff, float4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), r, voff, soff, 0);
}
typedef unsigned v2u __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void buf_store2(__amdgpu_buffer_rsrc_t r, int off, float2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, v), r, off, 0, 0);
}


// The erf GELU, 0.5 v (1 + erf(v/sqrt2)) = v * Phi(v), evaluated through the
// complementary error function so that one branch-free formula covers every v:
// with t = |v|/sqrt2, erfc(t) = exp(-t^2) * erfcx(t), and the scaled function
// erfcx is smooth and bounded on [0, inf), so it is u times a degree-4
// polynomial in u = 1/(1 + 0.478 t) (u in (0, 1]; the substitution of
// Abramowitz & Stegun 7.1.26 with a refitted p). The five coefficients
// (halved, so the result is erfc(t)/2 directly) are a fit of erfcx on
// t in [0, 9] weighted by what an error costs the GELU (|v| exp(-t^2) / 2),
// iterated toward equal ripple against scipy.special.erfcx: 4.3e-8 absolute
// on the GELU in exact arithmetic, below float32 rounding. With q = erfc(t)/2,
// Phi(v) is 1 - q for v > 0 and q otherwise, so v Phi(v) = max(v, 0) - |v| q:
// one max and one fused multiply-add, and the negative side keeps its
// relative accuracy instead of cancelling in 1 + erf. Evaluated in float32
// the absolute error against the exact GELU is below 2.6e-7 on [-12, 12], the
// same as the erff form's rounding. One reciprocal, one exp2 and 11 other
// VALU operations, with no divergent branch (a library erff evaluates two
// polynomial branches when a wavefront holds both small and large arguments).
__device__ __forceinline__ float gelu_erf(float v) {
    // u = 1 / (1 + 0.478 |v| / sqrt2)
    const float u = __builtin_amdgcn_rcpf(fmaf(fabsf(v), 0.33799704f, 1.0f));
    float p = -0.10729234942429587f;
    p = fmaf(p, u, 0.34028711412207455f);
    p = fmaf(p, u, -0.05061983683614841f);
    p = fmaf(p, u, 0.18978627981436072f);
    p = fmaf(p, u, 0.12783743829594208f);
    // exp(-t^2) = 2^(v^2 * (-log2(e) / 2)); q = erfc(t) / 2
    const float q = u * p * __builtin_amdgcn_exp2f(v * v * -0.72134752044448170368f);
    // max(v, 0) as one v_max_f32: fmaxf (and every builtin the compiler
    // recognises as a max) adds a NaN-quieting max(v, v) in front of it (a
    // NaN in v still gives a NaN through the fma)
    float m;
    asm("v_max_f32 %0, 0, %1" : "=v"(m) : "v"(v));
    return fmaf(-fabsf(v), q, m);
}

// ---------------------------------------------------------------------------
// k_gemm: out[m][n] = epi( sum_k A[m][k] * B[n][k] + bias[n] )
//
// A rows are tokens: either a plain row-major matrix (ALOAD_ROWS) or the 3x3
// im2col view of a channel-last plane (ALOAD_IM2COL: k = tap*cin + ci, taps
// outside the plane read zero, which is the reference's zero padding).
// B is a weight in torch layout [n][k] (k contiguous).
//
// A workgroup computes an MT x NT tile with 4 wavefronts laid out WM x WN;
// each wave owns (MT/WM) x (NT/WN) as 32x32 MFMA tiles. K is walked in chunks
// of 32 staged through LDS (row stride 34 floats: 16 consecutive rows start 2
// banks apart, so each 16-lane group of a float2 operand read covers the 32
// banks once; a stride of 36 put rows r and r+8 on the same banks and measured
// 0.5-1% slower; chunks of 64 measured 8% slower), with the next chunk's
// global loads in flight while the current chunk is multiplied. (Two LDS
// buffers, one barrier per chunk instead of two, measured 12% slower: the
// doubled LDS cuts the resident workgroups from 6 to 4 per CU.)
//
// Within a chunk, lane half h (= lane/32) reads k = 4kk + 2h + {0,1} as one
// float2 and feeds the two halves to two MFMAs: the A and B operands of a lane
// half always name the same k, so the pair of MFMAs sums over all four k of
// the group. (This permutes the reduction order, not the result.)
// ---------------------------------------------------------------------------

#define KC 32
#define LDS_S (KC + 2)
#define KQ (KC / 4)       // float4s per row of a K chunk
#define KRP (256 / KQ)    // rows one pass of the 256 threads loads

template <int MT, int NT, int WM, int WN, int ALOAD, int EPI>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g) {
    static_assert(WM * WN == 4, "four wavefronts");
    // IM2COL, IM2COL5 and SUB2 share the loader: an FS x FS footprint whose
    // first tap is at (oy, ox) from the row's pixel: (-RAD, -RAD) for the
    // centred 3x3 and 5x5, (a - 1, b - 1) for SUB2's phase (a, b)
    constexpr bool SUB2 = ALOAD == ALOAD_SUB2;
    constexpr bool IC = ALOAD == ALOAD_IM2COL || ALOAD == ALOAD_IM2COL5 || SUB2;
    static_assert(IC || ALOAD == ALOAD_ROWS, "operand loader");
    constexpr int RAD = ALOAD == ALOAD_IM2COL5 ? 2 : 1;
    constexpr int FS = SUB2 ? 2 : 2 * RAD + 1;
    constexpr int WTM = MT / WM / 32;
    constexpr int WTN = NT / WN / 32;
    static_assert(WTM * WM * 32 == MT && WTN * WN * 32 == NT, "tile shape");
    constexpr int AV = MT * (KC / 4) / 256;
    constexpr int BV = NT * (KC / 4) / 256;
    static_assert(AV * 256 == MT * (KC / 4) && BV * 256 == NT * (KC / 4), "loader shape");

    __shared__ float As[MT * LDS_S];
    __shared__ float Bs[NT * LDS_S];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN;
    const int wn = wave % WN;
    // XCD-aware tile order over a 1-D grid: workgroup b runs on XCD b % 8, so
    // XCD x takes the contiguous range [x*per + min(x, rem), ...) of the tiles
    // in row-major order (row tile outer, column tiles of one row tile
    // adjacent). The tiles resident on one XCD at a time then share their A
    // rows, and an im2col tile's halo rows, in that XCD's L2; with the
    // hardware's round-robin order over a 2-D grid every column tile pass and
    // every XCD re-read the whole plane from memory.
    const int ntn = (g.N + NT - 1) / NT;
    // SUB2: the four phases' tiles one after another (each phase's tiles
    // contiguous, so an XCD's resident tiles share their rows of A)
    const int ntp = ((g.M + MT - 1) / MT) * ntn;
    const int ntiles = SUB2 ? 4 * ntp : ntp;
    const int xcd = blockIdx.x & 7;
    int lin = xcd * (ntiles >> 3) + min(xcd, ntiles & 7) + (int)(blockIdx.x >> 3);
    const int phase = SUB2 ? lin / ntp : 0;
    lin -= phase * ntp;
    const int oy = SUB2 ? (phase >> 1) - 1 : -RAD, ox = SUB2 ? (phase & 1) - 1 : -RAD;
    if (SUB2) g.B += (size_t)phase * g.N * g.ldb;
    const int m0 = (lin / ntn) * MT;
    const int n0 = (lin - (lin / ntn) * ntn) * NT;
    const int lr = lane & 31;
    const int lh = lane >> 5;

    f16v acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    float4 ra[AV], rb[BV];
    const int nk = (g.K + KC - 1) / KC;

    // Loader state. Thread t copies float4 t % KQ of a K chunk for rows
    // m0 + t / KQ + KRP*i of A and n0 + t / KQ + KRP*i of B, the same k in every
    // chunk-relative slot, so everything that depends on the row (its pixel
    // y, x) is computed once, and the k-dependent part (tap, ci and the tap's
    // pixel shift) once per chunk for all of the thread's rows. Raw buffer
    // loads: an element outside A or B (rows past M or N, k past K, a tap
    // outside the plane) reads zero from an out-of-range offset, without a
    // branch.
    // A through a resource based at the first row (pixel) this tile can
    // touch, so the offsets stay small whatever the size of the plane
    const int pb = ALOAD == ALOAD_ROWS ? m0 : max(m0 - RAD * (g.W + 1), 0);
    const int arow = ALOAD == ALOAD_ROWS ? g.lda : g.cin;
    const size_t afloats = ALOAD == ALOAD_ROWS ? (size_t)g.M * g.lda : (size_t)g.H * g.W * g.cin;
    const __amdgpu_buffer_rsrc_t ra_rs =
        buf_rsrc(g.A + (size_t)pb * arow, (afloats - (size_t)pb * arow) * 4);
    const __amdgpu_buffer_rsrc_t rb_rs = buf_rsrc(g.B, (size_t)g.N * g.ldb * 4);
    const int kq = (tid % KQ) * 4;
    int am[AV], ay[AV], ax[AV], bo[BV];
#pragma unroll
    for (int i = 0; i < AV; ++i) {
        am[i] = m0 + tid / KQ + KRP * i;
        ay[i] = ALOAD == ALOAD_ROWS ? 0 : am[i] / g.W;
        ax[i] = ALOAD == ALOAD_ROWS ? 0 : am[i] - ay[i] * g.W;
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
        const int n = n0 + tid / KQ + KRP * i;
        bo[i] = n < g.N ? (n * g.ldb + kq) * 4 : -1;
    }
    // IM2COL(5), SUB2: each of the thread's rows as a byte offset from the
    // resource base, and a mask of the taps (bit FS ty + tx for the tap at
    // (oy + ty, ox + tx)) that read inside the plane (none for rows past M);
    // a chunk then costs an add, a bit test and a select per row instead of
    // the bounds checks and a multiply
    int aro[AV];
    unsigned tmask[AV];
    if (IC) {
#pragma unroll
        for (int i = 0; i < AV; ++i) {
            aro[i] = (am[i] - pb) * g.cin * 4;
            unsigned msk = 0;
            if (am[i] < g.M) {
#pragma unroll
                for (int ty = 0; ty < FS; ++ty)
#pragma unroll
                    for (int tx = 0; tx < FS; ++tx)
                        if ((unsigned)(ay[i] + oy + ty) < (unsigned)g.H &&
                            (unsigned)(ax[i] + ox + tx) < (unsigned)g.W)
                            msk |= 1u << (FS * ty + tx);
            }
            tmask[i] = msk;
        }
    }
    // (tap, ci) of k = k0 + kq for the chunk at k0, the tap's column dx, and
    // tapoff = ((dy * W + dx) * cin + ci) * 4 for the tap at (dy, dx): the
    // byte offset of that element from its row's pixel (unchanged when ci
    // wraps into the next tap of the same kernel row; + (W - FS) * cin * 4
    // into the next row)
    int tap = 0, ci = kq, dx = ox;
    int tapoff = IC ? ((oy * g.W + ox) * g.cin + kq) * 4 : 0;
    auto norm_k = [&]() __attribute__((always_inline)) {
        if (ALOAD == ALOAD_ROWS) return;
        while (ci >= g.cin) {
            ci -= g.cin;
            ++tap;
            if (++dx >= ox + FS) {
                dx = ox;
                tapoff += (g.W - FS) * g.cin * 4;
            }
        }
    };
    norm_k();

    auto load_chunk = [&](int k0) __attribute__((always_inline)) {
        const bool kok = k0 + kq < g.K;
        // (tap < FS^2 <= 25 while k < K; bit 31 of a tap mask is never set)
        const int tsel = kok ? tap : 31;
#pragma unroll
        for (int i = 0; i < AV; ++i) {
            int off;
            if (ALOAD == ALOAD_ROWS) {
                off = (am[i] < g.M && kok) ? ((am[i] - pb) * g.lda + k0 + kq) * 4 : BUF_OOB;
            } else {
                off = ((tmask[i] >> tsel) & 1u) ? aro[i] + tapoff : BUF_OOB;
            }
            ra[i] = buf_load4(ra_rs, off);
        }
#pragma unroll
        for (int i = 0; i < BV; ++i)
            rb[i] = buf_load4(rb_rs, (bo[i] >= 0 && kok) ? bo[i] + k0 * 4 : BUF_OOB);
        // on to the next chunk's k
        ci += KC;
        tapoff += KC * 4;
        norm_k();
    };

    load_chunk(0);
    for (int kc = 0; kc < nk; ++kc) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < AV; ++i) {
            const int idx = tid + i * 256;
            *reinterpret_cast<float4 *>(&As[(idx / KQ) * LDS_S + (idx % KQ) * 4]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < BV; ++i) {
            const int idx = tid + i * 256;
            *reinterpret_cast<float4 *>(&Bs[(idx / KQ) * LDS_S + (idx % KQ) * 4]) = rb[i];
        }
        __syncthreads();
        if (kc + 1 < nk) load_chunk((kc + 1) * KC);
#pragma unroll
        for (int kk = 0; kk < KC / 4; ++kk) {
            float2 a[WTM], b[WTN];
#pragma unroll
            for (int i = 0; i < WTM; ++i)
                a[i] = *reinterpret_cast<const float2 *>(
                    &As[((wm * WTM + i) * 32 + lr) * LDS_S + kk * 4 + lh * 2]);
#pragma unroll
            for (int j = 0; j < WTN; ++j)
                b[j] = *reinterpret_cast<const float2 *>(
                    &Bs[((wn * WTN + j) * 32 + lr) * LDS_S + kk * 4 + lh * 2]);
#pragma unroll
            for (int i = 0; i < WTM; ++i)
#pragma unroll
                for (int j = 0; j < WTN; ++j) acc[i][j] = MFMA32(a[i].x, b[j].x, acc[i][j]);
#pragma unroll
            for (int i = 0; i < WTM; ++i)
#pragma unroll
                for (int j = 0; j < WTN; ++j) acc[i][j] = MFMA32(a[i].y, b[j].y, acc[i][j]);
        }
    }

    // ---- epilogue ----------------------------------------------------------
    if (EPI == EPI_LN || EPI == EPI_LN_RES) {
        // The whole row is inside this workgroup (host guarantees N <= NT and
        // one column block). Per-row partial sums: over this lane's WTN
        // columns, then across the 32 lanes of the half, then across the WN
        // waves through LDS. Single-pass statistics, as the reference's
        // channel LayerNorm computes them.
        __syncthreads();
        float *red = As;  // [WN][MT][2]
        float bias_v[WTN], lnw[WTN], lnb[WTN];
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            const int n = n0 + (wn * WTN + j) * 32 + lr;
            const bool ok = n < g.N;
            bias_v[j] = (ok && g.bias) ? g.bias[n] : 0.f;
            lnw[j] = ok ? g.ln_w[n] : 0.f;
            lnb[j] = ok ? g.ln_b[n] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < WTM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float s1 = 0.f, s2 = 0.f;
#pragma unroll
                for (int j = 0; j < WTN; ++j) {
                    const int n = n0 + (wn * WTN + j) * 32 + lr;
                    const float v = (n < g.N) ? acc[i][j][r] + bias_v[j] : 0.f;
                    acc[i][j][r] = v;
                    s1 += v;
                    s2 += v * v;
                }
#pragma unroll
                for (int o = 16; o >= 1; o >>= 1) {
                    s1 += __shfl_xor(s1, o, 64);
                    s2 += __shfl_xor(s2, o, 64);
                }
                const int rl = (wm * WTM + i) * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (lr == 0) {
                    red[(wn * MT + rl) * 2 + 0] = s1;
                    red[(wn * MT + rl) * 2 + 1] = s2;
                }
            }
        }
        __syncthreads();
        const float invn = 1.0f / (float)g.N;
#pragma unroll
        for (int i = 0; i < WTM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rl = (wm * WTM + i) * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                float s1 = 0.f, s2 = 0.f;
#pragma unroll
                for (int q = 0; q < WN; ++q) {
                    s1 += red[(q * MT + rl) * 2 + 0];
                    s2 += red[(q * MT + rl) * 2 + 1];
                }
                const float mean = s1 * invn;
                float var = s2 * invn - mean * mean;
                var = var > 0.f ? var : 0.f;
                const float rstd = 1.0f / sqrtf(var + 1e-5f);
                const int m = m0 + rl;
                if (m >= g.M) continue;
#pragma unroll
                for (int j = 0; j < WTN; ++j) {
                    const int n = n0 + (wn * WTN + j) * 32 + lr;
                    if (n >= g.N) continue;
                    float y = (acc[i][j][r] - mean) * rstd * lnw[j] + lnb[j];
                    if (EPI == EPI_LN_RES) y += g.res[(size_t)m * g.ldr + n];
                    g.out[(size_t)m * g.ldo + n] = y;
                }
            }
        }
        return;
    }

    if constexpr (EPI == EPI_SHUFFLE) {
        // pixel_shuffle(2) store: n is the permuted output channel
        // (2dy+dx)*feat + ch, m a pixel (y, x) of the H x W plane; the value
        // lands at pixel (2y + dy, 2x + dx) of the channel-last 2H x 2W plane.
        // Per column: the sub-pixel offset and channel; per row: the pixel
        // (one division per row tile, the rest by carrying x past W).
        int qoff[WTN], chn[WTN];
        float bvs[WTN];
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            const int n = n0 + (wn * WTN + j) * 32 + lr;
            const int q = n / g.feat;
            const int ch = n - q * g.feat;
            chn[j] = n < g.N ? ch : -1;
            qoff[j] = (q >> 1) * (2 * g.W) + (q & 1);
            bvs[j] = (n < g.N && g.bias) ? g.bias[n] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < WTM; ++i) {
            const int mb = m0 + (wm * WTM + i) * 32 + 4 * lh;
            const int yb = mb / g.W;
            const int xb = mb - yb * g.W;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 8 * (r >> 2) + (r & 3);
                int x = xb + off, y = yb;
                while (x >= g.W) {
                    x -= g.W;
                    ++y;
                }
                if (mb + off >= g.M) continue;
                const int pbase = (2 * y) * (2 * g.W) + 2 * x;
#pragma unroll
                for (int j = 0; j < WTN; ++j) {
                    if (chn[j] < 0) continue;
                    const size_t px = (size_t)(pbase + qoff[j]);
                    float v = acc[i][j][r] + bvs[j];
                    if (g.res) v += g.res[px * g.feat + chn[j]];
                    g.out[px * g.feat + chn[j]] = v;
                }
            }
        }
        return;
    }

#pragma unroll
    for (int j = 0; j < WTN; ++j) {
        const int n = n0 + (wn * WTN + j) * 32 + lr;
        if (n >= g.N) continue;
        const float bv = g.bias ? g.bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < WTM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + (wm * WTM + i) * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m >= g.M) continue;
                float v = acc[i][j][r] + bv;
                if (EPI == EPI_GELU) v = gelu_erf(v);
                if (EPI == EPI_LRELU) v = v < 0.f ? v * g.slope : v;
                if (EPI == EPI_RES) v += g.res[(size_t)m * g.ldr + n];
                if (EPI == EPI_SHUFFLE_FINISH) {
                    // n is torch's channel c*s^2 + dy*s + dx of the conv; the
                    // pixel_shuffle(s) output pixel (s*y+dy, s*x+dx), channel c,
                    // denormalised and cropped like the reference's finish
                    const int s2 = g.scale * g.scale;
                    const int c = n / s2;
                    const int r = n - c * s2;
                    const int dy = r / g.scale, dx = r - dy * g.scale;
                    const int y = m / g.W;
                    const int x = m - y * g.W;
                    const int oy = g.scale * y + dy, ox = g.scale * x + dx;
                    if (oy < g.oh && ox < g.ow)
                        g.out[((size_t)c * g.oh + oy) * g.ow + ox] = v / g.img_range + g.mean[c];
                } else if (SUB2) {
                    // output pixel (2y + a, 2x + b) of the 2H x 2W plane
                    const int y = m / g.W;
                    const int x = m - y * g.W;
                    const size_t px = (size_t)(2 * y + (phase >> 1)) * (2 * g.W) + 2 * x + (phase & 1);
                    g.out[px * g.ldo + n] = v;
                } else {
                    g.out[(size_t)m * g.ldo + n] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// k_bsgemm: the token GEMMs (qkv, proj, fc1, fc2) with the
// WEIGHTS STATIONARY IN REGISTERS.
//
// Every token GEMM of the network has K in {C, 2C} and a weight of at most
// 540 x 360 floats, while M is the whole plane (69,696 tokens at 256x256).
// So the weight slice a wavefront needs is loaded into VGPRs once, and the
// activations stream past it exactly once:
//   - a workgroup owns one column group of <= 64 NTW output columns (4 waves
//     x NTW MFMA tiles of 16 columns: NTW = 3, 192 columns, in general; NTW =
//     1 for a GEMM of at most 64 columns) and, for K = 2*KPW, a second set of
//     4 waves holding the other half of K (their partial sums meet in LDS);
//   - it is persistent: it walks 16-row tasks p, p+P, p+2P, ... of the plane;
//     each task's A tile (16 rows x K, contiguous in HBM) is loaded once,
//     coalesced, into LDS (double-buffered: the next task's loads are in flight
//     while this one multiplies), and read by the 4 column waves;
//   - v_mfma_f32_16x16x4f32, fp32 in and out. A step s consumes k(s, q) from
//     lane group q = lane/16: k = 16(s/4) + 4q + s%4 for the full groups of 16
//     (so a lane's A operands for 4 steps are one ds_read_b128 and its B
//     operands are 4 consecutive floats of a weight row), and k = 16G + Rq + t
//     for the R-step tail. The permutation reorders the reduction, not the
//     result.
//   - the MFMA computes the transposed tile, weights as its A operand and the
//     token rows as its B operand, so a lane ends up holding ONE output row
//     (row l%16 of the tile) and 4 consecutive columns of it per MFMA tile
//     (4(l/16) .. 4(l/16) + 3): 12 values of the row in 3 tiles. The epilogue
//     then stores float4s (float2s with K split), reads the residual and the
//     LayerNorm weights as float4s, and the row statistics need only the
//     lane's own 12 values plus one reduction over the 4 lane groups
//     (v_permlane16_swap / v_permlane32_swap) before the 4 column waves (x2
//     K halves) meet in LDS;
//   - the whole row is inside the workgroup, so LayerNorm (+ residual) is an
//     epilogue.
// Blocks are numbered (batch*ngc + ng)*P + p; with several column groups P
// is a multiple of 8, so the groups that read the same A tile run on the same
// XCD and share its L2. Odd column groups take their slots in reverse, 8 at a
// time (p -> P - 8 - 8*(p/8) + p%8, same XCD): the dispatcher gives an XCD's
// CUs one workgroup each, in block order, before any a second, so the slots
// that walk one task more than the rest (the low p) then sit on other CUs
// than the even groups' ones, and such a CU runs its last task alone instead
// of next to another one (measured: the last half round of fc1 costs half a
// round instead of a whole one).
//
// MFMA 16x16x4 f32 lane layout: lane l supplies A[l%16][k] and B[k][l%16] for
// its k (above); accumulator register r of lane l holds D[4*(l/16) + r][l%16].
// With A = weights and B = tokens, D is the transposed output tile.
// ---------------------------------------------------------------------------

typedef float f4v __attribute__((ext_vector_type(4)));
#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x4f32((a), (b), (c), 0, 0, 0)

// LDS row stride (floats) of an A tile: a multiple of 4 that is an odd
// multiple of 4 modulo 32, so the 16 rows read by one ds_read_b128 (8 lanes
// per 128-byte bank sweep) land in distinct banks.
__host__ __device__ constexpr int bs_lds_stride(int k) {
    return (k % 32 == 4 || k % 32 == 12 || k % 32 == 20 || k % 32 == 28) ? k
           : (k % 8 == 0) ? k + 4 : k + 8;
}

// Direct global -> LDS copy (gfx950 buffer_load_dwordx4 ... lds): lane l of the
// wave writes its 16 bytes at lds + 16*l, so one instruction moves a contiguous
// 1 KiB chunk without staging it in VGPRs. Out-of-range offsets write zeros.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, float *lds, int off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                             off, 0, 0, 0);
}
// ... with a wave-uniform part of the offset in the instruction's SGPR offset
// (only for copies whose whole offset is in range: the range check sees the
// per-lane part alone)
__device__ __forceinline__ void dma16s(__amdgpu_buffer_rsrc_t r, float *lds, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                             voff, soff, 0, 0);
}
// s_waitcnt vmcnt(n) alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14,
// expcnt and lgkmcnt left at their maxima).
#define WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0F70)
// A workgroup barrier for LDS traffic only: this wave's LDS writes retired
// (lgkmcnt(0)), then s_barrier, with compiler fences on both sides. Unlike
// __syncthreads() it does not drain outstanding global stores (its release
// fence does), so a task's output stores and the next task's copies stay in
// flight across it. Data copied into LDS by DMA is covered by a WAIT_VMCNT
// before the barrier.
__device__ __forceinline__ void lds_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Sum over the 16 lanes of a DPP row, every lane receiving the total: four
// DPP moves on the VALU (quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror) instead of LDS-routed lane shuffles.
#define DPP_ADD(v, ctrl)                                                                       \
    ((v) + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), \
                                                              (ctrl), 0xF, 0xF, true)))
__device__ __forceinline__ float row16_sum(float v) {
    v = DPP_ADD(v, 0xB1);
    v = DPP_ADD(v, 0x4E);
    v = DPP_ADD(v, 0x141);
    v = DPP_ADD(v, 0x140);
    return v;
}

// Two sums over the four 16-lane rows at once: lane j of row 0 (lanes 0-15)
// gets a[j] + a[j+16] + a[j+32] + a[j+48], lane j of row 1 the same sum of b
// (rows 2 and 3 repeat rows 0 and 1). v_permlane16_swap(a, b) leaves rows
// (a0, b0, a2, b2) in a and (a1, b1, a3, b3) in b, so a + b holds the pair
// sums of a in rows 0 and 2 and of b in rows 1 and 3; v_permlane32_swap(c, d)
// with d a copy of c leaves rows (c0, c1, c0, c1) in c and (c2, c3, c2, c3) in
// d (gfx950). The order is (x0 + x1) + (x2 + x3) for both. Inline assembly:
// the compiler's builtins for these swaps have added one result to itself
// instead of to the other one; the s_nop covers the VALU-write-then-permlane
// hazard.
__device__ __forceinline__ float xrow_sum2(float a, float b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    float c = a + b;
    float d = c;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(c), "+v"(d));
    return c + d;
}

// The two 32-lane halves of a wave exchanged on the VALU (gfx950
// v_permlane32_swap with both operands a copy of x): `lo` gets lanes 0-31 of x
// in both halves, `hi` lanes 32-63, so lo + hi (or max(lo, hi)) combines lane
// l with lane l ^ 32 in every lane. Inline assembly for the reason above.
__device__ __forceinline__ void halves(float x, float &lo, float &hi) {
    lo = x;
    hi = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
}
__device__ __forceinline__ float half_sum(float x) {
    float lo, hi;
    halves(x, lo, hi);
    return lo + hi;
}
__device__ __forceinline__ float half_max(float x) {
    float lo, hi;
    halves(x, lo, hi);
    return fmaxf(lo, hi);
}

template <int KPW, int KS, int RB, int EPI, int NTW>
__global__ __launch_bounds__(256 * KS, 2) void k_bsgemm(BsArgs g) {
    constexpr int NT = 256 * KS;
    constexpr int NW = 4 * KS;                 // waves
    constexpr int TR = 16 * RB;                // rows per task
    constexpr int G = KPW / 16;
    constexpr int R = (KPW % 16) / 4;
    constexpr int S = KPW / 4;
    constexpr int KT = KPW * KS;
    constexpr bool HAS_RES = EPI == EPI_RES || EPI == EPI_LN_RES;
    constexpr bool HAS_LN = EPI == EPI_LN || EPI == EPI_LN_RES;
    // EPI_QKV_WIN: task k is tokens TR*(k % TPW) .. of shifted window k / TPW
    constexpr bool WIN = EPI == EPI_QKV_WIN;
    constexpr int TPW = 64 / TR;
    // A tile: TR rows x KT floats, contiguous in HBM and in LDS; copied in
    // 1 KiB chunks, NCA per wave
    constexpr int CA = (TR * KT * 4 + 1023) / 1024;
    constexpr int NCA = (CA + NW - 1) / NW;
    constexpr int ATILE = NCA * NW * 256;      // floats reserved per buffer
    // a column group: 4 waves x NTW MFMA tiles of 16 columns
    constexpr int GW = 64 * NTW;
    // residual tile: TR rows x N (<= GW) floats
    constexpr int CR = HAS_RES ? (TR * GW * 4 + 1023) / 1024 : 0;
    constexpr int NCR = HAS_RES ? (CR + NW - 1) / NW : 0;
    constexpr int RTILE = HAS_RES ? NCR * NW * 256 : 1;
    // The MFMA computes the transposed tile (a lane holds one row, 4
    // consecutive columns per tile) except for the unit-layout store, whose
    // 8-byte-aligned rows take one dword per column: there a lane holds one
    // column and 4 rows per tile, and 16 lanes store 64 contiguous bytes.
    constexpr bool TT = !WIN;
    // buffer stores per lane per task: a float4 per tile (float2 with K
    // split), or one dword per value for the unit layout
    constexpr int NSTORE = TT ? NTW * RB : (KS == 2 ? 2 : 4) * NTW * RB;
    static_assert(KPW % 4 == 0, "K must be a multiple of 4");
    (void)NT;

    // Separate arrays, not [2][..]: the compiler then knows a copy into one
    // cannot alias reads of the other and does not wait for it.
    __shared__ __attribute__((aligned(16))) float As0[ATILE];
    __shared__ __attribute__((aligned(16))) float As1[ATILE];
    __shared__ __attribute__((aligned(16))) float Rs0[RTILE];
    __shared__ __attribute__((aligned(16))) float Rs1[RTILE];
    // K halves swap their accumulators: [sender half][column wave][rb][tile]
    // [lane][register]
    __shared__ __attribute__((aligned(16))) float ksum[KS == 2 ? 2 * 4 * RB * NTW * 4 * 64 : 1];
    // row statistics: [K half * 4 + column wave][row][sum, sum of squares]
    __shared__ float rst0[4 * KS][TR][2];
    __shared__ float rst1[4 * KS][TR][2];
    // bias, LN weight, LN bias of the group's columns
    __shared__ __attribute__((aligned(16))) float prm[3][GW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int cg = wave & 3;
    const int kq = KS == 1 ? 0 : wave >> 2;
    const int j = lane & 15;
    const int q = lane >> 4;
    // workgroup (batch bt, column group ng, slot p); a batch's A, B and out
    // start bt strides in
    const int ngc = (g.N + g.ngw - 1) / g.ngw;
    // Batched launches in an XCD-aware order: the dispatcher deals workgroup b
    // to XCD b % 8, and XCD k takes the k-th eighth of the (batch, slot)
    // pairs (a bijection for any grid size), so each XCD's L2 fetches the
    // weights of a few batches instead of all of them (Winograd GEMMs 1-3%,
    // the K = 64 one 10% faster). One batch keeps the plain order, which puts
    // the column groups of one A tile on one XCD.
    int lb = (int)blockIdx.x;
    if (g.nb > 1) {
        const int G8 = (int)(gridDim.x >> 3), k = (int)(blockIdx.x & 7);
        lb = k * G8 + min(k, (int)(gridDim.x & 7)) + (int)(blockIdx.x >> 3);
    }
    const int grp = lb / g.P;
    int p = lb - grp * g.P;
    const int bt = grp / ngc;
    const int ng = grp - bt * ngc;
    if ((ng & 1) && g.P % 8 == 0) p = g.P - 8 - (p & ~7) + (p & 7);
    if (g.nb > 1) {
        g.A += bt * g.a_bs;
        g.B += bt * g.b_bs;
        g.out += bt * g.o_bs;
    }
    const int gc0 = ng * g.ngw;
    const int gw = min(gc0 + g.ngw, g.N) - gc0;  // columns in this group
    const int kbase = kq * KPW;

    const __amdgpu_buffer_rsrc_t ra_rs = buf_rsrc(g.A, (size_t)g.M * g.lda * 4);
    // B in register order (a block of TFL floats per group, K half, column
    // wave and tile) or in rows
    constexpr int TFL = G * 256 + R * 64;
    const __amdgpu_buffer_rsrc_t rb_rs =
        buf_rsrc(g.B, g.bpk ? (size_t)ngc * KS * 4 * NTW * TFL * 4 : (size_t)g.N * g.ldb * 4);
    // EPI_QKV_WIN: a unit is 64 rows of RSU floats, HG units per window
    const int RSU = WIN ? attn_unit_stride(g.hd) : 0;
    const int HGU = WIN ? ((g.heads + 1) >> 1) * 64 * RSU : 0;
    const size_t out_floats = WIN ? (size_t)(g.M / 64) * HGU : (size_t)g.M * g.ldo;
    const bool out_wide = out_floats * 4 >= BUF_MAX_BYTES;
    const __amdgpu_buffer_rsrc_t ro_all = buf_rsrc(g.out, out_floats * 4);
    // The epilogue: with K split over two wave sets, each finishes half of the
    // accumulator registers (columns 4q + R0 .. 4q + R0 + NR - 1 of a tile, or
    // rows for the unit layout), which the K exchange leaves in registers
    // 0 .. NR - 1.
    constexpr int NR = KS == 2 ? 2 : 4;
    const int R0 = KS == 2 ? 2 * kq : 0;
    // output byte offsets: a column part per tile (out of range past the
    // group) plus a row part; their sum stays below 2^32, so an out-of-range
    // part keeps the whole offset out of range
    unsigned colo[NTW];
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
        // the first of the NR consecutive columns this lane finishes in tile t
        // (a run never straddles the group's end, a multiple of 4), or the
        // lane's column for the unit layout
        const int cl = TT ? 16 * NTW * cg + 16 * t + 4 * q + R0 : 16 * NTW * cg + 16 * t + j;
        if (WIN) {
            // column seg*C + head*hd + d -> unit (head/2), segment seg, the
            // head's half of it, d
            const int c = gc0 + cl;
            const int C = g.heads * g.hd;
            const int seg = c / C;
            const int head = (c - seg * C) / g.hd;
            const int d = c - seg * C - head * g.hd;
            colo[t] = cl < gw ? (unsigned)((head >> 1) * 64 * RSU + (2 * seg + (head & 1)) * g.hd + d) * 4u
                              : (unsigned)BUF_OOB;
        } else {
            colo[t] = cl < gw ? (unsigned)(gc0 + cl) * 4u : (unsigned)BUF_OOB;
        }
    }
    const __amdgpu_buffer_rsrc_t rr_rs = buf_rsrc(HAS_RES ? g.res : g.out,
                                                  HAS_RES ? (size_t)g.M * g.ldr * 4 : 0);

    // the weight slice (loaded after the first tiles are requested, below)
    float bw[NTW][S];
    // bias and LayerNorm parameters of the group's columns: loaded first,
    // stored to LDS once the tile copies and the weight loads are on their way
    float pv[3] = {0.f, 0.f, 0.f};
    if (tid < GW) {
        const bool ok = tid < gw;
        pv[0] = (ok && g.bias) ? g.bias[gc0 + tid] : 0.f;
        pv[1] = (HAS_LN && ok) ? g.ln_w[gc0 + tid] : 0.f;
        pv[2] = (HAS_LN && ok) ? g.ln_b[gc0 + tid] : 0.f;
    }

    const int ntask = (g.M + TR - 1) / TR;
    // EPI_QKV_WIN: float4 c*256 + 4*lane of the tile is column `col` of tile
    // row `tr` (token tr of the task): its plane offset from the task's first
    // pixel, when no token of the window wraps around the plane edge
    int avo[WIN ? NCA : 1];
    if (WIN) {
#pragma unroll
        for (int u = 0; u < NCA; ++u) {
            const int f = min((wave + NW * u) * 256 + 4 * lane, TR * KT - 4);
            const int tr = f / KT;
            const int col = f - tr * KT;
            avo[u] = (((tr >> 3) * g.wp + (tr & 7)) * g.lda + col) * 4;
        }
    }
    auto dma_a = [&](int task, float *dst) {
        if (WIN) {
            // the task's tokens, gathered from the plane (the shifted window's
            // pixels); a window in the last row or column of a shifted plane
            // wraps around its edges and takes the per-token path
            const int wi = task / TPW;
            const int tk0 = (task - wi * TPW) * TR;
            const int wh = wi / g.nww;
            const int ww = wi - wh * g.nww;
            const bool wrap = g.shift && (8 * wh + 8 >= g.hp || 8 * ww + 8 >= g.wp);
            if (!wrap) {
                const int soff = ((8 * wh + (tk0 >> 3) + g.shift) * g.wp + 8 * ww + g.shift) * g.lda * 4;
#pragma unroll
                for (int u = 0; u < NCA; ++u) dma16s(ra_rs, dst + (wave + NW * u) * 256, avo[u], soff);
            } else {
#pragma unroll
                for (int u = 0; u < NCA; ++u) {
                    const int f = min((wave + NW * u) * 256 + 4 * lane, TR * KT - 4);
                    const int tr = f / KT;
                    const int col = f - tr * KT;
                    const int tk = tk0 + tr;
                    int y = 8 * wh + (tk >> 3) + g.shift;
                    if (y >= g.hp) y -= g.hp;
                    int x = 8 * ww + (tk & 7) + g.shift;
                    if (x >= g.wp) x -= g.wp;
                    dma16(ra_rs, dst + (wave + NW * u) * 256, ((y * g.wp + x) * g.lda + col) * 4);
                }
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < NCA; ++u) {
            const int c = wave + NW * u;
            dma16(ra_rs, dst + c * 256, (task * TR * g.lda + c * 256 + 4 * lane) * 4);
        }
    };
    auto dma_r = [&](int task, float *dst) {
#pragma unroll
        for (int u = 0; u < NCR; ++u) {
            const int c = wave + NW * u;
            dma16(rr_rs, dst + c * 256, (task * TR * g.ldr + c * 256 + 4 * lane) * 4);
        }
    };

    // The epilogue of a task (normalise, activation, residual, store) runs
    // one task late, under the next task's MFMAs: `pacc` holds the previous
    // task's bias-added sums, its row statistics sit in `prst`, its residual
    // tile in `pres`.
    f4v pacc[RB][NTW];
    auto finish = [&](int task, const float (*prst)[TR][2], const float *pres)
        __attribute__((always_inline)) {
        const float invn = 1.0f / (float)gw;
        // an output past the resource limit is stored through a resource
        // based at the task's first output row, so the offsets stay small
        const int wi = task / TPW;
        const size_t tbase = out_wide ? (WIN ? (size_t)wi * HGU : (size_t)task * TR * g.ldo) : 0;
        const __amdgpu_buffer_rsrc_t ro_rs =
            out_wide ? buf_rsrc(g.out + tbase, (out_floats - tbase) * 4) : ro_all;
        const unsigned tofs = out_wide ? 0u : (unsigned)(WIN ? (size_t)wi * HGU : (size_t)task * TR * g.ldo) * 4u;
        if constexpr (!TT) {
            // unit layout (no LayerNorm, no residual): register rr of tile t is
            // row 16rb + 4q + R0 + rr, the lane's column j; one dword store per
            // value. The lane's part of the offset (row 4q + R0 of the task,
            // its column; out of range past the group) goes in the VGPR, the
            // wave-uniform row step 16rb + rr in the SGPR offset: every row of
            // a task lies in its window's unit, so the whole address stays in
            // the buffer
            const unsigned tro = tofs + (unsigned)(((task - wi * TPW) * TR + 4 * q + R0) * RSU) * 4u;
#pragma unroll
            for (int t = 0; t < NTW; ++t) {
                const int vo = (int)(tro + colo[t]);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int rr = 0; rr < NR; ++rr)
                        buf_store1s(ro_rs, vo, (rb * 16 + rr) * RSU * 4, pacc[rb][t][rr]);
            }
            return;
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int row = rb * 16 + j;
            const int m = task * TR + row;
            unsigned rowo = m < g.M ? tofs + (unsigned)row * (unsigned)g.ldo * 4u : (unsigned)BUF_OOB;
            // EPI_QKV_WIN: token tk0 + row of window task / TPW (every task is
            // whole)
            if (WIN) rowo = tofs + (unsigned)(((task - wi * TPW) * TR + row) * RSU) * 4u;
            float rstd = 1.f, mr = 0.f;
            if (HAS_LN) {
                float a1 = prst[0][row][0], a2 = prst[0][row][1];
#pragma unroll
                for (int c = 1; c < 4 * KS; ++c) {
                    a1 += prst[c][row][0];
                    a2 += prst[c][row][1];
                }
                const float mean = a1 * invn;
                float var = a2 * invn - mean * mean;
                var = var > 0.f ? var : 0.f;
                rstd = __builtin_amdgcn_rsqf(var + 1e-5f);
                mr = mean * rstd;
            }
#pragma unroll
            for (int t = 0; t < NTW; ++t) {
                // columns cl .. cl + NR - 1; columns past the group read
                // inside the tile's allocation and are dropped at the store
                const int cl = 16 * NTW * cg + 16 * t + 4 * q + R0;
                float v[NR], lw[NR], lb[NR], rs[NR];
#pragma unroll
                for (int rr = 0; rr < NR; ++rr) v[rr] = pacc[rb][t][rr];
                if (HAS_LN) {
                    if (NR == 4) {
                        const float4 w4 = *reinterpret_cast<const float4 *>(&prm[1][cl]);
                        const float4 b4 = *reinterpret_cast<const float4 *>(&prm[2][cl]);
                        lw[0] = w4.x; lw[1] = w4.y; lw[2 % NR] = w4.z; lw[3 % NR] = w4.w;
                        lb[0] = b4.x; lb[1] = b4.y; lb[2 % NR] = b4.z; lb[3 % NR] = b4.w;
                    } else {
                        const float2 w2 = *reinterpret_cast<const float2 *>(&prm[1][cl]);
                        const float2 b2 = *reinterpret_cast<const float2 *>(&prm[2][cl]);
                        lw[0] = w2.x; lw[1] = w2.y;
                        lb[0] = b2.x; lb[1] = b2.y;
                    }
                }
                if (HAS_RES) {
                    if (NR == 4) {
                        const float4 r4 = *reinterpret_cast<const float4 *>(&pres[row * g.ldr + cl]);
                        rs[0] = r4.x; rs[1] = r4.y; rs[2 % NR] = r4.z; rs[3 % NR] = r4.w;
                    } else {
                        const float2 r2 = *reinterpret_cast<const float2 *>(&pres[row * g.ldr + cl]);
                        rs[0] = r2.x; rs[1] = r2.y;
                    }
                }
#pragma unroll
                for (int rr = 0; rr < NR; ++rr) {
                    float x = v[rr];
                    if (HAS_LN) x = fmaf(fmaf(x, rstd, -mr), lw[rr], lb[rr]);
                    if (EPI == EPI_GELU) x = gelu_erf(x);
                    if (EPI == EPI_LRELU) x = x < 0.f ? x * g.slope : x;
                    if (HAS_RES) x += rs[rr];
                    v[rr] = x;
                }
                const int off = (int)(rowo + colo[t]);
                if (NR == 4 && !WIN) {
                    buf_store4(ro_rs, off, make_float4(v[0], v[1], v[2 % NR], v[3 % NR]));
                } else if (NR == 4) {
                    buf_store2(ro_rs, off, make_float2(v[0], v[1]));
                    buf_store2(ro_rs, colo[t] == (unsigned)BUF_OOB ? BUF_OOB : off + 8,
                               make_float2(v[2 % NR], v[3 % NR]));
                } else {
                    buf_store2(ro_rs, off, make_float2(v[0], v[1]));
                }
            }
        }
    };

    // One task: the next A tile streams into `nxt_buf` while this one
    // multiplies from `cur` and the previous task is finished; then this
    // task's row statistics go to `wrst` and, past the barrier, the residual
    // tile of the task after next starts streaming into `rnext`.
    auto body = [&](auto have_prev, int task, const float *cur, float *nxt_buf, int prev_task,
                    const float (*prst)[TR][2], const float *pres, float (*wrst)[TR][2],
                    float *rnext) __attribute__((always_inline)) {
        constexpr bool HP = decltype(have_prev)::value;
        const int nxt = task + g.P;
        dma_a(nxt < ntask ? nxt : task, nxt_buf);

        f4v acc[RB][NTW];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int t = 0; t < NTW; ++t) {
                // the accumulators start from the bias (the reference's CPU
                // order: bias first, then the K sum) of the lane's 4 columns;
                // with K split, one half carries it
                if (TT) {
                    const float4 b4 = (KS == 1 || kq == 0)
                                          ? *reinterpret_cast<const float4 *>(&prm[0][16 * NTW * cg + 16 * t + 4 * q])
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
                    acc[rb][t] = f4v{b4.x, b4.y, b4.z, b4.w};
                } else {
                    const float bv = (KS == 1 || kq == 0) ? prm[0][16 * NTW * cg + 16 * t + j] : 0.f;
                    acc[rb][t] = f4v{bv, bv, bv, bv};
                }
            }
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float av[RB][4];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const float4 a = *reinterpret_cast<const float4 *>(
                    &cur[(rb * 16 + j) * KT + kbase + 16 * gi + 4 * q]);
                av[rb][0] = a.x;
                av[rb][1] = a.y;
                av[rb][2] = a.z;
                av[rb][3] = a.w;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int t = 0; t < NTW; ++t)
                        acc[rb][t] = TT ? MFMA16(bw[t][4 * gi + i], av[rb][i], acc[rb][t])
                                        : MFMA16(av[rb][i], bw[t][4 * gi + i], acc[rb][t]);
            // the previous task's epilogue, issued while these MFMAs run
            if constexpr (HP) {
                if (gi == 0) finish(prev_task, prst, pres);
            }
        }
#pragma unroll
        for (int i = 0; i < R; ++i) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const float a = cur[(rb * 16 + j) * KT + kbase + 16 * G + R * q + i];
#pragma unroll
                for (int t = 0; t < NTW; ++t)
                    acc[rb][t] = TT ? MFMA16(bw[t][4 * G + i], a, acc[rb][t])
                                    : MFMA16(a, bw[t][4 * G + i], acc[rb][t]);
            }
        }

        if (KS == 2) {
            // the two K halves' partial sums meet in LDS: each half writes its
            // four registers of a tile as one float4 and reads back the pair it
            // finishes, its own and the other half's, at addresses that depend
            // on the half (indexing the registers by the half instead would
            // cost a select per register); own + other, as before the swap
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int t = 0; t < NTW; ++t)
                    *reinterpret_cast<f4v *>(&ksum[((((kq * 4 + cg) * RB + rb) * NTW + t) * 64 + lane) * 4]) =
                        acc[rb][t];
            lds_sync();
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int t = 0; t < NTW; ++t) {
                    const float2 own = *reinterpret_cast<const float2 *>(
                        &ksum[((((kq * 4 + cg) * RB + rb) * NTW + t) * 64 + lane) * 4 + R0]);
                    const float2 oth = *reinterpret_cast<const float2 *>(
                        &ksum[(((((1 - kq) * 4 + cg) * RB + rb) * NTW + t) * 64 + lane) * 4 + R0]);
                    acc[rb][t][0] = own.x + oth.x;
                    acc[rb][t][1] = own.y + oth.y;
                }
        }

        // the row statistics when a LayerNorm follows (single-pass, as the
        // reference's channel LayerNorm computes them; padding columns hold
        // exact zeros)
        if (HAS_LN) {
            // this row's sums over the lane's NR x NTW columns, then over the 4
            // lane groups (the row's other columns in this wave)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                float s1 = acc[rb][0][0], s2 = acc[rb][0][0] * acc[rb][0][0];
#pragma unroll
                for (int t = 0; t < NTW; ++t)
#pragma unroll
                    for (int rr = (t == 0 ? 1 : 0); rr < NR; ++rr) {
                        const float x = acc[rb][t][rr];
                        s1 += x;
                        s2 = fmaf(x, x, s2);
                    }
                // row 0 of the wave holds the row's sum, row 1 its sum of squares
                const float tot = xrow_sum2(s1, s2);
                if (q < 2) wrst[kq * 4 + cg][rb * 16 + j][q] = tot;
            }
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int t = 0; t < NTW; ++t) pacc[rb][t] = acc[rb][t];

        // everything this task needs next (the next A tile, and the residual
        // tile copied during the previous task) has landed; the previous
        // task's reads of `pres` are done past this barrier
        // (outstanding, oldest first: this task's residual, the next A tile,
        // the previous task's stores)
        if constexpr (HP) {
            WAIT_VMCNT(NSTORE);
        } else {
            WAIT_VMCNT(0);
        }
        lds_sync();
        if (HAS_RES) dma_r(nxt < ntask ? nxt : task, rnext);
    };

    int task = p;
    if (task < ntask) {
        dma_a(task, As0);
        if (HAS_RES) dma_r(task, Rs0);
    }
    // ---- the weight slice, once, requested after the first tiles and in the
    // order the first task's MFMAs use it: the barrier below waits for the
    // tiles alone, and each MFMA for its own weights (measured 0.5-1.6 us
    // per launch). Register bw[t][4 gi + i] of lane (j, q) is column
    // 16 NTW cg + 16 t + j of the group (the MFMA's A row l%16), k = kbase +
    // 16 gi + 4 q + i, the tail's bw[t][4 G + i] k = kbase + 16 G + R q + i;
    // B in register order (bs_pack_weights) or in rows (columns past the
    // group then out of range, reading zeros) ----
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    {
        const int ostep = g.bpk ? 1024 : 64;  // bytes between k groups
        const int tstep = g.bpk ? 256 : 4;    // bytes between tail steps
        int base[NTW], tail[NTW];
#pragma unroll
        for (int t = 0; t < NTW; ++t) {
            const int cl = 16 * NTW * cg + 16 * t + j;
            base[t] = g.bpk ? (((ng * KS + kq) * 4 + cg) * NTW + t) * TFL * 4 + lane * 16
                            : (cl < gw ? ((gc0 + cl) * g.ldb + kbase + 4 * q) * 4 : BUF_OOB);
            tail[t] = g.bpk ? G * 1024 - lane * 12 : (16 * G - 4 * q + R * q) * 4;
        }
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int t = 0; t < NTW; ++t) {
                const float4 v = buf_load4(rb_rs, base[t] + gi * ostep);
                bw[t][4 * gi + 0] = v.x;
                bw[t][4 * gi + 1] = v.y;
                bw[t][4 * gi + 2] = v.z;
                bw[t][4 * gi + 3] = v.w;
            }
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int t = 0; t < NTW; ++t) bw[t][4 * G + i] = buf_load1(rb_rs, base[t] + tail[t] + i * tstep);
    }
    if (tid < GW) {
        prm[0][tid] = pv[0];
        prm[1][tid] = pv[1];
        prm[2][tid] = pv[2];
    }
    // (vmcnt counts in issue order: all but the weight loads done = the tiles)
    static_assert(NTW * (G + R) <= 63, "the weight loads fit the vmcnt counter");
    WAIT_VMCNT(NTW * (G + R));
    lds_sync();
    if (task < ntask) {
        // task k multiplies from As[k%2], writes its statistics to rst[k%2] and
        // finds its residual in Rs[k%2]; it is finished during task k+1
        using std::false_type;
        using std::true_type;
        body(false_type{}, task, As0, As1, 0, rst1, Rs1, rst0, Rs1);
        int prev = task;
        bool last_even = true;
        task += g.P;
        while (task < ntask) {
            body(true_type{}, task, As1, As0, prev, rst0, Rs0, rst1, Rs0);
            prev = task;
            last_even = false;
            task += g.P;
            if (task >= ntask) break;
            body(true_type{}, task, As0, As1, prev, rst1, Rs1, rst0, Rs1);
            prev = task;
            last_even = true;
            task += g.P;
        }
        if (last_even) finish(prev, rst0, Rs0);
        else finish(prev, rst1, Rs1);
    }
}

// ---------------------------------------------------------------------------
// The shifted-window maps (reference src/plan.rs:72-108), shared by the
// attention kernel and the map test kernel so the tested code is the code
// that runs. Window side 8.
//
// win_pixel: window (wh, ww), token t = 8i + j reads plane pixel
//   ((8wh + i + shift) mod hp, (8ww + j + shift) mod wp)  - torch.roll(-shift).
// win_band:  the mask band of a token on the ROLLED (unwrapped) coordinate a:
//   0 if a + 8 < len, 1 if a + shift < len, else 2     - calculate_mask's slices.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int win_pixel(int wh, int ww, int t, int shift, int hp, int wp) {
    int y = wh * 8 + (t >> 3) + shift;
    int x = ww * 8 + (t & 7) + shift;
    if (y >= hp) y -= hp;  // shift < 8 <= hp: one subtraction is the modulo
    if (x >= wp) x -= wp;
    return y * wp + x;
}

__device__ __forceinline__ int win_band(int a, int len, int shift) {
    return (a + 8 < len) ? 0 : ((a + shift < len) ? 1 : 2);
}

__global__ void k_window_map(int hp, int wp, int shift, int32_t *yx, uint8_t *reg) {
    const int nww = wp / 8, nw = (hp / 8) * nww;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nw * 64) return;
    const int wi = i >> 6, t = i & 63;
    const int wh = wi / nww, ww = wi - (wi / nww) * nww;
    const int p = win_pixel(wh, ww, t, shift, hp, wp);
    yx[2 * i] = p / wp;
    yx[2 * i + 1] = p - (p / wp) * wp;
    reg[2 * i] = (uint8_t)win_band(wh * 8 + (t >> 3), hp, shift);
    reg[2 * i + 1] = (uint8_t)win_band(ww * 8 + (t & 7), wp, shift);
}

// ---------------------------------------------------------------------------
// k_attention: scaled-cosine window attention, one wavefront per (window, head).
//
// reference cpu::attention (src/cpu.rs:1244-1402) / ss_attention
// (cuda/swin2sr.cu:182-323): s = (q.k)/(|q||k|) * exp(min(ls, ln 100))
// + cpb[h][q][k] - 100*[band(q) != band(k)] (shifted blocks only); max-
// subtracted softmax over the 64 keys; out = sum_k p_k v_k. No 1/sqrt(d).
//
// The 64 tokens of window wi are read straight from the channel-last qkv
// plane [P][3c] at plane pixel index(wi, t, shift) (the roll is the modulo),
// and the output rows go back to the same pixels: the partition and its
// reverse are index math, never copies.
//
// Lane l = (r = l%32, hh = l/32). The wave holds, per 32-token tile, q and k
// head rows split in d halves: lane (r, hh) keeps d = 16*hh .. 16*hh+15 of
// token 32*tile + r (zero past head_dim), pre-scaled by exp(ls)/|q| and 1/|k|.
//   S^T = K Q^T : A = K (rows = keys), B = Q^T (cols = queries); the MFMA
//                 k-step j of lane half hh is d = 16*hh + j.
//   softmax    : a query is a lane column; its 64 keys are 2 tiles x 16
//                registers x the two lane halves -> one xor-32 exchange.
//   O^T = V^T P^T : B = P^T straight from the S^T accumulators (register
//                 4a+b of tile kt is key 32kt + 8a + 4hh + b), A = V^T loaded
//                 per key row (lane r reads d = r).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_attention(AttnArgs g) {
    const int wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wave_id >= g.nw * g.heads) return;
    const int wi = wave_id / g.heads;
    const int h = wave_id - wi * g.heads;
    const int lane = threadIdx.x & 63;
    const int r = lane & 31;
    const int hh = lane >> 5;
    const int wh = wi / g.nww;
    const int ww = wi - wh * g.nww;
    const int shift = g.shift;
    const int hd = g.head_dim;
    const size_t ld = (size_t)3 * g.c;

    auto pix = [&](int t) -> int { return win_pixel(wh, ww, t, shift, g.hp, g.wp); };

    const float ls = ATTN_LOG2E * __expf(fminf(g.logit_scale[h], 4.605170185988092f));

    // Every global read of the wave is issued here, before any arithmetic, so
    // their latencies overlap: q and k rows (lane half hh takes d = 16hh..+15,
    // as pairs when head_dim is even), and the 32 v values this lane feeds
    // the AV product (key 32kt + 8a + 4hh + b, dimension r).
    float qv[2][16], kv[2][16], vv[2][16];
    const bool even = (hd & 1) == 0;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
        const float *row = g.qkv + (size_t)pix(32 * t2 + r) * ld + h * hd;
        if (even) {
#pragma unroll
            for (int j = 0; j < 16; j += 2) {
                const int d = 16 * hh + j;
                float2 a = make_float2(0.f, 0.f), b = a;
                if (d < hd) {
                    a = *reinterpret_cast<const float2 *>(row + d);
                    b = *reinterpret_cast<const float2 *>(row + g.c + d);
                }
                qv[t2][j] = a.x;
                qv[t2][j + 1] = a.y;
                kv[t2][j] = b.x;
                kv[t2][j + 1] = b.y;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int d = 16 * hh + j;
                qv[t2][j] = d < hd ? row[d] : 0.f;
                kv[t2][j] = d < hd ? row[g.c + d] : 0.f;
            }
        }
    }
    {
        const float *vbase = g.qkv + 2 * g.c + h * hd + r;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int key = 32 * kt + 8 * (e >> 2) + 4 * hh + (e & 3);
                vv[kt][e] = (r < hd) ? vbase[(size_t)pix(key) * ld] : 0.f;
            }
    }
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
        float qs = 0.f, ks = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            qs += qv[t2][j] * qv[t2][j];
            ks += kv[t2][j] * kv[t2][j];
        }
        qs += __shfl_xor(qs, 32, 64);
        ks += __shfl_xor(ks, 32, 64);
        const float qn = fmaxf(sqrtf(qs), 1e-12f);
        const float kn = fmaxf(sqrtf(ks), 1e-12f);
        const float qsc = ls / qn;
        const float ksc = 1.0f / kn;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            qv[t2][j] *= qsc;
            kv[t2][j] *= ksc;
        }
    }

    f16v s[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e) s[a][b][e] = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) s[kt][qt] = MFMA32(kv[kt][j], qv[qt][j], s[kt][qt]);

    // Bias table [head][query][key] and the shift mask. A key's band only
    // depends on its row (t/8) and column (t%8) inside the window.
    const float *cpb = g.cpbt + (size_t)h * 64 * 64;
    int bq_y[2], bq_x[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int t = 32 * qt + r;
        bq_y[qt] = win_band(wh * 8 + (t >> 3), g.hp, shift);
        bq_x[qt] = win_band(ww * 8 + (t & 7), g.wp, shift);
    }
    float inv[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qtok = 32 * qt + r;
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int k0 = 32 * kt + 8 * a + 4 * hh;
                const float4 bias4 = *reinterpret_cast<const float4 *>(cpb + qtok * 64 + k0);
                const float bb[4] = {bias4.x, bias4.y, bias4.z, bias4.w};
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int key = k0 + b;
                    float v = s[kt][qt][4 * a + b] + bb[b];
                    if (shift) {
                        const int by = win_band(wh * 8 + (key >> 3), g.hp, shift);
                        const int bx = win_band(ww * 8 + (key & 7), g.wp, shift);
                        if (by != bq_y[qt] || bx != bq_x[qt]) v -= 100.f * ATTN_LOG2E;
                    }
                    s[kt][qt][4 * a + b] = v;
                    mx = fmaxf(mx, v);
                }
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        float sum = 0.f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float p = __builtin_amdgcn_exp2f(s[kt][qt][e] - mx);
                s[kt][qt][e] = p;
                sum += p;
            }
        sum += __shfl_xor(sum, 32, 64);
        inv[qt] = 1.0f / sum;
    }

    f16v o[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[qt][e] = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e)
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) o[qt] = MFMA32(vv[kt][e], s[kt][qt][e], o[qt]);

#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        float *orow = g.out + (size_t)pix(32 * qt + r) * g.c + h * hd;
        if (even) {
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
                const int d = 8 * (e >> 2) + 4 * hh + (e & 3);
                if (d < hd)
                    *reinterpret_cast<float2 *>(orow + d) =
                        make_float2(o[qt][e] * inv[qt], o[qt][e + 1] * inv[qt]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int d = 8 * (e >> 2) + 4 * hh + (e & 3);
                if (d < hd) orow[d] = o[qt][e] * inv[qt];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// k_wattn: the same window attention, persistent workgroups that each own one
// head pair and walk a list of windows, reading qkv in the unit layout.
//
// A unit of work is (window, head pair), and its q, k and v slices (64 tokens
// x 3 x 2*hd floats) are one contiguous unit written by the qkv GEMM: rows of
// 6*hd + 2 floats, [q | k | v | 2 padding], an odd number of float2s, so 16
// consecutive rows read by a ds_read_b64 land in distinct bank pairs. The
// unit is copied straight into LDS (buffer_load ... lds, 1 KiB per wave
// instruction, no VGPR staging). Wave w handles head 2*hg + w/2 and query
// tile w%2 (32 queries):
//   - its q row and the 64 k rows come out of LDS as MFMA operands (step j of
//     lane half hh covers d = 4(j/2) + 2hh + j%2, then d = hd-2+hh for the odd
//     tail pair), scaled in registers by exp(min(ls, ln 100))/|q| and 1/|k|;
//   - S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x2f32 with the softmax in
//     registers between them, as in k_attention; S^T starts from the bias (an
//     L2-resident table, the same for every window), loaded as soon as AV has
//     consumed the accumulators;
//   - O^T goes back into the wave's own q rows of the LDS tile (no other wave
//     reads them); after a barrier every thread reads its share of the
//     window's output slices, after another the next window's unit is copied
//     in, and the output goes out with coalesced float4 stores behind it.
// Three workgroups share a CU at hd = 30 (46 KB of LDS each), so one
// workgroup's copy overlaps the others' math. Barriers are LDS-only
// (lds_sync): the output stores stay in flight across them.
//
// Work assignment: workgroup b runs on XCD b % 8 (round-robin dispatch); its
// slot s = b / 8 on that XCD fixes the head pair hg = s % HG and a window lane
// ws = s / HG, and it takes windows xcd + 8 * (ws + nws * k), k = 0, 1, ...
// where nws is the number of window lanes per XCD. All head pairs of a window
// then run at the same time on the same XCD.
// ---------------------------------------------------------------------------
// Resident workgroups per CU: 3 by LDS (46 KB each at hd = 30) and by
// registers; at hd = 32 the tile leaves room for 3 but the registers for 2.
__host__ __device__ constexpr int wattn_per_cu(int hd) { return hd > 30 ? 2 : 3; }

template <int HD>
__global__ __launch_bounds__(256, wattn_per_cu(HD)) void k_wattn(AttnArgs g) {
    static_assert(HD % 2 == 0 && HD <= 32, "even head_dim <= 32");
    constexpr int NS = HD / 2;          // MFMA k-steps over d
    constexpr int G4 = HD / 4;          // float2 pairs of steps
    constexpr bool TAIL = (HD % 4) != 0;
    constexpr int W = 2 * HD;           // floats per segment (two heads)
    constexpr int RS = attn_unit_stride(HD);  // LDS row stride = unit row
    constexpr int UF = 64 * RS;         // floats per unit
    constexpr int NCH = (UF + 255) / 256;   // 1 KiB copies per unit
    constexpr int NCW = (NCH + 3) / 4;      // ... per wave (at most)
    __shared__ __attribute__((aligned(16))) float tile[NCH * 256];
    // The softmax denominators come out of the AV product: lane r = HD supplies
    // a column of ones (the first padding float of every tile row, set after
    // each copy has landed), so row HD of O^T is sum_k P[k][q]. Needs a spare
    // O^T row (HD < 32).
    constexpr bool MSUM = HD < 32;
    constexpr int SUM_E = 4 * (HD / 8) + (HD % 8) % 4;   // d = 8(e/4) + 4hh + e%4
    constexpr int SUM_HH = (HD % 8) / 4;

    const int HG = (g.heads + 1) >> 1;
    const int xcd = blockIdx.x & 7;
    const int slot = blockIdx.x >> 3;
    const int hg = slot % HG;
    const int ws = slot / HG;
    const int wstep = 8 * g.nws;        // window stride of one workgroup
    const int nh = min(2, g.heads - 2 * hg);
    const int v4 = nh * HD / 4;         // float4s per segment in this group
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hl = wave >> 1;
    const int qt = wave & 1;
    const int r = lane & 31;
    const int hh = lane >> 5;
    const int shift = g.shift;
    const int head = 2 * hg + hl;
    const bool active = hl < nh;
    const int C = g.c;
    const int qtok = 32 * qt + r;

    // Copy-in: chunk c = wave + 4u of the unit (floats 256c .. 256c + 255),
    // lane l moving float4 l of it; the unit's last chunk runs past it into
    // the next unit (or out of range: zeros) and lands in the tile's slack.
    // (a qkv buffer past the resource limit is reached through a resource
    // based at each unit, so the offsets stay small; the last chunk's tail
    // then reads zeros)
    const size_t qkv_bytes = (size_t)g.nw * HG * UF * 4;
    const bool qkv_wide = qkv_bytes >= BUF_MAX_BYTES;
    const __amdgpu_buffer_rsrc_t rq_all = buf_rsrc(g.qkv, qkv_bytes);
    // (the resource and base of a unit, computed ahead of the copy so that
    // the scalar arithmetic is off the path from the barrier to the copy)
    auto unit_rsrc = [&](int wi, int &base) __attribute__((always_inline)) {
        const size_t ub = (size_t)(wi * HG + hg) * UF;
        base = qkv_wide ? 0 : (int)ub * 4;
        return qkv_wide ? buf_rsrc(g.qkv + ub, UF * 4) : rq_all;
    };
    auto copy_unit = [&](__amdgpu_buffer_rsrc_t rq, int base) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NCW; ++u) {
            const int c = wave + 4 * u;
            if (u < NCW - 1 || c < NCH) dma16(rq, tile + c * 256, base + c * 1024 + 16 * lane);
        }
    };

    // Copy-out: 4 tokens per instruction, 16 lanes each (lane 16t + c takes
    // float4 c of token 16u + 4w + t); the row is scalar, the column per lane.
    const int otq = lane >> 4;
    const int oc4 = min(lane & 15, v4 - 1);
    const int otj = 4 * (wave & 1) + otq;                           // column in the window
    const float *const ldso = tile + (4 * wave + otq) * RS + 4 * oc4;  // + 16u * RS
    const int colo = (2 * hg * HD + 4 * oc4) * 4;
    const __amdgpu_buffer_rsrc_t ro = buf_rsrc(g.out, (size_t)g.hp * g.wp * C * 4);

    // the clamped logit scale (per head, the same for every window) and the
    // bias values this lane adds: query 32qt + r, keys 32kt + 8a + 4hh + b
    const float ls = active ? ATTN_LOG2E * __expf(fminf(g.logit_scale[head], 4.605170185988092f)) : 0.f;
    const float *cp = g.cpbt + ((size_t)(active ? head : 0) * 64 + qtok) * 64 + 4 * hh;

    f16v s[2];
    auto load_bias = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const float4 b4 = *reinterpret_cast<const float4 *>(cp + 32 * kt + 8 * a);
                s[kt][4 * a + 0] = b4.x;
                s[kt][4 * a + 1] = b4.y;
                s[kt][4 * a + 2] = b4.z;
                s[kt][4 * a + 3] = b4.w;
            }
    };

    // The ones column: a wave sets the padding floats that lie in chunks it
    // copied itself, after its own wait for them (another wave's copy may
    // still land up to the barrier and would overwrite an earlier write).
    const bool own_one = MSUM && ((lane * RS + 6 * HD) >> 8) % 4 == wave;

    constexpr int NST = 4;              // output stores per thread
    int wi = xcd + 8 * ws;
    if (wi < g.nw) {
        int b0;
        const __amdgpu_buffer_rsrc_t r0 = unit_rsrc(wi, b0);
        copy_unit(r0, b0);
    }
    load_bias();
    // as many dropped stores as a window's output has: the loop is then entered
    // with the same queue (copies and bias loads, then stores) as it loops back
    // with, and the wait for the copies need not drain the previous stores
    {
        const __amdgpu_buffer_rsrc_t rnull = buf_rsrc(g.out, 0);  // every offset out of range
#pragma unroll
        for (int u = 0; u < NST; ++u) buf_store4(rnull, 16 * u, make_float4(0.f, 0.f, 0.f, 0.f));
    }
    while (wi < g.nw) {
        // ---- this window's unit has landed (outstanding: at most the
        // previous window's stores) ----
        WAIT_VMCNT(NST);
        if (own_one) tile[lane * RS + 6 * HD] = 1.0f;
        lds_sync();
        const int wn = wi + wstep;
        int nbase;
        const __amdgpu_buffer_rsrc_t nrq = unit_rsrc(wn < g.nw ? wn : wi, nbase);
        const int wh = wi / g.nww;
        const int ww = wi - wh * g.nww;

        float inv = 0.f;
        f16v o;
        if (active) {
            // q operands (this lane's query, its half of d), normalised and scaled
            float qop[NS];
            {
                const float *qrow = tile + qtok * RS + hl * HD;
#pragma unroll
                for (int s2 = 0; s2 < G4; ++s2) {
                    const float2 v = *reinterpret_cast<const float2 *>(qrow + 4 * s2 + 2 * hh);
                    qop[2 * s2] = v.x;
                    qop[2 * s2 + 1] = v.y;
                }
                if (TAIL) qop[NS - 1] = qrow[4 * G4 + hh];
                float qs = 0.f;
#pragma unroll
                for (int j = 0; j < NS; ++j) qs += qop[j] * qop[j];
                qs = half_sum(qs);
                // ls / max(|q|, 1e-12) = ls * rsq(max(|q|^2, 1e-24)), one
                // hardware reciprocal square root (1 ulp) instead of the
                // correctly rounded sqrt and division sequences
                const float qsc = ls * __builtin_amdgcn_rsqf(fmaxf(qs, 1e-24f));
#pragma unroll
                for (int j = 0; j < NS; ++j) qop[j] *= qsc;
            }
            float kop[2][NS];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const float *krow = tile + (32 * kt + r) * RS + W + hl * HD;
#pragma unroll
                for (int s2 = 0; s2 < G4; ++s2) {
                    const float2 v = *reinterpret_cast<const float2 *>(krow + 4 * s2 + 2 * hh);
                    kop[kt][2 * s2] = v.x;
                    kop[kt][2 * s2 + 1] = v.y;
                }
                if (TAIL) kop[kt][NS - 1] = krow[4 * G4 + hh];
                float ks = 0.f;
#pragma unroll
                for (int j = 0; j < NS; ++j) ks += kop[kt][j] * kop[kt][j];
                ks = half_sum(ks);
                const float ksc = __builtin_amdgcn_rsqf(fmaxf(ks, 1e-24f));
#pragma unroll
                for (int j = 0; j < NS; ++j) kop[kt][j] *= ksc;
            }

#pragma unroll
            for (int j = 0; j < NS; ++j)
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) s[kt] = MFMA32(kop[kt][j], qop[j], s[kt]);

            // bias, shift mask, softmax over the query's 64 keys (2 lanes). The
            // mask bands (win_band) are all 0 except in the last window row and
            // column of a shifted block, where a token's band is 1 or 2 by
            // whether its row (column) inside the window is below 8 - shift.
            const bool ey = shift && (wh * 8 + 8 >= g.hp);
            const bool ex = shift && (ww * 8 + 8 >= g.wp);
            const bool qy = (qtok >> 3) < 8 - shift;
            const bool qx = (qtok & 7) < 8 - shift;
            if (ey || ex) {  // the same for the whole workgroup: one branch
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int krow = 4 * kt + (e >> 2);        // key >> 3
                        const int kcol = 4 * hh + (e & 3);         // key & 7
                        const bool dy = ey && ((krow < 8 - shift) != qy);
                        const bool dx = ex && ((kcol < 8 - shift) != qx);
                        if (dy || dx) s[kt][e] -= 100.f * ATTN_LOG2E;
                    }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][e]);
            mx = half_max(mx);
            float sum = 0.f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float p = __builtin_amdgcn_exp2f(s[kt][e] - mx);
                    s[kt][e] = p;
                    if (!MSUM) sum += p;
                }
            if (!MSUM) {
                sum = half_sum(sum);
                inv = 1.0f / sum;
            }

            // O^T = V^T P^T: lane r supplies V[key][d = r]. Rows d >= HD of
            // O^T are never stored, so lanes r >= HD may feed any value: they
            // read column HD-1. A key tile's 16 values are read before its
            // MFMAs, so the LDS latency is paid once per tile.
#pragma unroll
            for (int e = 0; e < 16; ++e) o[e] = 0.f;
            const float *vcol = (MSUM && r == HD) ? tile + 6 * HD : tile + 2 * W + hl * HD + min(r, HD - 1);
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                float vv[16];
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    vv[e] = vcol[(32 * kt + 8 * (e >> 2) + 4 * hh + (e & 3)) * RS];
#pragma unroll
                for (int e = 0; e < 16; ++e) o = MFMA32(vv[e], s[kt][e], o);
            }
            if (MSUM) {
                // row HD of O^T is the sum of the query's probabilities: lane
                // half SUM_HH, register SUM_E
                float lo, hi;
                halves(o[SUM_E], lo, hi);
                const float sum = SUM_HH ? hi : lo;
                inv = 1.0f / sum;
            }
        }
        load_bias();  // the accumulators are free again: the next window's bias
        if (active) {
            // into this wave's own q rows (the other head's waves read other
            // columns of them), as float2s: register pairs (e, e+1) hold d, d+1
            // with d even, and HD is even, so d < HD covers the pair
            float *orow = tile + qtok * RS + hl * HD;
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
                const int d = 8 * (e >> 2) + 4 * hh + (e & 3);
                if (d < HD)
                    *reinterpret_cast<float2 *>(orow + d) = make_float2(o[e] * inv, o[e + 1] * inv);
            }
        }
        lds_sync();
        float4 ov[NST];
#pragma unroll
        for (int u = 0; u < NST; ++u) {
            const float *src = ldso + 16 * u * RS;
            const float2 a = *reinterpret_cast<const float2 *>(src);
            const float2 b = *reinterpret_cast<const float2 *>(src + 2);
            ov[u] = make_float4(a.x, a.y, b.x, b.y);
        }
        lds_sync();  // every wave has read the tile: the next unit may land
        if (wn < g.nw) copy_unit(nrq, nbase);

        // ---- the window's output slices, coalesced ----
        {
            int x = 8 * ww + otj + shift;
            if (x >= g.wp) x -= g.wp;
            const int xo = x * C * 4 + colo;
#pragma unroll
            for (int u = 0; u < NST; ++u) {
                int y = 8 * wh + 2 * u + (wave >> 1) + shift;
                if (y >= g.hp) y -= g.hp;
                buf_store4s(ro, xo, y * g.wp * C * 4, ov[u]);
            }
        }
        wi = wn;
    }
}

// ---------------------------------------------------------------------------
// k_qkv_wattn: a block's qkv projection and window attention in one kernel,
// for 6 heads of 30 (C = 180: the released classical, real-world and
// compressed checkpoints). The unit a head pair's attention reads never
// leaves the CU: a workgroup owns one head pair and walks windows as k_wattn
// does, and per window
//   - copies the window's 64 token rows of x (the block's shifted-window
//     order, torch.roll's wrap at the plane edge, as EPI_QKV_WIN gathers them)
//     into LDS by buffer_load ... lds, as a 64 x 180 A tile;
//   - multiplies them by the pair's 180 q|k|v weight rows held in registers
//     (the weight-stationary layout of k_bsgemm: wave w owns columns
//     48w .. 48w + 47, the transposed 16x16x4 tile, 64 rows as 4 row blocks);
//   - writes the products (+ bias) over the A tile as the attention's unit,
//     [q_A | q_B | k_A | k_B | v_A | v_B | 1 | 0] per token (the weight rows
//     are stored in that order at upload), and then runs k_wattn's
//     per-window attention on it, its output stored through the plane's
//     shifted-window pixels.
// The A tile and the unit share one 48 KiB buffer, so two workgroups run per
// CU and one's copy overlaps the other's arithmetic. Workgroup b runs on XCD
// x = b % 8 as slot s = b / 8, which fixes its head pair, (x + 2s) % 3, and its
// window lane, s / 3. The whole rounds go as in k_wattn: lane ws takes
// windows x + 8 ws + 8 nws k, so the three head pairs of a window read its
// rows from the same L2. The T windows left over are dealt out item by item:
// item i = 3 j + pair of leftover window j goes to slot i / 8 of XCD i % 8,
// whose pair is the item's ((x + 2 s) % 3 = i % 3). The workgroups with one
// window more are then slots 0, 1, ... of each XCD - one per CU while there
// are at most 32 per XCD - instead of three whole lanes of one XCD, which put
// two of them on one CU (at 264 x 264, 81 leftover windows: that CU ran 6 us
// past the others).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void k_qkv_wattn(QkvAttnArgs g) {
    constexpr int HD = 30, C = 180, HG = 3;
    constexpr int NS = HD / 2;          // attention MFMA k-steps over d
    constexpr int G4 = HD / 4;          // float2 pairs of steps
    constexpr int W2 = 2 * HD;          // floats per segment (two heads)
    constexpr int RS = attn_unit_stride(HD);  // unit row stride (182)
    constexpr int GK = C / 16;          // GEMM k-groups of 16 (11), then one of 4
    constexpr int S = C / 4;            // weight registers per column tile (45)
    constexpr int BUFF = 64 * RS;       // floats: the unit, over the 64 x 180 A tile
    static_assert(64 * C <= BUFF, "the A tile fits the unit's buffer");
    constexpr int NST = 4;              // output stores per thread
    constexpr int SUM_E = 4 * (HD / 8) + (HD % 8) % 4;
    constexpr int SUM_HH = (HD % 8) / 4;
    __shared__ __attribute__((aligned(16))) float buf[BUFF];
    __shared__ __attribute__((aligned(16))) float prm[192];

    const int xcd = blockIdx.x & 7;
    const int slot = blockIdx.x >> 3;
    static_assert(HG == 3, "the pair of a slot cycles through three");
    const int hg = (xcd + 2 * slot) % HG;
    const int ws = slot / HG;
    const int wstep = 8 * g.nws;
    // window k of this workgroup: whole rounds, then at most one leftover
    // window (its item's pair is hg: (xcd + 8 slot) % 3 == hg)
    const int R0 = g.nw / wstep;
    const int T = g.nw - R0 * wstep;
    const int ti = xcd + 8 * slot;
    const int wtail = ti < 3 * T ? R0 * wstep + ti / 3 : g.nw;
    auto window_k = [&](int k) { return k < R0 ? xcd + 8 * ws + wstep * k : (k == R0 ? wtail : g.nw); };
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15;
    const int q = lane >> 4;
    const int hl = wave >> 1;
    const int qt = wave & 1;
    const int r = lane & 31;
    const int hh = lane >> 5;
    const int shift = g.shift;
    const int head = 2 * hg + hl;
    const int qtok = 32 * qt + r;

    // ---- the pair's weights, once: wave w, column tile t, MFMA A row j is
    // unit column 48w + 16t + j; step 4gi + i takes k = 16gi + 4q + i, the
    // tail step k = 176 + q. Each pair's rows are stored in k_bsgemm's
    // register order (bs_pack_weights of its 180 x 180 rows: 4 waves x 3
    // tiles, blocks of TFL floats) ----
    constexpr int TFL = GK * 256 + 64;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(g.w + (size_t)hg * 12 * TFL, (size_t)12 * TFL * 4);
    float bw[3][S];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        const int boff = (wave * 3 + t) * TFL * 4;
#pragma unroll
        for (int gi = 0; gi < GK; ++gi) {
            const float4 v = buf_load4(rw, boff + (gi * 256 + lane * 4) * 4);
            bw[t][4 * gi + 0] = v.x;
            bw[t][4 * gi + 1] = v.y;
            bw[t][4 * gi + 2] = v.z;
            bw[t][4 * gi + 3] = v.w;
        }
        bw[t][4 * GK] = buf_load1(rw, boff + (GK * 256 + lane) * 4);
    }
    if (tid < 192) prm[tid] = tid < C ? g.bias[hg * C + tid] : 0.f;

    // ---- the A tile copy: one instruction per token row (45 lanes x 16 B =
    // 720 B; the other lanes are masked off), token t of the window at LDS
    // row t, its plane pixel (torch.roll's wrap at the plane edge) as the
    // scalar offset; wave w copies tokens w, w + 4, ... ----
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(g.x, (size_t)g.hp * g.wp * C * 4);
    auto copy_a = [&](int wi) __attribute__((always_inline)) {
        const int wh = __builtin_amdgcn_readfirstlane(wi / g.nww);
        const int ww = __builtin_amdgcn_readfirstlane(wi - wh * g.nww);
        if (lane < C / 4) {
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                // (scalar: the token is the same for the whole wave)
                const int t = __builtin_amdgcn_readfirstlane(tid >> 6) + 4 * u;
                int y = 8 * wh + (t >> 3) + shift;
                if (y >= g.hp) y -= g.hp;
                int x = 8 * ww + (t & 7) + shift;
                if (x >= g.wp) x -= g.wp;
                dma16s(rx, buf + t * C, 16 * lane,
                       __builtin_amdgcn_readfirstlane((y * g.wp + x) * C * 4));
            }
        }
    };

    // ---- attention state (k_wattn's) ----
    const float ls = ATTN_LOG2E * __expf(fminf(g.logit_scale[head], 4.605170185988092f));
    const float *cp = g.cpbt + ((size_t)head * 64 + qtok) * 64 + 4 * hh;
    f16v s[2];
    auto load_bias = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const float4 b4 = *reinterpret_cast<const float4 *>(cp + 32 * kt + 8 * a);
                s[kt][4 * a + 0] = b4.x;
                s[kt][4 * a + 1] = b4.y;
                s[kt][4 * a + 2] = b4.z;
                s[kt][4 * a + 3] = b4.w;
            }
    };
    // copy-out: 4 tokens per instruction, 16 lanes each (lane 16t + c takes
    // float4 c of token 16u + 4w + t; 15 float4s a token, lane 15 repeats 14)
    const int otq = lane >> 4;
    const int oc4 = min(lane & 15, W2 / 4 - 1);
    const int otj = 4 * (wave & 1) + otq;
    const float *const ldso = buf + (4 * wave + otq) * RS + 4 * oc4;
    const int colo = (hg * W2 + 4 * oc4) * 4;
    const __amdgpu_buffer_rsrc_t ro = buf_rsrc(g.out, (size_t)g.hp * g.wp * C * 4);

    int kw = 0;
    int wi = window_k(0);
    if (wi < g.nw) copy_a(wi);
    // as many dropped stores as a window's output has: the loop is entered
    // with the same queue (the copy, then stores) as it loops back with
    {
        const __amdgpu_buffer_rsrc_t rnull = buf_rsrc(g.out, 0);
#pragma unroll
        for (int u = 0; u < NST; ++u) buf_store4(rnull, 16 * u, make_float4(0.f, 0.f, 0.f, 0.f));
    }
    while (wi < g.nw) {
        // ---- the window's A tile has landed (outstanding: at most the
        // previous window's stores) ----
        WAIT_VMCNT(NST);
        lds_sync();
        const int wn = window_k(kw + 1);
        const int wh = wi / g.nww;
        const int ww = wi - wh * g.nww;

        // ---- q|k|v of the pair: 64 tokens x 180 unit columns ----
        f4v acc[4][3];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int t = 0; t < 3; ++t) {
                const float4 b4 = *reinterpret_cast<const float4 *>(&prm[48 * wave + 16 * t + 4 * q]);
                acc[rb][t] = f4v{b4.x, b4.y, b4.z, b4.w};
            }
#pragma unroll
        for (int gi = 0; gi < GK; ++gi) {
            float av[4][4];
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const float4 a = *reinterpret_cast<const float4 *>(&buf[(16 * rb + j) * C + 16 * gi + 4 * q]);
                av[rb][0] = a.x;
                av[rb][1] = a.y;
                av[rb][2] = a.z;
                av[rb][3] = a.w;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                    for (int t = 0; t < 3; ++t) acc[rb][t] = MFMA16(bw[t][4 * gi + i], av[rb][i], acc[rb][t]);
        }
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const float a = buf[(16 * rb + j) * C + 16 * GK + q];
#pragma unroll
            for (int t = 0; t < 3; ++t) acc[rb][t] = MFMA16(bw[t][4 * GK], a, acc[rb][t]);
        }
        lds_sync();  // every wave has read the A tile
        // ---- the unit over it: lane (j, q) holds token 16rb + j, unit
        // columns 48w + 16t + 4q .. + 3; column 180 is the ones column ----
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int t = 0; t < 3; ++t) {
                // (only wave 3's last tile runs past column 179: lanes q > 0)
                const int col = 48 * wave + 16 * t + 4 * q;
                if (t < 2 || col < C) {
                    float *dst = &buf[(16 * rb + j) * RS + col];
                    *reinterpret_cast<float2 *>(dst) = make_float2(acc[rb][t][0], acc[rb][t][1]);
                    *reinterpret_cast<float2 *>(dst + 2) = make_float2(acc[rb][t][2], acc[rb][t][3]);
                }
            }
        if (tid < 64) buf[tid * RS + 6 * HD] = 1.0f;
        // S^T starts from the bias (the accumulators are free again)
        load_bias();
        lds_sync();

        // ---- the attention of head 2hg + hl, queries 32qt .. 32qt + 31 ----
        f16v o;
        float inv;
        {
            float qop[NS];
            {
                const float *qrow = buf + qtok * RS + hl * HD;
#pragma unroll
                for (int s2 = 0; s2 < G4; ++s2) {
                    const float2 v = *reinterpret_cast<const float2 *>(qrow + 4 * s2 + 2 * hh);
                    qop[2 * s2] = v.x;
                    qop[2 * s2 + 1] = v.y;
                }
                qop[NS - 1] = qrow[4 * G4 + hh];
                float qs = 0.f;
#pragma unroll
                for (int k = 0; k < NS; ++k) qs += qop[k] * qop[k];
                qs = half_sum(qs);
                const float qsc = ls * __builtin_amdgcn_rsqf(fmaxf(qs, 1e-24f));
#pragma unroll
                for (int k = 0; k < NS; ++k) qop[k] *= qsc;
            }
            // one key tile at a time (the weights hold 135 registers
            // throughout): S^T rows 32kt .. 32kt + 31
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                float kop[NS];
                const float *krow = buf + (32 * kt + r) * RS + W2 + hl * HD;
#pragma unroll
                for (int s2 = 0; s2 < G4; ++s2) {
                    const float2 v = *reinterpret_cast<const float2 *>(krow + 4 * s2 + 2 * hh);
                    kop[2 * s2] = v.x;
                    kop[2 * s2 + 1] = v.y;
                }
                kop[NS - 1] = krow[4 * G4 + hh];
                float ks = 0.f;
#pragma unroll
                for (int k = 0; k < NS; ++k) ks += kop[k] * kop[k];
                ks = half_sum(ks);
                const float ksc = __builtin_amdgcn_rsqf(fmaxf(ks, 1e-24f));
#pragma unroll
                for (int k = 0; k < NS; ++k) kop[k] *= ksc;
#pragma unroll
                for (int k = 0; k < NS; ++k) s[kt] = MFMA32(kop[k], qop[k], s[kt]);
            }
            // shift mask (last window row / column of a shifted block), softmax
            const bool ey = shift && (wh * 8 + 8 >= g.hp);
            const bool ex = shift && (ww * 8 + 8 >= g.wp);
            const bool qy = (qtok >> 3) < 8 - shift;
            const bool qx = (qtok & 7) < 8 - shift;
            if (ey || ex) {
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int krw = 4 * kt + (e >> 2);
                        const int kcl = 4 * hh + (e & 3);
                        const bool dy = ey && ((krw < 8 - shift) != qy);
                        const bool dx = ex && ((kcl < 8 - shift) != qx);
                        if (dy || dx) s[kt][e] -= 100.f * ATTN_LOG2E;
                    }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][e]);
            mx = half_max(mx);
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int e = 0; e < 16; ++e) s[kt][e] = __builtin_amdgcn_exp2f(s[kt][e] - mx);
            // O^T = V^T P^T; lane r = HD reads the ones column, so row HD of
            // O^T is the softmax denominator
#pragma unroll
            for (int e = 0; e < 16; ++e) o[e] = 0.f;
            const float *vcol = r == HD ? buf + 6 * HD : buf + 2 * W2 + hl * HD + min(r, HD - 1);
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                float vv[16];
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    vv[e] = vcol[(32 * kt + 8 * (e >> 2) + 4 * hh + (e & 3)) * RS];
#pragma unroll
                for (int e = 0; e < 16; ++e) o = MFMA32(vv[e], s[kt][e], o);
            }
            float lo, hi;
            halves(o[SUM_E], lo, hi);
            inv = 1.0f / (SUM_HH ? hi : lo);
        }
        // into this wave's own q rows (the other head's waves read other
        // columns of them)
        {
            float *orow = buf + qtok * RS + hl * HD;
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
                const int d = 8 * (e >> 2) + 4 * hh + (e & 3);
                if (d < HD)
                    *reinterpret_cast<float2 *>(orow + d) = make_float2(o[e] * inv, o[e + 1] * inv);
            }
        }
        lds_sync();
        float4 ov[NST];
#pragma unroll
        for (int u = 0; u < NST; ++u) {
            const float *src = ldso + 16 * u * RS;
            const float2 a = *reinterpret_cast<const float2 *>(src);
            const float2 b = *reinterpret_cast<const float2 *>(src + 2);
            ov[u] = make_float4(a.x, a.y, b.x, b.y);
        }
        lds_sync();  // every wave has read the buffer: the next A tile may land
        if (wn < g.nw) copy_a(wn);
        {
            int x = 8 * ww + otj + shift;
            if (x >= g.wp) x -= g.wp;
            const int xo = x * C * 4 + colo;
#pragma unroll
            for (int u = 0; u < NST; ++u) {
                int y = 8 * wh + 2 * u + (wave >> 1) + shift;
                if (y >= g.hp) y -= g.hp;
                buf_store4s(ro, xo, y * g.wp * C * 4, ov[u]);
            }
        }
        wi = wn;
        ++kw;
    }
}

// ---------------------------------------------------------------------------
// Streaming kernels.
// ---------------------------------------------------------------------------

// reference src/plan.rs:116-140 (pad_reflect) fused with the layout change:
// [3][h][w] -> channel-last [hp*wp][4] (channel 3 = 0, so the conv_first
// operand loads are float4). The mirror is of the whole plane: sy = 2h-1-y.
__global__ void k_pad_input(const float *__restrict__ in, float *__restrict__ out, int h, int w,
                            int hp, int wp) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hp * wp) return;
    const int y = i / wp, x = i - (i / wp) * wp;
    const int sy = y < h ? y : 2 * h - 1 - min(y, 2 * h - 1);
    const int sx = x < w ? x : 2 * w - 1 - min(x, 2 * w - 1);
    const size_t hw = (size_t)h * w;
    const size_t s = (size_t)sy * w + sx;
    *reinterpret_cast<float4 *>(out + (size_t)i * 4) =
        make_float4(in[s], in[hw + s], in[2 * hw + s], 0.f);
}

// Channel LayerNorm over a channel-last plane (reference cpu::channel_layer_norm,
// src/cpu.rs:1019-1073, single-pass statistics). A pixel is one 16-lane DPP
// row (float4s l, l+16, l+32, ... of its channels, all loaded before any is
// used), its sums reduced with four DPP adds; each row takes LN_PIX pixels,
// every load of all of them issued up front so that many bytes are in flight
// per thread. Optional residual: out = res + LN(x). C <= 192.
#define LN_PIX 2
__global__ __launch_bounds__(256) void k_layernorm(const float *__restrict__ x,
                                                   const float *__restrict__ w,
                                                   const float *__restrict__ b,
                                                   const float *__restrict__ res,
                                                   float *__restrict__ out, int P, int C) {
    const int l = threadIdx.x & 15;
    const int pix0 = (blockIdx.x * 16 + (threadIdx.x >> 4)) * LN_PIX;
    const int nv = C >> 2;
    float4 v[LN_PIX][3];
#pragma unroll
    for (int k = 0; k < LN_PIX; ++k)
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int q = l + 16 * i;
            const int pix = pix0 + k;
            v[k][i] = (pix < P && q < nv)
                          ? *reinterpret_cast<const float4 *>(x + (size_t)pix * C + 4 * q)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    float4 ww[3], bb[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int q = min(l + 16 * i, nv - 1);
        ww[i] = *reinterpret_cast<const float4 *>(w + 4 * q);
        bb[i] = *reinterpret_cast<const float4 *>(b + 4 * q);
    }
    const float invc = 1.0f / (float)C;
#pragma unroll
    for (int k = 0; k < LN_PIX; ++k) {
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            s1 += (v[k][i].x + v[k][i].y) + (v[k][i].z + v[k][i].w);
            s2 += (v[k][i].x * v[k][i].x + v[k][i].y * v[k][i].y) +
                  (v[k][i].z * v[k][i].z + v[k][i].w * v[k][i].w);
        }
        s1 = row16_sum(s1);
        s2 = row16_sum(s2);
        const int pix = pix0 + k;
        if (pix >= P) continue;
        const float mean = s1 * invc;
        float var = s2 * invc - mean * mean;
        var = var > 0.f ? var : 0.f;
        const float rstd = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int q = l + 16 * i;
            if (q >= nv) continue;
            float4 y;
            y.x = (v[k][i].x - mean) * rstd * ww[i].x + bb[i].x;
            y.y = (v[k][i].y - mean) * rstd * ww[i].y + bb[i].y;
            y.z = (v[k][i].z - mean) * rstd * ww[i].z + bb[i].z;
            y.w = (v[k][i].w - mean) * rstd * ww[i].w + bb[i].w;
            if (res) {
                const float4 rr = *reinterpret_cast<const float4 *>(res + (size_t)pix * C + 4 * q);
                y.x += rr.x;
                y.y += rr.y;
                y.z += rr.z;
                y.w += rr.w;
            }
            *reinterpret_cast<float4 *>(out + (size_t)pix * C + 4 * q) = y;
        }
    }
}

// conv_first (3 -> C, 3x3) and patch_embed (its 1x1 conv folded into a second
// set of conv_first weights, then LayerNorm) in one pass over the padded
// input (reference src/gpu.rs:474-478): both read the same 3x3 x 3 taps. On
// fp32 MFMA as 16x16x4 products with K = 36 (tap-major, the input's zero
// fourth channel as the fourth k of each tap): a task is 16 consecutive
// pixels; wave w holds channels 48w .. 48w + 47 of both weight sets in
// registers (A operand: lane (j, q) the weight of channel 48w + 16t + j for
// input channel q of tap s), and each lane gathers its pixel's tap-s input
// channel q as the B operand, so lane (j, q) ends with channels
// 48w + 16t + 4q .. + 3 of pixel j. Set 0 (conv_first, the body's long skip)
// is stored as it is; set 1 gets its LayerNorm: the row sums over the lane's
// values, the four lane rows (xrow_sum2) and the four waves (through LDS),
// single-pass statistics as the reference's channel LayerNorm. Channels past
// C have zero weights and bias, so they add nothing to the sums. A persistent
// grid walks the tasks; each task's gathers are issued during the one before.
// C <= 192, C % 4 == 0.
__global__ __launch_bounds__(256, 2) void k_embed(const float *__restrict__ in4,
                                                  const float *__restrict__ wts,
                                                  const float *__restrict__ b0,
                                                  const float *__restrict__ b1,
                                                  const float *__restrict__ lnw,
                                                  const float *__restrict__ lnb,
                                                  float *__restrict__ body, float *__restrict__ cur,
                                                  int H, int W, int C) {
    __shared__ float rst[2][4][16][2];  // [task parity][wave][pixel][sum, sum of squares]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int j = lane & 15;
    const int q = lane >> 4;
    const int P = H * W;
    const int ntask = (P + 15) / 16;
    // the wave's weights, biases and LayerNorm parameters (zeros past C: the
    // loads past a resource's end read zero)
    float wa[2][3][9];
    float4 bs[2][3], gw[3], gb[3];
    bool cok[3];
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(wts, (size_t)2 * 9 * 4 * C * 4);
    const __amdgpu_buffer_rsrc_t rb0 = buf_rsrc(b0, (size_t)C * 4), rb1 = buf_rsrc(b1, (size_t)C * 4);
    const __amdgpu_buffer_rsrc_t rlw = buf_rsrc(lnw, (size_t)C * 4), rlb = buf_rsrc(lnb, (size_t)C * 4);
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        const int ch = 48 * wave + 16 * t + j;  // the A row this lane supplies
        const int c4 = 48 * wave + 16 * t + 4 * q;  // the output channels it finishes
        cok[t] = c4 < C;
#pragma unroll
        for (int set = 0; set < 2; ++set)
#pragma unroll
            for (int st = 0; st < 9; ++st)
                wa[set][t][st] = buf_load1(rw, ch < C ? (((set * 9 + st) * 4 + q) * C + ch) * 4 : BUF_OOB);
        const int o4 = cok[t] ? c4 * 4 : BUF_OOB;
        bs[0][t] = buf_load4(rb0, o4);
        bs[1][t] = buf_load4(rb1, o4);
        gw[t] = buf_load4(rlw, o4);
        gb[t] = buf_load4(rlb, o4);
    }
    const __amdgpu_buffer_rsrc_t rin = buf_rsrc(in4, (size_t)P * 16);
    const __amdgpu_buffer_rsrc_t rbody = buf_rsrc(body, (size_t)P * C * 4);
    const __amdgpu_buffer_rsrc_t rcur = buf_rsrc(cur, (size_t)P * C * 4);
    // the B operand of task k: input channel q of each tap around pixel 16k + j
    // (zero outside the plane: the conv's zero padding)
    auto gather = [&](int task, float *xb) __attribute__((always_inline)) {
        // (selects, not branches: every lane issues the same nine loads)
        const int pj = 16 * task + j;
        const int y = pj / W, x = pj - y * W;
        const int base = (pj * 4 + q) * 4;
        const unsigned in_p = pj < P ? ~0u : 0u;
#pragma unroll
        for (int st = 0; st < 9; ++st) {
            const int dy = st / 3 - 1, dx = st % 3 - 1;
            const unsigned ok = in_p & ((unsigned)(y + dy) < (unsigned)H ? ~0u : 0u) &
                                ((unsigned)(x + dx) < (unsigned)W ? ~0u : 0u);
            xb[st] = buf_load1(rin, ok ? base + (dy * W + dx) * 16 : BUF_OOB);
        }
    };
    float xb[9];
    int task = blockIdx.x;
    if (task < ntask) gather(task, xb);
    for (int k = 0; task < ntask; ++k, task += gridDim.x) {
        float xn[9];
        const int nxt = task + gridDim.x;
        gather(nxt < ntask ? nxt : task, xn);
        // (the next task's loads stay ahead of this task's MFMAs)
        __builtin_amdgcn_sched_barrier(0);
        f4v acc[2][3];
#pragma unroll
        for (int set = 0; set < 2; ++set)
#pragma unroll
            for (int t = 0; t < 3; ++t) acc[set][t] = f4v{bs[set][t].x, bs[set][t].y, bs[set][t].z, bs[set][t].w};
#pragma unroll
        for (int st = 0; st < 9; ++st)
#pragma unroll
            for (int set = 0; set < 2; ++set)
#pragma unroll
                for (int t = 0; t < 3; ++t) acc[set][t] = MFMA16(wa[set][t][st], xb[st], acc[set][t]);
        const int pj = 16 * task + j;
        // conv_first: the long skip
#pragma unroll
        for (int t = 0; t < 3; ++t) {
            const int c4 = 48 * wave + 16 * t + 4 * q;
            buf_store4(rbody, (pj < P && cok[t]) ? (pj * C + c4) * 4 : BUF_OOB,
                       make_float4(acc[0][t][0], acc[0][t][1], acc[0][t][2], acc[0][t][3]));
        }
        // patch_embed's LayerNorm
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int t = 0; t < 3; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s1 += acc[1][t][r];
                s2 = fmaf(acc[1][t][r], acc[1][t][r], s2);
            }
        const float tot = xrow_sum2(s1, s2);
        if (q < 2) rst[k & 1][wave][j][q] = tot;
        lds_sync();
        float a1 = 0.f, a2 = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            a1 += rst[k & 1][w][j][0];
            a2 += rst[k & 1][w][j][1];
        }
        const float invc = 1.0f / (float)C;
        const float mean = a1 * invc;
        float var = a2 * invc - mean * mean;
        var = var > 0.f ? var : 0.f;
        const float rstd = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
        for (int t = 0; t < 3; ++t) {
            const int c4 = 48 * wave + 16 * t + 4 * q;
            float4 y;
            y.x = (acc[1][t][0] - mean) * rstd * gw[t].x + gb[t].x;
            y.y = (acc[1][t][1] - mean) * rstd * gw[t].y + gb[t].y;
            y.z = (acc[1][t][2] - mean) * rstd * gw[t].z + gb[t].z;
            y.w = (acc[1][t][3] - mean) * rstd * gw[t].w + gb[t].w;
            buf_store4(rcur, (pj < P && cok[t]) ? (pj * C + c4) * 4 : BUF_OOB, y);
        }
#pragma unroll
        for (int st = 0; st < 9; ++st) xb[st] = xn[st];
    }
}

// conv_last (feat -> 3, 3x3, zero pad) fused with the reference's host
// epilogue cpu::finish (src/cpu.rs:1925-1941): y/img_range + mean, cropped to
// the unpadded output, written planar [3][oh][ow].
//
// It reads the 64-channel plane of the last octave once (HBM) and does 27 FMAs
// per input value on the VALU (N = 3 would waste 13/16 of an MFMA tile). A
// workgroup owns a 16 x 64 output tile: lane = column, wave w = rows 4w..4w+3,
// 12 accumulators per lane. The 18 x 66 input halo moves through LDS 8
// channels at a time, double-buffered: the next chunk's loads are in flight
// while this one is multiplied. The chunk's weights (layout [tap][ci][3])
// travel with it into LDS and are read as broadcast float4s, 12 at a time (one
// tap, 4 channels), for the wave's 4 output rows.
//
// AUX: the compressed head's conv_aux (feat -> 3 on the padded plane,
// reference src/gpu.rs:703-706) with cpu::finish_aux: over the whole H x W
// plane (oh = H, ow = W), the conv's output to aux4 [H*W][4] (channel 3 zero,
// which conv_after_aux reads as zero padding) and the aux image
// v / img_range + mean to out [3][H][W].
#define CL_ROWS 16
#define CL_COLS 64
#define CL_CC 8
template <bool AUX>
__global__ __launch_bounds__(256, 2) void k_conv_last_finish(const float *__restrict__ in,
                                                             const float *__restrict__ wt,
                                                             const float *__restrict__ bias,
                                                             float *__restrict__ out, int H, int W,
                                                             int feat, int oh, int ow,
                                                             float inv_range, float m0, float m1,
                                                             float m2, float *__restrict__ aux4,
                                                             float img_range) {
    constexpr int TH = CL_ROWS + 2, TW = CL_COLS + 2;
    constexpr int Q = CL_CC / 4;                 // float4s per pixel per chunk
    constexpr int NV = TH * TW * Q;
    constexpr int NLD = (NV + 255) / 256;
    constexpr int NW4 = 9 * CL_CC * 3 / 4;       // the chunk's weights, float4s
    __shared__ float4 tile[2][NV];
    __shared__ float4 wsh[2][NW4];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int x0 = blockIdx.x * CL_COLS, y0 = blockIdx.y * CL_ROWS;
    const int nch = feat / CL_CC;

    // this thread's halo elements: (pixel p, float4 q) = divmod(tid + 256u, Q),
    // out-of-plane taps (the zero padding) and elements past the halo read zero.
    // Offsets are taken from the tile's first halo row (a resource per chunk
    // based there), so they stay small whatever the size of the plane.
    const int ybase = max(y0 - 1, 0);
    const size_t pbase = (size_t)ybase * W * feat;  // floats
    const size_t cfloats = (size_t)H * W * feat;
    int eoff[NLD];
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
        const int i = tid + 256 * u;
        const int p = i / Q, q = i - p * Q;
        const int sy = y0 - 1 + p / TW, sx = x0 - 1 + p % TW;
        const bool ok = i < NV && sy >= 0 && sy < H && sx >= 0 && sx < W;
        eoff[u] = ok ? (((sy - ybase) * W + sx) * feat + 4 * q) * 4 : BUF_OOB;
    }
    // the chunk's weights [tap][ci 0..7][3] as float4s: thread t < NW4 takes
    // float4 t (tap t / 6, then 6 float4s of 8 channels x 3)
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(wt, (size_t)9 * feat * 3 * 4);
    const int wtap = tid / (NW4 / 9), wq = tid - wtap * (NW4 / 9);
    float4 ld[NLD], lw;
    auto load = [&](int c0) __attribute__((always_inline)) {
        // chunk c0 / CL_CC: its 8 channels of every pixel
        const size_t cb = (size_t)c0 + pbase;
        const __amdgpu_buffer_rsrc_t rin = buf_rsrc(in + cb, (cfloats - cb) * 4);
#pragma unroll
        for (int u = 0; u < NLD; ++u) ld[u] = buf_load4(rin, eoff[u]);
        lw = buf_load4(rw, tid < NW4 ? ((wtap * feat + c0) * 3 + 4 * wq) * 4 : BUF_OOB);
    };
    auto stash = [&](int b) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NLD; ++u) {
            const int i = tid + 256 * u;
            if (NV % 256 == 0 || i < NV) tile[b][i] = ld[u];
        }
        if (tid < NW4) wsh[b][tid] = lw;
    };

    float acc[4][3];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        acc[rr][0] = bias[0];
        acc[rr][1] = bias[1];
        acc[rr][2] = bias[2];
    }
    load(0);
    stash(0);
    __syncthreads();
    for (int k = 0; k < nch; ++k) {
        const int c0 = k * CL_CC;
        if (k + 1 < nch) load(c0 + CL_CC);
        const float4 *t = tile[k & 1];
        const float4 *ws = wsh[k & 1];
        // one tap and 4 channels at a time: their 12 weights (three broadcast
        // LDS reads) serve the wave's 4 output rows (the tap loop is kept
        // rolled, so only one tap's operands are live)
#pragma unroll 1
        for (int tap = 0; tap < 9; ++tap)
#pragma unroll
                for (int qq = 0; qq < Q; ++qq) {
                    const int dy = tap / 3, dx = tap - 3 * (tap / 3);
                    float wk[12];
#pragma unroll
                    for (int f = 0; f < 3; ++f) {
                        const float4 w4 = ws[tap * (NW4 / 9) + 3 * qq + f];
                        wk[4 * f + 0] = w4.x;
                        wk[4 * f + 1] = w4.y;
                        wk[4 * f + 2] = w4.z;
                        wk[4 * f + 3] = w4.w;
                    }
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        const float4 v = t[((4 * wave + rr + dy) * TW + lane + dx) * Q + qq];
                        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            acc[rr][0] = fmaf(wk[3 * u + 0], vv[u], acc[rr][0]);
                            acc[rr][1] = fmaf(wk[3 * u + 1], vv[u], acc[rr][1]);
                            acc[rr][2] = fmaf(wk[3 * u + 2], vv[u], acc[rr][2]);
                        }
                    }
                }
        if (k + 1 < nch) stash((k + 1) & 1);
        __syncthreads();
    }
    const int x = x0 + lane;
    if (x >= ow) return;
    const size_t plane = (size_t)oh * ow;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const int y = y0 + 4 * wave + rr;
        if (y >= oh) break;
        const size_t o = (size_t)y * ow + x;
        if (AUX) {
            *reinterpret_cast<float4 *>(aux4 + o * 4) = make_float4(acc[rr][0], acc[rr][1], acc[rr][2], 0.f);
            out[o] = acc[rr][0] / img_range + m0;
            out[plane + o] = acc[rr][1] / img_range + m1;
            out[2 * plane + o] = acc[rr][2] / img_range + m2;
        } else {
            out[o] = acc[rr][0] * inv_range + m0;
            out[plane + o] = acc[rr][1] * inv_range + m1;
            out[2 * plane + o] = acc[rr][2] * inv_range + m2;
        }
    }
}

// The classical head's last pixel-shuffle octave and conv_last, composed
// (reference src/gpu.rs:601-623: upsample = [conv3x3 F -> 4F, PixelShuffle(2)]
// per octave, then conv_last F -> 3; nothing non-linear between the last
// octave's conv and conv_last, and the octave's plane feeds nothing else).
// Output pixel (2y + sy, 2x + sx), channel k, is a linear function of the 5 x 5
// neighbourhood of pixel (y, x) of the octave's input plane: 12 outputs (4
// sub-pixels x 3 channels, s = (2 sy + sx) * 3 + k) per input pixel, K = 25 taps
// x feat. The host composes the weights ([25][feat][12]) and biases; conv_last's
// zero padding at the top row and left column is left to k_up_last_edge (the
// bottom and right edges of the padded plane are always cropped away). Fused
// with cpu::finish (src/cpu.rs:1925-1941) as k_conv_last_finish is.
//
// VALU, as k_conv_last_finish (12 outputs would fill 3/4 of an MFMA tile): a
// workgroup owns a 4 RPW x 64 tile of input pixels, lane = column, wave w =
// rows RPW w .. RPW w + RPW - 1, 12 RPW accumulators per lane; the halo and
// the chunk's weights move through LDS 8 channels at a time, double-buffered,
// the weights read as broadcast float4s (one tap, 4 channels, 12 outputs),
// each serving the wave's RPW rows. RPW = 2 (8-row tiles) where that still
// gives two workgroups per CU, else 1 (a 256^2 input at x2 has 128 8-row
// tiles: half the CUs idle). Only pixels whose outputs survive the crop are
// computed.
#define UL_COLS 64
#define UL_CC 8
template <int RPW>
__global__ __launch_bounds__(256, 2) void k_up_last(const float *__restrict__ in,
                                                    const float *__restrict__ wt,
                                                    const float *__restrict__ bias,
                                                    float *__restrict__ out, int H, int W,
                                                    int feat, int oh, int ow, float inv_range,
                                                    float m0, float m1, float m2) {
    constexpr int UL_ROWS = 4 * RPW;
    constexpr int TH = UL_ROWS + 4, TW = UL_COLS + 4;
    constexpr int Q = UL_CC / 4;               // float4s per pixel per chunk
    constexpr int NV = TH * TW * Q;
    constexpr int NLD = (NV + 255) / 256;
    constexpr int NW4 = 25 * UL_CC * 12 / 4;   // the chunk's weights, float4s
    constexpr int NLW = (NW4 + 255) / 256;
    constexpr int TW4 = UL_CC * 12 / 4;        // ... per tap
    __shared__ float4 tile[2][NV];
    __shared__ float4 wsh[2][NW4];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int x0 = blockIdx.x * UL_COLS, y0 = blockIdx.y * UL_ROWS;
    const int nch = feat / UL_CC;

    // this thread's halo elements: (pixel p, float4 q) = divmod(tid + 256u, Q);
    // taps outside the plane (the octave conv's zero padding) and elements past
    // the halo read zero. Offsets from the tile's first halo row (a resource
    // per chunk based there), so they stay small whatever the plane's size.
    const int ybase = max(y0 - 2, 0);
    const size_t pbase = (size_t)ybase * W * feat;
    const size_t total = (size_t)H * W * feat;
    int eoff[NLD];
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
        const int i = tid + 256 * u;
        const int p = i / Q, q = i - p * Q;
        const int sy = y0 - 2 + p / TW, sx = x0 - 2 + p % TW;
        const bool ok = i < NV && sy >= 0 && sy < H && sx >= 0 && sx < W;
        eoff[u] = ok ? (((sy - ybase) * W + sx) * feat + 4 * q) * 4 : BUF_OOB;
    }
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(wt, (size_t)25 * feat * 12 * 4);
    int woff[NLW];
#pragma unroll
    for (int v = 0; v < NLW; ++v) {
        const int i = tid + 256 * v;
        const int tap = i / TW4, r = i - tap * TW4;
        woff[v] = i < NW4 ? (tap * feat * 12 + 4 * r) * 4 : BUF_OOB;
    }
    float4 ld[NLD], lw[NLW];
    auto load = [&](int c0) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rin = buf_rsrc(in + pbase + c0, (total - pbase - c0) * 4);
#pragma unroll
        for (int u = 0; u < NLD; ++u) ld[u] = buf_load4(rin, eoff[u]);
#pragma unroll
        for (int v = 0; v < NLW; ++v)
            lw[v] = buf_load4(rw, woff[v] == BUF_OOB ? BUF_OOB : woff[v] + c0 * 12 * 4);
    };
    auto stash = [&](int b) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NLD; ++u) {
            const int i = tid + 256 * u;
            if (NV % 256 == 0 || i < NV) tile[b][i] = ld[u];
        }
#pragma unroll
        for (int v = 0; v < NLW; ++v) {
            const int i = tid + 256 * v;
            if (NW4 % 256 == 0 || i < NW4) wsh[b][i] = lw[v];
        }
    };

    float acc[RPW][12];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
        for (int s = 0; s < 12; ++s) acc[rr][s] = bias[s];
    load(0);
    stash(0);
    __syncthreads();
    for (int k = 0; k < nch; ++k) {
        if (k + 1 < nch) load((k + 1) * UL_CC);
        const float4 *t = tile[k & 1];
        const float4 *ws = wsh[k & 1];
        // one tap and 4 channels at a time: their 48 weights (12 broadcast
        // float4 reads) serve the wave's RPW rows (the tap loop stays rolled,
        // so only one tap's operands are live)
#pragma unroll 1
        for (int tap = 0; tap < 25; ++tap) {
            const int ty = tap / 5, tx = tap - 5 * (tap / 5);
#pragma unroll
            for (int qq = 0; qq < Q; ++qq) {
                float wk[48];
#pragma unroll
                for (int f = 0; f < 12; ++f) {
                    const float4 w4 = ws[tap * TW4 + 12 * qq + f];
                    wk[4 * f + 0] = w4.x;
                    wk[4 * f + 1] = w4.y;
                    wk[4 * f + 2] = w4.z;
                    wk[4 * f + 3] = w4.w;
                }
#pragma unroll
                for (int rr = 0; rr < RPW; ++rr) {
                    const float4 v = t[((RPW * wave + rr + ty) * TW + lane + tx) * Q + qq];
                    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
                        for (int s = 0; s < 12; ++s)
                            acc[rr][s] = fmaf(wk[12 * cc + s], vv[cc], acc[rr][s]);
                }
            }
        }
        if (k + 1 < nch) stash((k + 1) & 1);
        __syncthreads();
    }
    // out[k][2y + sy][2x + sx] = v / img_range + mean[k]; ow and oh are even
    // (a multiple of the scale), so the two sub-pixel columns of a row go
    // out as one float2
    const int x = x0 + lane;
    if (2 * x >= ow) return;
    const size_t plane = (size_t)oh * ow;
    const float mk[3] = {m0, m1, m2};
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        const int y = y0 + RPW * wave + rr;
        if (2 * y >= oh) break;
#pragma unroll
        for (int sy = 0; sy < 2; ++sy)
#pragma unroll
            for (int kk = 0; kk < 3; ++kk) {
                const size_t o = (size_t)kk * plane + (size_t)(2 * y + sy) * ow + 2 * x;
                *reinterpret_cast<float2 *>(out + o) =
                    make_float2(acc[rr][(2 * sy) * 3 + kk] * inv_range + mk[kk],
                                acc[rr][(2 * sy + 1) * 3 + kk] * inv_range + mk[kk]);
            }
    }
}

// The outputs k_up_last gets wrong: row 0 (sub-pixel row 0 of input row 0)
// and column 0 of the output, where conv_last's zero padding drops taps that
// the interior composition includes. They are recomputed with the composition
// restricted to the in-plane taps (variant (ey, ex): conv_last's kernel row 0 /
// column 0 dropped), weights [variant][12][25][feat]: one wave per (border
// pixel, output), lane = input channel (25 taps each, coalesced), then a sum
// over the wave. Waves whose output needs no variant leave at once.
__global__ __launch_bounds__(256) void k_up_last_edge(const float *__restrict__ in,
                                                      const float *__restrict__ wv,
                                                      const float *__restrict__ bv,
                                                      float *__restrict__ out, int H, int W,
                                                      int feat, int oh, int ow, float inv_range,
                                                      float m0, float m1, float m2) {
    const int cw = ow >> 1, chh = oh >> 1;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (item >= (cw + chh - 1) * 12) return;
    const int b = item / 12, s = item - 12 * b;
    const int y = b < cw ? 0 : b - cw + 1, x = b < cw ? b : 0;
    const int kk = s % 3, sy = (s / 3) >> 1, sx = (s / 3) & 1;
    const int ey = y == 0 && sy == 0, ex = x == 0 && sx == 0;
    if (!ey && !ex) return;
    const float *w = wv + (size_t)((2 * ey + ex) * 12 + s) * 25 * feat;
    float acc = 0.f;
    for (int tap = 0; tap < 25; ++tap) {
        const int yy = y + tap / 5 - 2, xx = x + tap % 5 - 2;
        if (yy < 0 || yy >= H || xx < 0 || xx >= W) continue;
        const float *px = in + ((size_t)yy * W + xx) * feat;
        for (int ci = lane; ci < feat; ci += 64) acc = fmaf(w[tap * feat + ci], px[ci], acc);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) {
        const float mk = kk == 0 ? m0 : (kk == 1 ? m1 : m2);
        out[(size_t)kk * oh * ow + (size_t)(2 * y + sy) * ow + 2 * x + sx] =
            (acc + bv[(2 * ey + ex) * 12 + s]) * inv_range + mk;
    }
}

// The two-octave composition's outputs at input row 0 and column 0, where the
// middle plane's and conv_last's zero padding drop terms the interior
// composition includes: recomputed with the variant for the pixel (ey = row
// 0, ex = column 0), weights [4][48][25][64]. One workgroup per border pixel,
// lane = input channel, wave w computing outputs 12w .. 12w + 11: the lane's
// 25 tap values stay in registers, each output is 25 coalesced weight loads
// and 25 FMAs per lane, and the 64 partial sums of an output meet through LDS
// (thread s adds up output s) rather than through 48 chains of lane shuffles.
#define U2E_FEAT 64
__global__ __launch_bounds__(256) void k_up2_last_edge(const float *__restrict__ in,
                                                       const float *__restrict__ wv,
                                                       const float *__restrict__ bv,
                                                       float *__restrict__ out, int H, int W,
                                                       int oh, int ow, float inv_range,
                                                       float m0, float m1, float m2) {
    __shared__ float part[48][U2E_FEAT + 1];
    const int cw = (ow + 3) >> 2;
    const int wave = threadIdx.x >> 6;
    const int b = blockIdx.x;  // the launch has exactly one workgroup per border pixel
    const int lane = threadIdx.x & 63;
    const int y = b < cw ? 0 : b - cw + 1, x = b < cw ? b : 0;
    const int var = 2 * (y == 0) + (x == 0);
    float xv[25];
#pragma unroll
    for (int tap = 0; tap < 25; ++tap) {
        const int yy = y + tap / 5 - 2, xx = x + tap % 5 - 2;
        const bool ok = yy >= 0 && yy < H && xx >= 0 && xx < W;
        xv[tap] = ok ? in[((size_t)yy * W + xx) * U2E_FEAT + lane] : 0.f;
    }
#pragma unroll 2
    for (int k = 0; k < 12; ++k) {
        const int s = 12 * wave + k;
        const float *w = wv + (size_t)(var * 48 + s) * 25 * U2E_FEAT + lane;
        float acc = 0.f;
#pragma unroll
        for (int tap = 0; tap < 25; ++tap) acc = fmaf(w[tap * U2E_FEAT], xv[tap], acc);
        part[s][lane] = acc;
    }
    __syncthreads();
    if (threadIdx.x < 48) {
        const int s = threadIdx.x;
        float acc = 0.f;
        for (int l = 0; l < U2E_FEAT; ++l) acc += part[s][l];
        const int kk = s >> 4, oy = 4 * y + ((s >> 2) & 3), ox = 4 * x + (s & 3);
        if (oy < oh && ox < ow) {
            const float mk = kk == 0 ? m0 : (kk == 1 ? m1 : m2);
            out[((size_t)kk * oh + oy) * ow + ox] = (acc + bv[var * 48 + s]) * inv_range + mk;
        }
    }
}

// torch's bicubic resize, as the reference's cpu::bicubic_resize computes it
// (src/cpu.rs:875-935: a = -0.75, align_corners = False, taps clamped to the
// edge, the four horizontal products summed pairwise, then the vertical
// accumulation in tap order), on a channel-last [h*w][4] plane.
__device__ __forceinline__ float cubic_w(float t) {
    const float A = -0.75f;
    t = fabsf(t);
    if (t <= 1.0f) return ((A + 2.0f) * t - (A + 3.0f)) * t * t + 1.0f;
    if (t < 2.0f) return (((t - 5.0f) * t + 8.0f) * t - 4.0f) * A;
    return 0.0f;
}

__device__ __forceinline__ void cubic_taps(int i, int n_in, int n_out, int idx[4], float wt[4]) {
    const float src = ((float)i + 0.5f) * ((float)n_in / (float)n_out) - 0.5f;
    const float base = floorf(src);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        int id = (int)base - 1 + m;
        id = id < 0 ? 0 : (id > n_in - 1 ? n_in - 1 : id);
        idx[m] = id;
        wt[m] = cubic_w(src - (base + (float)m - 1.0f));
    }
}

__global__ void k_bicubic4(const float *__restrict__ in, float *__restrict__ out, int h, int w,
                           int oh, int ow) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= oh * ow) return;
    const int y = i / ow, x = i - (i / ow) * ow;
    int iy[4], ix[4];
    float wy[4], wx[4];
    cubic_taps(y, h, oh, iy, wy);
    cubic_taps(x, w, ow, ix, wx);
    float acc[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const float *r = in + (size_t)iy[m] * w * 4;
        const float4 p0 = *reinterpret_cast<const float4 *>(r + ix[0] * 4);
        const float4 p1 = *reinterpret_cast<const float4 *>(r + ix[1] * 4);
        const float4 p2 = *reinterpret_cast<const float4 *>(r + ix[2] * 4);
        const float4 p3 = *reinterpret_cast<const float4 *>(r + ix[3] * 4);
        const float v0[3] = {p0.x, p0.y, p0.z}, v1[3] = {p1.x, p1.y, p1.z};
        const float v2[3] = {p2.x, p2.y, p2.z}, v3[3] = {p3.x, p3.y, p3.z};
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float a0 = wx[0] * v0[c], a1 = wx[1] * v1[c];
            const float a2 = wx[2] * v2[c], a3 = wx[3] * v3[c];
            acc[c] += wy[m] * ((a0 + a1) + (a2 + a3));
        }
    }
    *reinterpret_cast<float4 *>(out + (size_t)i * 4) = make_float4(acc[0], acc[1], acc[2], 0.f);
}

// The compressed head (reference src/gpu.rs:678-730) adds its bicubic branch,
// conv_bicubic (3 -> F) of the bicubic-resized input, to the last octave's
// output just before conv_last; conv_last being linear, conv_last(octaves(x) +
// Bc) = conv_last(octaves(x)) + conv_last(Bc), and the first term is the
// classical head's composition (up2_last / up_last). The second is
// conv_last o conv_bicubic composed on the host into one 5x5 conv from the 3
// bicubic channels to the 3 outputs (the inner conv's bias folded in), with
// edge variants for output row 0 / column 0, where conv_last's zero padding
// drops taps (the bottom and right edges are cropped away). This kernel adds
// it to the finished output (divided by img_range, the denormalisation's
// scale), so neither the F-channel bicubic plane (16 P x F floats) nor the
// octaves' planes exist. A workgroup owns 4 x 64 output pixels (lane = column,
// wave = row); the 8 x 68 halo of the bicubic plane and the weights sit in
// LDS; one thread computes the 3 channels of its pixel.
#define BL_ROWS 4
#define BL_COLS 64
__global__ __launch_bounds__(256) void k_bic_last_add(const float *__restrict__ bic, int qh, int qw,
                                                      const float *__restrict__ wt,
                                                      const float *__restrict__ bias,
                                                      float *__restrict__ out, int oh, int ow,
                                                      float inv_range) {
    constexpr int HR = BL_ROWS + 4, HC = BL_COLS + 4;
    constexpr int NW = 4 * 25 * 3 * 4;
    __shared__ float4 halo[HR * HC];
    __shared__ float4 ws[NW / 4];
    __shared__ float bs[12];
    const int tid = threadIdx.x;
    const int x0 = blockIdx.x * BL_COLS, y0 = blockIdx.y * BL_ROWS;
    for (int i = tid; i < NW / 4; i += 256) ws[i] = reinterpret_cast<const float4 *>(wt)[i];
    if (tid < 12) bs[tid] = bias[tid];
    for (int i = tid; i < HR * HC; i += 256) {
        const int r = i / HC, c = i - (i / HC) * HC;
        const int y = y0 - 2 + r, x = x0 - 2 + c;
        halo[i] = (y >= 0 && y < qh && x >= 0 && x < qw)
                      ? *reinterpret_cast<const float4 *>(bic + ((size_t)y * qw + x) * 4)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    const int lx = tid & 63, ly = tid >> 6;
    const int X = x0 + lx, Y = y0 + ly;
    if (X >= ow || Y >= oh) return;
    const int v = 2 * (Y == 0) + (X == 0);
    const float4 *w = ws + v * 75;
    float a0 = bs[3 * v], a1 = bs[3 * v + 1], a2 = bs[3 * v + 2];
#pragma unroll 5
    for (int t = 0; t < 25; ++t) {
        const float4 p = halo[(ly + t / 5) * HC + lx + t % 5];
        const float4 w0 = w[3 * t], w1 = w[3 * t + 1], w2 = w[3 * t + 2];
        a0 = fmaf(w0.z, p.z, fmaf(w0.y, p.y, fmaf(w0.x, p.x, a0)));
        a1 = fmaf(w1.z, p.z, fmaf(w1.y, p.y, fmaf(w1.x, p.x, a1)));
        a2 = fmaf(w2.z, p.z, fmaf(w2.y, p.y, fmaf(w2.x, p.x, a2)));
    }
    const size_t plane = (size_t)oh * ow, o = (size_t)Y * ow + X;
    out[o] += a0 * inv_range;
    out[plane + o] += a1 * inv_range;
    out[2 * plane + o] += a2 * inv_range;
}

hipError_t launch_bic_last_add(const float *bic, int qh, int qw, const float *w, const float *bias,
                               float *out, int oh, int ow, float img_range, hipStream_t st) {
    // every output pixel's 5x5 footprint reads the bicubic plane at offsets
    // -2..2 (zero outside); the output is the crop of that plane's grid
    if (oh < 1 || ow < 1 || oh > qh || ow > qw) return hipErrorInvalidValue;
    const dim3 grid((ow + BL_COLS - 1) / BL_COLS, (oh + BL_ROWS - 1) / BL_ROWS);
    hipLaunchKernelGGL(k_bic_last_add, grid, dim3(256), 0, st, bic, qh, qw, w, bias, out, oh, ow,
                       1.0f / img_range);
    return hipGetLastError();
}

// The continuous position bias table (reference tools/convert.py:141-167 and
// network_swin2sr.py:101-136), built on the device from the cpb_mlp weights:
// one workgroup per relative offset (dy, dx) in [-(win-1), win-1]^2, the
// 512-wide hidden layer in LDS, then one lane per head. tab is [heads][side^2].
__global__ __launch_bounds__(256) void k_cpb_mlp(const float *__restrict__ w0,
                                                 const float *__restrict__ b0,
                                                 const float *__restrict__ w2,
                                                 float *__restrict__ tab, int win, int heads) {
    __shared__ float hid[512];
    const int side = 2 * win - 1;
    const int e = blockIdx.x;
    const int a = e / side, b = e - (e / side) * side;
    float co[2] = {(float)(a - (win - 1)), (float)(b - (win - 1))};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        float v = co[k] / (float)(win - 1);
        v = v * 8.0f;
        const float sg = v > 0.f ? 1.f : (v < 0.f ? -1.f : 0.f);
        co[k] = sg * log2f(fabsf(v) + 1.0f) / 3.0f;
    }
    for (int j = threadIdx.x; j < 512; j += blockDim.x) {
        const float hv = co[0] * w0[j * 2] + co[1] * w0[j * 2 + 1] + b0[j];
        hid[j] = hv > 0.f ? hv : 0.f;
    }
    __syncthreads();
    // one wavefront per head: lanes stride the hidden layer, then reduce
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int hh = wave; hh < heads; hh += 4) {
        float acc = 0.f;
        for (int j = lane; j < 512; j += 64) acc += hid[j] * w2[hh * 512 + j];
        for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (lane == 0) tab[hh * side * side + e] = acc;
    }
}

// Gather the table to [heads][n][n] (query-major, key contiguous) through the
// relative position index (yq-yk+win-1)*(2win-1) + (xq-xk+win-1), with 16*sigmoid.
__global__ void k_cpb_gather(const float *__restrict__ tab, float *__restrict__ cpbt, int win,
                             int heads) {
    const int n = win * win, side = 2 * win - 1;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= heads * n * n) return;
    const int h = i / (n * n), qk = i - h * n * n;
    const int q = qk / n, k = qk - (qk / n) * n;
    const int idx = ((q / win) - (k / win) + win - 1) * side + ((q % win) - (k % win) + win - 1);
    const float v = tab[h * side * side + idx];
    cpbt[i] = ATTN_LOG2E * (16.0f / (1.0f + expf(-v)));  // (base-2 softmax)
}

// ---------------------------------------------------------------------------
// Host-side launchers (one per kernel family; the GEMM shapes are chosen here).
// ---------------------------------------------------------------------------

template <int MT, int NT, int WM, int WN, int ALOAD, int EPI>
static hipError_t run_gemm_t(const GemmArgs &g, hipStream_t st) {
    // one workgroup per tile (per phase for SUB2), in k_gemm's XCD-aware order
    const dim3 grid((unsigned)(((g.M + MT - 1) / MT) * ((g.N + NT - 1) / NT) * (ALOAD == ALOAD_SUB2 ? 4 : 1)));
    hipLaunchKernelGGL((k_gemm<MT, NT, WM, WN, ALOAD, EPI>), grid, dim3(256), 0, st, g);
    return hipGetLastError();
}

// The tile shapes (rows MT x columns NT, wavefront grid WM x WN).
static const int kVariants[GEMM_NVARIANTS][4] = {
    {128, 192, 2, 2}, {64, 192, 2, 2}, {128, 64, 4, 1}, {128, 128, 2, 2}, {64, 128, 2, 2},
    {64, 64, 2, 2}};

template <int MT, int NT, int WM, int WN, int ALOAD>
static hipError_t run_gemm_e(const GemmArgs &g, int epi, hipStream_t st) {
    if constexpr (ALOAD == ALOAD_SUB2) {
        // the real-world head's conv_up1 / conv_up2 (+ LeakyReLU 0.2)
        if (epi == EPI_LRELU) return run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_LRELU>(g, st);
        return hipErrorInvalidValue;
    } else if constexpr (ALOAD == ALOAD_IM2COL5) {
        // the classical head's last two octaves and conv_last, composed
        if (epi == EPI_SHUFFLE_FINISH) return run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_SHUFFLE_FINISH>(g, st);
        return hipErrorInvalidValue;
    } else {
        switch (epi) {
        case EPI_STORE: return run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_STORE>(g, st);
        case EPI_GELU: return run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_GELU>(g, st);
        case EPI_RES: return run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_RES>(g, st);
        case EPI_LRELU: return run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_LRELU>(g, st);
        case EPI_SHUFFLE: return run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_SHUFFLE>(g, st);
        case EPI_SHUFFLE_FINISH:
            return run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_SHUFFLE_FINISH>(g, st);
        case EPI_LN:
        case EPI_LN_RES:
            // the whole row must be one column tile
            if constexpr (NT >= 192) {
                return epi == EPI_LN ? run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_LN>(g, st)
                                     : run_gemm_t<MT, NT, WM, WN, ALOAD, EPI_LN_RES>(g, st);
            }
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
        }
    }
}

template <int MT, int NT, int WM, int WN>
static hipError_t run_gemm_v(const GemmArgs &g, int aload, int epi, hipStream_t st) {
    switch (aload) {
    case ALOAD_ROWS: return run_gemm_e<MT, NT, WM, WN, ALOAD_ROWS>(g, epi, st);
    case ALOAD_IM2COL: return run_gemm_e<MT, NT, WM, WN, ALOAD_IM2COL>(g, epi, st);
    case ALOAD_IM2COL5: return run_gemm_e<MT, NT, WM, WN, ALOAD_IM2COL5>(g, epi, st);
    case ALOAD_SUB2: return run_gemm_e<MT, NT, WM, WN, ALOAD_SUB2>(g, epi, st);
    default: return hipErrorInvalidValue;
    }
}

const char *gemm_kernel_name(const GemmArgs &g, int aload, int epi) {
    (void)g;
    static const char *names[5][9] = {
        {"gemm_rows_store", "gemm_rows_gelu", "gemm_rows_res", "gemm_rows_ln", "gemm_rows_ln_res",
         "gemm_rows_lrelu", "gemm_rows_shuffle", "gemm_rows_shuffle_finish", "gemm_rows_qkv_win"},
        {"conv3x3_store", "conv3x3_gelu", "conv3x3_res", "conv3x3_ln", "conv3x3_ln_res",
         "conv3x3_lrelu", "conv3x3_shuffle", "conv3x3_shuffle_finish", "conv3x3_qkv_win"},
        {"gemm_unknown", "gemm_unknown", "gemm_unknown", "gemm_unknown", "gemm_unknown",
         "gemm_unknown", "gemm_unknown", "gemm_unknown", "gemm_unknown"},  // (2: no loader)
        {"conv5x5_store", "conv5x5_gelu", "conv5x5_res", "conv5x5_ln", "conv5x5_ln_res",
         "conv5x5_lrelu", "conv5x5_shuffle", "conv5x5_shuffle_finish", "conv5x5_qkv_win"},
        {"conv_sub2_store", "conv_sub2_gelu", "conv_sub2_res", "conv_sub2_ln", "conv_sub2_ln_res",
         "conv_sub2_lrelu", "conv_sub2_shuffle", "conv_sub2_shuffle_finish", "conv_sub2_qkv_win"}};
    if (aload < 0 || aload > 4 || epi < 0 || epi > 8) return "gemm_unknown";
    return names[aload][epi];
}

// Tile choice by shape, from a sweep of every variant on the forward's own
// shapes on MI355X. These GEMMs are short in K (180-1620) and latency-bound:
// the 64x64 tile (one 32x32 MFMA tile per wavefront, ~18 KB of LDS) keeps the
// most wavefronts resident and wins everywhere except the shuffle octaves
// (K = 576, 256 columns: 64x128). LayerNorm epilogues need the whole row in
// one 192-wide column tile; 64 rows keeps that grid from ending in a nearly
// empty round of workgroups.
int gemm_pick(const GemmArgs &g, int aload, int epi) {
    (void)aload;
    (void)g;
    if (epi == EPI_LN || epi == EPI_LN_RES) return 1;
    if (epi == EPI_SHUFFLE) return 4;
    return 5;
}

void gemm_variant_grid(const GemmArgs &g, int variant, unsigned *gx, unsigned *gy) {
    const int MT = kVariants[variant][0], NT = kVariants[variant][1];
    *gx = (unsigned)((g.M + MT - 1) / MT);
    *gy = (unsigned)((g.N + NT - 1) / NT);
}

void gemm_grid(const GemmArgs &g, int aload, int epi, unsigned *gx, unsigned *gy) {
    gemm_variant_grid(g, gemm_pick(g, aload, epi), gx, gy);
    if (aload == ALOAD_SUB2) *gx *= 4;  // the four phases
}

hipError_t launch_gemm_variant(const GemmArgs &g, int aload, int epi, int variant,
                               hipStream_t st) {
    if ((epi == EPI_LN || epi == EPI_LN_RES) && g.N > 192) return hipErrorInvalidValue;
    switch (variant) {
    case 1: return run_gemm_v<64, 192, 2, 2>(g, aload, epi, st);
    case 4: return run_gemm_v<64, 128, 2, 2>(g, aload, epi, st);
    case 5: return run_gemm_v<64, 64, 2, 2>(g, aload, epi, st);
    default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// k_mfma_peak: the fp32 matrix peak of the device, measured. Every wave issues
// `iters` rounds of four independent v_mfma_f32_16x16x4f32 (four accumulator
// tiles, so no MFMA waits for the previous one's result) and nothing else in
// its loop; one 512-thread workgroup per CU puts two such waves on each SIMD.
// The result (one float per thread) is stored so the work is not removed.
// Timed by the caller: 2048 FLOPs per MFMA over the elapsed time is the
// matrix rate the chip sustains under pure MFMA load, and at 64 FLOPs per
// cycle per SIMD the implied shader clock.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(512) void k_mfma_peak(float *out, int iters, float x) {
    f4v a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0, a3 = a0;
    const float p = x + (float)threadIdx.x, q = x - (float)threadIdx.x;
    for (int i = 0; i < iters; ++i) {
        a0 = MFMA16(p, q, a0);
        a1 = MFMA16(q, p, a1);
        a2 = MFMA16(p, p, a2);
        a3 = MFMA16(q, q, a3);
    }
    out[(size_t)blockIdx.x * 512 + threadIdx.x] = a0[0] + a1[1] + a2[2] + a3[3];
}

hipError_t launch_mfma_peak(float *out, int blocks, int iters, hipStream_t st) {
    if (blocks <= 0 || iters <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_mfma_peak, dim3((unsigned)blocks), dim3(512), 0, st, out, iters, 1.0f);
    return hipGetLastError();
}

// ---- k_bsgemm dispatch ----------------------------------------------------

static int cu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            v <= 0) {
            (void)hipGetLastError();
            v = 256;
        }
        n = v;
    }
    return n;
}

// K per wave and K halves of a weight shape k_bsgemm is built for (the embed
// widths of the released checkpoints: 180 and 60, with K = 2*KPW split over
// two wave sets, and the x4 head's 64-feature Winograd products), with its
// tiles per wave
static bool bs_weight_shape(int N, int K, int epi, int *kpw, int *ks, int *ntw) {
    *ntw = (N <= 64 && (epi == EPI_STORE || epi == EPI_LN_RES)) ? 1 : 3;
    if (N <= 0) return false;
    if (K == 180 || K == 60) {
        *kpw = K;
        *ks = 1;
    } else if (K == 64 && epi == EPI_STORE && *ntw == 1) {
        *kpw = 64;
        *ks = 1;
    } else if (K == 360 || K == 120) {
        *kpw = K / 2;
        *ks = 2;
    } else {
        return false;
    }
    return true;
}

// k_bsgemm takes a row GEMM whose K per wave is one it is built for (the
// embed widths of the released checkpoints: 180 and 60, with K = 2*KPW split
// over two wave sets).
// MFMA tiles of 16 columns per wave: one for a GEMM of at most 64 columns
// whose epilogue has a narrow build (a column group of 64), else three (192).
static int bs_ntw(const GemmArgs &g, int epi) {
    int kpw, ks, ntw;
    (void)bs_weight_shape(g.N, g.K, epi, &kpw, &ks, &ntw);
    return ntw;
}

size_t bs_weight_floats(int N, int K, int epi) {
    int kpw, ks, ntw;
    if (!bs_weight_shape(N, K, epi, &kpw, &ks, &ntw)) return 0;
    const int ng = (N + 64 * ntw - 1) / (64 * ntw);
    return (size_t)ng * ks * 4 * ntw * ((kpw / 16) * 256 + ((kpw % 16) / 4) * 64);
}

void bs_pack_weights(const float *w, int ldb, int N, int K, int epi, float *dst) {
    int kpw, ks, ntw;
    if (!bs_weight_shape(N, K, epi, &kpw, &ks, &ntw)) return;
    const int ng = (N + 64 * ntw - 1) / (64 * ntw);
    const int ngw = (N + ng - 1) / ng;  // columns per group, as the launch sets it
    const int G = kpw / 16, R = (kpw % 16) / 4, tfl = G * 256 + R * 64;
    size_t blk = 0;
    for (int gp = 0; gp < ng; ++gp) {
        const int gw = std::min(ngw, N - gp * ngw);
        for (int kq = 0; kq < ks; ++kq)
            for (int cg = 0; cg < 4; ++cg)
                for (int t = 0; t < ntw; ++t, ++blk) {
                    float *b = dst + blk * tfl;
                    for (int lane = 0; lane < 64; ++lane) {
                        const int j = lane & 15, q = lane >> 4;
                        const int cl = 16 * ntw * cg + 16 * t + j;
                        const float *row = cl < gw ? w + (size_t)(gp * ngw + cl) * ldb + kq * kpw : nullptr;
                        for (int gi = 0; gi < G; ++gi)
                            for (int i = 0; i < 4; ++i)
                                b[gi * 256 + lane * 4 + i] = row ? row[16 * gi + 4 * q + i] : 0.f;
                        for (int i = 0; i < R; ++i)
                            b[G * 256 + i * 64 + lane] = row ? row[16 * G + R * q + i] : 0.f;
                    }
                }
    }
}

static bool bs_eligible(const GemmArgs &g, int aload, int epi, int *kpw, int *ks) {
    if (aload != ALOAD_ROWS || epi == EPI_SHUFFLE) return false;
    if (g.nb > 1 && (epi != EPI_STORE || g.bias)) return false;
    if (g.lda % 4 || g.ldb % 4 || g.M <= 0 || g.N <= 0) return false;
    // each lane stores runs of 4 (2) consecutive columns as one float4 (float2):
    // the column groups and the row strides are multiples of 4
    {
        const int gw = 64 * bs_ntw(g, epi);
        const int ng = (g.N + gw - 1) / gw;
        if (g.N % 4 || ((g.N + ng - 1) / ng) % 4 || g.ldo % 4) return false;
        if ((epi == EPI_RES || epi == EPI_LN_RES) && g.ldr % 4) return false;
    }
    // the A tile (and the residual tile) are copied as contiguous blocks
    if (g.lda != g.K) return false;
    if ((epi == EPI_RES || epi == EPI_LN_RES) && (g.ldr != g.N || g.N > 192)) return false;
    int ntw;
    if (!bs_weight_shape(g.N, g.K, epi, kpw, ks, &ntw)) return false;
    if ((epi == EPI_LN || epi == EPI_LN_RES) && g.N > 192) return false;
    if (epi == EPI_QKV_WIN) {
        // whole windows of the plane, three head-major column blocks
        if (g.H <= 0 || g.W <= 0 || g.H % 8 || g.W % 8 || g.M != g.H * g.W) return false;
        if (g.heads <= 0 || g.hd <= 0 || g.N != 3 * g.heads * g.hd) return false;
        if (g.shift < 0 || g.shift >= 8) return false;
    }
    return true;
}

template <int KPW, int KS, int RB, int EPI, int NTW>
static hipError_t run_bs(const GemmArgs &g, hipStream_t st, bool launch, dim3 *grid_out) {
    static int per_cu = 0;  // resident workgroups per CU, from the occupancy query
    if (!per_cu) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_bsgemm<KPW, KS, RB, EPI, NTW>, 256 * KS,
                                                         0) != hipSuccess ||
            nb < 1) {
            (void)hipGetLastError();
            nb = 1;
        }
        per_cu = nb;
    }
    const int ng = (g.N + 64 * NTW - 1) / (64 * NTW);
    const int ngw = (g.N + ng - 1) / ng;
    const int nb = std::max(g.nb, 1);
    const int ntask = (g.M + 16 * RB - 1) / (16 * RB);
    int P = per_cu * cu_count() / (ng * nb);
    // several column groups: P a multiple of 8 puts the groups of one A tile
    // on one XCD (shared L2); batches share nothing, and fill the machine
    if (P >= 8 && ng > 1) P -= P % 8;
    P = std::max(1, std::min(P, ntask));
    const dim3 grid((unsigned)(P * ng * nb));
    if (grid_out) *grid_out = grid;
    if (!launch) return hipSuccess;
    BsArgs a{};
    a.A = g.A;
    a.lda = g.lda;
    a.B = g.B;
    a.ldb = g.ldb;
    a.bias = g.bias;
    a.out = g.out;
    a.ldo = g.ldo;
    a.res = g.res;
    a.ldr = g.ldr;
    a.ln_w = g.ln_w;
    a.ln_b = g.ln_b;
    a.slope = g.slope;
    a.M = g.M;
    a.N = g.N;
    a.K = g.K;
    a.P = P;
    a.ngw = ngw;
    a.hp = g.H;
    a.wp = g.W;
    a.nww = g.W / 8;
    a.shift = g.shift;
    a.heads = g.heads;
    a.hd = g.hd;
    a.nb = nb;
    a.a_bs = g.a_bstride;
    a.b_bs = g.b_bstride;
    a.o_bs = g.o_bstride;
    a.bpk = g.b_packed;
    hipLaunchKernelGGL((k_bsgemm<KPW, KS, RB, EPI, NTW>), grid, dim3(256 * KS), 0, st, a);
    return hipGetLastError();
}

template <int KPW, int KS, int RB>
static hipError_t run_bs_e(const GemmArgs &g, int epi, hipStream_t st, bool launch, dim3 *grid) {
    if (bs_ntw(g, epi) == 1) {
        // the narrow builds
        if (epi == EPI_STORE) return run_bs<KPW, KS, RB, EPI_STORE, 1>(g, st, launch, grid);
        if constexpr (RB == 1) {
            if (epi == EPI_LN_RES) return run_bs<KPW, KS, RB, EPI_LN_RES, 1>(g, st, launch, grid);
        }
        return hipErrorInvalidValue;
    }
    switch (epi) {
    case EPI_STORE: return run_bs<KPW, KS, RB, EPI_STORE, 3>(g, st, launch, grid);
    case EPI_GELU: return run_bs<KPW, KS, RB, EPI_GELU, 3>(g, st, launch, grid);
    case EPI_LRELU: return run_bs<KPW, KS, RB, EPI_LRELU, 3>(g, st, launch, grid);
    case EPI_QKV_WIN: return run_bs<KPW, KS, RB, EPI_QKV_WIN, 3>(g, st, launch, grid);
    default: break;
    }
    // residual and LayerNorm epilogues run with 16-row tasks only (bs_rb)
    if constexpr (RB == 1) {
        switch (epi) {
        case EPI_RES: return run_bs<KPW, KS, RB, EPI_RES, 3>(g, st, launch, grid);
        case EPI_LN: return run_bs<KPW, KS, RB, EPI_LN, 3>(g, st, launch, grid);
        case EPI_LN_RES: return run_bs<KPW, KS, RB, EPI_LN_RES, 3>(g, st, launch, grid);
        default: break;
        }
    }
    return hipErrorInvalidValue;
}

// 32-row tasks (two row blocks) when several column groups or batches share
// the machine and the epilogue keeps no per-row state; else 16-row tasks.
// The GELU GEMM (fc1) and the Winograd batches at K = C keep 16-row tasks:
// their planes rarely divide into whole rounds of 32-row tasks, and the last,
// partial round of the finer tasks is half as long (measured at 264 x 264:
// fc1 2.8%, the body convs' 36-batch GEMM 4.5% faster). The x4 head's K = 64
// batches, bound by HBM rather than MFMA, keep 32-row tasks (16-row: 7% slower).
static int bs_rb(const GemmArgs &g, int ks, int epi) {
    const int gw = 64 * bs_ntw(g, epi);
    const int ng = (g.N + gw - 1) / gw * std::max(g.nb, 1);  // column groups x batches
    const bool simple = epi == EPI_STORE || epi == EPI_LRELU || epi == EPI_QKV_WIN;
    (void)ks;
    if (g.nb > 1 && g.K != 64) return 1;
    return (ng >= 2 && simple) ? 2 : 1;
}

static hipError_t run_bs_any(const GemmArgs &g, int kpw, int ks, int epi, hipStream_t st,
                             bool launch, dim3 *grid) {
    const int rb = bs_rb(g, ks, epi);
    if (kpw == 64) {
        if (ks != 1 || epi != EPI_STORE || bs_ntw(g, epi) != 1) return hipErrorInvalidValue;
        return rb == 1 ? run_bs<64, 1, 1, EPI_STORE, 1>(g, st, launch, grid)
                       : run_bs<64, 1, 2, EPI_STORE, 1>(g, st, launch, grid);
    }
    if (kpw == 180) {
        if (ks == 1) return rb == 1 ? run_bs_e<180, 1, 1>(g, epi, st, launch, grid)
                                    : run_bs_e<180, 1, 2>(g, epi, st, launch, grid);
        return rb == 1 ? run_bs_e<180, 2, 1>(g, epi, st, launch, grid)
                       : run_bs_e<180, 2, 2>(g, epi, st, launch, grid);
    }
    if (ks == 1) return rb == 1 ? run_bs_e<60, 1, 1>(g, epi, st, launch, grid)
                                : run_bs_e<60, 1, 2>(g, epi, st, launch, grid);
    return rb == 1 ? run_bs_e<60, 2, 1>(g, epi, st, launch, grid)
                   : run_bs_e<60, 2, 2>(g, epi, st, launch, grid);
}

bool bs_takes(const GemmArgs &g, int aload, int epi) {
    int kpw, ks;
    return bs_eligible(g, aload, epi, &kpw, &ks);
}

void gemm_geometry(const GemmArgs &g, int aload, int epi, dim3 *grid, dim3 *block) {
    int kpw, ks;
    if (bs_eligible(g, aload, epi, &kpw, &ks)) {
        (void)run_bs_any(g, kpw, ks, epi, 0, false, grid);
        *block = dim3(256 * ks);
        return;
    }
    unsigned gx, gy;
    gemm_grid(g, aload, epi, &gx, &gy);
    *grid = dim3(gx * gy);  // the 1-D launch of k_gemm's tiles
    *block = dim3(256);
}

hipError_t launch_gemm(const GemmArgs &g, int aload, int epi, hipStream_t st) {
    int kpw, ks;
    if (bs_eligible(g, aload, epi, &kpw, &ks)) return run_bs_any(g, kpw, ks, epi, st, true, nullptr);
    // a packed B only k_bsgemm reads; batches and the unit-layout store only
    // k_bsgemm runs
    if (g.b_packed || g.nb > 1 || epi == EPI_QKV_WIN) return hipErrorInvalidValue;
    return launch_gemm_variant(g, aload, epi, gemm_pick(g, aload, epi), st);
}

// k_wattn takes every even head_dim it is built for whose head-pair output
// slices are float4-aligned (all released checkpoints: 30 and 10) from the
// unit layout; k_attention the rest, from the plane layout.
bool attn_unit_eligible(int heads, int hd, int c) {
    if (hd != 2 && hd != 10 && hd != 30 && hd != 32) return false;
    if (heads <= 0 || c != heads * hd || c % 4) return false;
    if ((heads & 1) && hd % 4) return false;  // a lone last head's slice must be float4s
    return true;
}

bool qkv_unit_layout(int heads, int hd, int c) {
    // the qkv GEMM (K = c) must run on k_bsgemm, which writes the layout
    return attn_unit_eligible(heads, hd, c) && (c == 180 || c == 60 || c == 360 || c == 120);
}

static bool wattn_eligible(const AttnArgs &g) {
    return g.unit && attn_unit_eligible(g.heads, g.head_dim, g.c);
}

// k_wattn's persistent grid: 8 XCDs x HG head pairs x nws window lanes, about
// as many workgroups as the CUs hold at once, never more lanes than an XCD has
// windows.
static int wattn_lanes(const AttnArgs &g) {
    const int HG = (g.heads + 1) / 2;
    const int per_xcd = (g.nw + 7) / 8;
    return std::max(1, std::min(per_xcd, wattn_per_cu(g.head_dim) * cu_count() / (8 * HG)));
}

hipError_t launch_attention(const AttnArgs &g0, hipStream_t st, unsigned *grid_out) {
    if (wattn_eligible(g0)) {
        AttnArgs g = g0;
        g.nws = wattn_lanes(g);
        const unsigned grid = (unsigned)(8 * ((g.heads + 1) / 2) * g.nws);
        if (grid_out) *grid_out = grid;
        switch (g.head_dim) {
        case 2: hipLaunchKernelGGL(k_wattn<2>, dim3(grid), dim3(256), 0, st, g); break;
        case 10: hipLaunchKernelGGL(k_wattn<10>, dim3(grid), dim3(256), 0, st, g); break;
        case 30: hipLaunchKernelGGL(k_wattn<30>, dim3(grid), dim3(256), 0, st, g); break;
        default: hipLaunchKernelGGL(k_wattn<32>, dim3(grid), dim3(256), 0, st, g); break;
        }
        return hipGetLastError();
    }
    if (g0.unit) return hipErrorInvalidValue;  // no unit-layout kernel for this head shape
    const AttnArgs &g = g0;
    const unsigned grid = (unsigned)((g.nw * g.heads + 3) / 4);
    if (grid_out) *grid_out = grid;
    hipLaunchKernelGGL(k_attention, dim3(grid), dim3(256), 0, st, g);
    return hipGetLastError();
}

unsigned attention_grid(const AttnArgs &g) {
    return wattn_eligible(g) ? (unsigned)(8 * ((g.heads + 1) / 2) * wattn_lanes(g))
                             : (unsigned)((g.nw * g.heads + 3) / 4);
}

void qkv_pair_weights(const float *w, const float *b, int heads, int hd, float *w_out,
                      float *b_out) {
    const int c = heads * hd;
    for (int p = 0; p < heads / 2; ++p)
        for (int u = 0; u < 6 * hd; ++u) {
            // unit column u: segment u / (2hd) (q, k, v), head 2p + (u / hd) % 2, d
            const int seg = u / (2 * hd), hp = (u / hd) & 1, d = u % hd;
            const int src = seg * c + (2 * p + hp) * hd + d;
            for (int k = 0; k < c; ++k) w_out[((size_t)p * 6 * hd + u) * c + k] = w[(size_t)src * c + k];
            b_out[p * 6 * hd + u] = b[src];
        }
}

// k_qkv_wattn's persistent grid: 8 XCDs x 3 head pairs x window lanes, two
// workgroups per CU, never more lanes than an XCD has windows.
static int qkv_attn_lanes(int nw) {
    return std::max(1, std::min((nw + 7) / 8, 2 * cu_count() / (8 * 3)));
}

unsigned qkv_attention_grid(int hp, int wp) {
    return (unsigned)(8 * 3 * qkv_attn_lanes((hp / 8) * (wp / 8)));
}

hipError_t launch_qkv_attention(const QkvAttnArgs &g0, hipStream_t st, unsigned *grid_out) {
    if (g0.hp <= 0 || g0.wp <= 0 || g0.hp % 8 || g0.wp % 8 || g0.shift < 0 || g0.shift >= 8)
        return hipErrorInvalidValue;
    QkvAttnArgs g = g0;
    g.nww = g.wp / 8;
    g.nw = (g.hp / 8) * g.nww;
    g.nws = qkv_attn_lanes(g.nw);
    const unsigned grid = (unsigned)(8 * 3 * g.nws);
    if (grid_out) *grid_out = grid;
    hipLaunchKernelGGL(k_qkv_wattn, dim3(grid), dim3(256), 0, st, g);
    return hipGetLastError();
}

hipError_t launch_pad_input(const float *in, float *out, int h, int w, int hp, int wp,
                            hipStream_t st) {
    const int n = hp * wp;
    hipLaunchKernelGGL(k_pad_input, dim3((n + 255) / 256), dim3(256), 0, st, in, out, h, w, hp,
                       wp);
    return hipGetLastError();
}

hipError_t launch_layernorm(const float *x, const float *w, const float *b, const float *res,
                            float *out, int P, int C, hipStream_t st) {
    if (C > 192 || C % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_layernorm, dim3((P + 16 * LN_PIX - 1) / (16 * LN_PIX)), dim3(256), 0, st, x,
                       w, b, res, out, P,
                       C);
    return hipGetLastError();
}

dim3 conv_last_grid(int oh, int ow) {
    return dim3((ow + CL_COLS - 1) / CL_COLS, (oh + CL_ROWS - 1) / CL_ROWS);
}

hipError_t launch_conv_last_finish(const float *in, const float *wt, const float *bias,
                                   float *out, int H, int W, int feat, int oh, int ow,
                                   float img_range, const float *mean, hipStream_t st) {
    if (feat % CL_CC) return hipErrorInvalidValue;
    const dim3 grid = conv_last_grid(oh, ow);
    hipLaunchKernelGGL(k_conv_last_finish<false>, grid, dim3(256), 0, st, in, wt, bias, out, H, W,
                       feat, oh, ow, 1.0f / img_range, mean[0], mean[1], mean[2], nullptr, img_range);
    return hipGetLastError();
}

hipError_t launch_conv_aux(const float *in, const float *wt, const float *bias, float *aux4,
                           float *auxp, int H, int W, int feat, float img_range, const float *mean,
                           hipStream_t st) {
    if (feat % CL_CC) return hipErrorInvalidValue;
    const dim3 grid = conv_last_grid(H, W);
    hipLaunchKernelGGL(k_conv_last_finish<true>, grid, dim3(256), 0, st, in, wt, bias, auxp, H, W,
                       feat, H, W, 1.0f / img_range, mean[0], mean[1], mean[2], aux4, img_range);
    return hipGetLastError();
}

// rows per wave of k_up_last: 2 while 8-row tiles give two workgroups per CU
static int up_last_rpw(int oh, int ow) {
    const long long tiles8 = (long long)((ow / 2 + UL_COLS - 1) / UL_COLS) * ((oh / 2 + 7) / 8);
    return tiles8 >= 2LL * cu_count() ? 2 : 1;
}

dim3 up_last_grid(int oh, int ow) {
    const int rows = 4 * up_last_rpw(oh, ow);
    return dim3((ow / 2 + UL_COLS - 1) / UL_COLS, (oh / 2 + rows - 1) / rows);
}

hipError_t launch_up_last(const float *in, const float *wt, const float *bias, const float *wedge,
                          const float *bedge, float *out, int H, int W, int feat, int oh, int ow,
                          float img_range, const float *mean, hipStream_t st) {
    // the kernels' assumptions: whole 8-channel chunks, even output sides, and
    // every computed input pixel inside the plane
    if (feat % UL_CC || oh % 2 || ow % 2 || oh / 2 > H || ow / 2 > W) return hipErrorInvalidValue;
    const float ir = 1.0f / img_range;
    hipLaunchKernelGGL(up_last_rpw(oh, ow) == 2 ? k_up_last<2> : k_up_last<1>, up_last_grid(oh, ow),
                       dim3(256), 0, st, in, wt, bias, out, H, W,
                       feat, oh, ow, ir, mean[0], mean[1], mean[2]);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int n = (ow / 2 + oh / 2 - 1) * 12;  // (border pixel, output) pairs, one wave each
    hipLaunchKernelGGL(k_up_last_edge, dim3((n + 3) / 4), dim3(256), 0, st, in, wedge, bedge,
                       out, H, W, feat, oh, ow, ir, mean[0], mean[1], mean[2]);
    return hipGetLastError();
}

hipError_t launch_up2_last_edge(const float *in, const float *wedge, const float *bedge, float *out,
                               int H, int W, int feat, int oh, int ow, float img_range,
                               const float *mean, hipStream_t st) {
    if (feat != U2E_FEAT || (oh + 3) / 4 > H || (ow + 3) / 4 > W) return hipErrorInvalidValue;
    const int n = (ow + 3) / 4 + (oh + 3) / 4 - 1;  // border pixels, one workgroup each
    hipLaunchKernelGGL(k_up2_last_edge, dim3(n), dim3(256), 0, st, in, wedge, bedge, out, H, W, oh,
                       ow, 1.0f / img_range, mean[0], mean[1], mean[2]);
    return hipGetLastError();
}

hipError_t launch_embed(const float *in4, const float *wts, const float *b0, const float *b1,
                        const float *lnw, const float *lnb, float *body, float *cur, int H, int W,
                        int C, hipStream_t st) {
    if (C % 4 || C > 192 || W < 1 || H < 1 || (long long)H * W * C * 4 >= BUF_MAX_BYTES)
        return hipErrorInvalidValue;
    static int per_cu = 0;  // resident workgroups per CU, from the occupancy query
    if (!per_cu) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_embed, 256, 0) != hipSuccess || nb < 1) {
            (void)hipGetLastError();
            nb = 1;
        }
        per_cu = nb;
    }
    const int ntask = (H * W + 15) / 16;
    const int grid = std::max(1, std::min(ntask, per_cu * cu_count()));
    hipLaunchKernelGGL(k_embed, dim3(grid), dim3(256), 0, st, in4, wts, b0, b1, lnw, lnb, body, cur,
                       H, W, C);
    return hipGetLastError();
}

hipError_t launch_cpb(const float *w0, const float *b0, const float *w2, float *tab, float *cpbt,
                      int win, int heads, hipStream_t st) {
    const int side = 2 * win - 1, n = win * win;
    hipLaunchKernelGGL(k_cpb_mlp, dim3(side * side), dim3(256), 0, st, w0, b0, w2, tab, win,
                       heads);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int total = heads * n * n;
    hipLaunchKernelGGL(k_cpb_gather, dim3((total + 255) / 256), dim3(256), 0, st, tab, cpbt, win,
                       heads);
    return hipGetLastError();
}

// Winograd F(4x4,3x3): a 4x4 output tile from its 6x6 input patch with 36
// products per (input, output) channel pair instead of 144. The transforms
// come from the Toom-Cook construction with the interpolation points
// 0, 3/2, -3/2, 2/3, -2/3 and infinity (on unit-normal data at C = 180 their
// fp32 error is about a third of that of the points 0, +-1, +-2):
//   B^T = [1    0    -97/36  0      1  0]    G = [1       0       0    ]
//         [0  -2/3   -4/9    3/2    1  0]        [8/65    12/65   18/65]
//         [0   2/3   -4/9   -3/2    1  0]        [8/65   -12/65   18/65]
//         [0  -3/2   -9/4    2/3    1  0]        [-81/130 -27/65 -18/65]
//         [0   3/2   -9/4   -2/3    1  0]        [-81/130  27/65 -18/65]
//         [0    1     0    -97/36   0  1]        [0       0       1    ]
//   A^T = [1   1     1     1     1    0]
//         [0  3/2  -3/2   2/3  -2/3   0]
//         [0  9/4   9/4   4/9   4/9   0]
//         [0 27/8 -27/8  8/27 -8/27   1]
// so that, for the cross-correlation the conv layers compute (tap (a, b) of
// output pixel (y, x) reads input (y + a - 1, x + b - 1)),
// Y = A^T [ (G g G^T) .* (B^T d B) ] A per tile and channel pair, summed over
// the input channels by the transform-domain GEMM.

// B^T applied to the 6 values x[0], x[S], ..., x[5S], in place (14 VALU).
template <int S> __device__ __forceinline__ void wino4_bt(float *x) {
    const float d0 = x[0], d1 = x[S], d2 = x[2 * S], d3 = x[3 * S], d4 = x[4 * S], d5 = x[5 * S];
    const float e1 = fmaf(-4.f / 9.f, d2, d4), o1 = fmaf(1.5f, d3, (-2.f / 3.f) * d1);
    const float e2 = fmaf(-2.25f, d2, d4), o2 = fmaf(2.f / 3.f, d3, -1.5f * d1);
    x[0] = fmaf(-97.f / 36.f, d2, d0 + d4);
    x[S] = e1 + o1;
    x[2 * S] = e1 - o1;
    x[3 * S] = e2 + o2;
    x[4 * S] = e2 - o2;
    x[5 * S] = fmaf(-97.f / 36.f, d3, d1 + d5);
}
// A^T applied to m[0], m[S], ..., m[5S], into y[0], y[T], y[2T], y[3T].
template <int S, int T> __device__ __forceinline__ void wino4_at(const float *m, float *y) {
    const float s12 = m[S] + m[2 * S], d12 = m[S] - m[2 * S];
    const float s34 = m[3 * S] + m[4 * S], d34 = m[3 * S] - m[4 * S];
    y[0] = m[0] + s12 + s34;
    y[T] = fmaf(1.5f, d12, (2.f / 3.f) * d34);
    y[2 * T] = fmaf(2.25f, s12, (4.f / 9.f) * s34);
    y[3 * T] = fmaf(3.375f, d12, fmaf(8.f / 27.f, d34, m[5 * S]));
}

// NE consecutive floats (4: a float4, 2: a float2) at p.
template <int NE> __device__ __forceinline__ void ld_vec(const float *p, float *v) {
    if constexpr (NE == 4) {
        const float4 t = *reinterpret_cast<const float4 *>(p);
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
    } else {
        const float2 t = *reinterpret_cast<const float2 *>(p);
        v[0] = t.x;
        v[1] = t.y;
    }
}
template <int NE> __device__ __forceinline__ void st_vec(float *p, const float *v) {
    if constexpr (NE == 4)
        *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
    else
        *reinterpret_cast<float2 *>(p) = make_float2(v[0], v[1]);
}

// channels per thread of the two transforms
#ifndef WINO_IN_NE
#define WINO_IN_NE 4
#endif
#ifndef WINO_OUT_NE
#define WINO_OUT_NE 2
#endif

// Input transform: tile (ty, tx) of the grid of MT x MT output tiles that
// covers Ho x Wo (rounded up), channels c .. c+NE-1: its 6x6 patch d (rows
// MT ty - PAD .. MT ty - PAD + 5, the same for columns, zero outside the H x W
// plane) to V = B^T d B, stored as V[6 xi + nu][tile][c]. F(4x4,3x3) takes
// MT = 4, PAD = 1; F(2x2,5x5) MT = 2, PAD = 2 - the same B^T for the same six
// points. One thread per (tile, NE channels); consecutive threads read and
// write consecutive channel groups.
template <int NE, int MT, int PAD>
__global__ __launch_bounds__(256) void k_wino_in(const float *__restrict__ in, int ldi,
                                                  float *__restrict__ v, int H, int W, int C,
                                                  int T, int tw) {
    const int cgn = C / NE;
    // F(4x4,3x3): workgroups in an XCD-aware order. The dispatcher deals
    // workgroup b to XCD b % 8; with a grid that is a multiple of 8, XCD k
    // takes the k-th eighth of the tiles, so the two patch rows that
    // vertically adjacent tiles share are read through one L2 (measured
    // 34.2 -> 31.4 us at 264^2 x 180). The 5x5 form reads a 64-channel plane
    // and keeps the plain order.
    int bl = (int)blockIdx.x;
    if (MT == 4 && (gridDim.x & 7) == 0)
        bl = (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
    const long long i = (long long)bl * blockDim.x + threadIdx.x;
    if (i >= (long long)T * cgn) return;
    const int tile = (int)(i / cgn);
    const int c = NE * (int)(i - (long long)tile * cgn);
    const int ty = tile / tw, tx = tile - (tile / tw) * tw;
    float p[6][6][NE];  // [row][column][channel]
#pragma unroll
    for (int r = 0; r < 6; ++r)
#pragma unroll
        for (int q = 0; q < 6; ++q) {
            const int y = MT * ty - PAD + r, x = MT * tx - PAD + q;
            if ((unsigned)y < (unsigned)H && (unsigned)x < (unsigned)W) {
                ld_vec<NE>(in + ((size_t)y * W + x) * ldi + c, p[r][q]);
            } else {
#pragma unroll
                for (int e = 0; e < NE; ++e) p[r][q][e] = 0.f;
            }
        }
#pragma unroll
    for (int q = 0; q < 6; ++q)
#pragma unroll
        for (int e = 0; e < NE; ++e) wino4_bt<6 * NE>(&p[0][q][e]);
    const size_t plane = (size_t)T * C;
    float *out = v + (size_t)tile * C + c;
#pragma unroll
    for (int xi = 0; xi < 6; ++xi) {
#pragma unroll
        for (int e = 0; e < NE; ++e) wino4_bt<NE>(&p[xi][0][e]);
#pragma unroll
        for (int nu = 0; nu < 6; ++nu) st_vec<NE>(out + (6 * xi + nu) * plane, p[xi][nu]);
    }
}

unsigned wino_in_grid(int H, int W, int C) {
    // (a multiple of 8 workgroups: k_wino_in's XCD-aware order)
    return (unsigned)(((long long)wino_tiles(H, W) * (C / WINO_IN_NE) + 2047) / 2048 * 8);
}

hipError_t launch_wino_in(const float *in, int ldi, float *v, int H, int W, int C, hipStream_t st) {
    if (H < 1 || W < 1 || C % 4 || ldi % 4) return hipErrorInvalidValue;
    const int tw = (W + 3) / 4;
    const int T = (int)wino_tiles(H, W);
    hipLaunchKernelGGL((k_wino_in<WINO_IN_NE, 4, 1>), dim3(wino_in_grid(H, W, C)), dim3(256), 0, st,
                       in, ldi, v, H, W, C, T, tw);
    return hipGetLastError();
}

unsigned wino5_in_grid(int Ho, int Wo, int C) {
    return (unsigned)(((long long)wino5_tiles(Ho, Wo) * (C / WINO_IN_NE) + 255) / 256);
}

hipError_t launch_wino5_in(const float *in, int ldi, float *v, int H, int W, int Ho, int Wo, int C,
                           hipStream_t st) {
    if (H < 1 || W < 1 || Ho < 1 || Wo < 1 || C % 4 || ldi % 4) return hipErrorInvalidValue;
    const int tw = (Wo + 1) / 2;
    const int T = (int)wino5_tiles(Ho, Wo);
    hipLaunchKernelGGL((k_wino_in<WINO_IN_NE, 2, 2>), dim3(wino5_in_grid(Ho, Wo, C)), dim3(256), 0,
                       st, in, ldi, v, H, W, C, T, tw);
    return hipGetLastError();
}

// Output transform: tile (ty, tx), channels c .. c+NE-1: M[6 xi + nu][tile][c]
// to Y = A^T M A, + bias, + the residual, then LeakyReLU when asked, into the
// tile's 4x4 output pixels that lie inside the plane. One thread per (tile,
// NE channels); M's 36 planes are read with consecutive threads on
// consecutive channel groups.
template <int NE>
__global__ __launch_bounds__(256) void k_wino_out(const float *__restrict__ m,
                                                   const float *__restrict__ bias,
                                                   const float *__restrict__ res, int ldr,
                                                   float *__restrict__ out, int ldo, int H, int W,
                                                   int C, int T, int tw, int lrelu, float slope) {
    const int cgn = C / NE;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)T * cgn) return;
    const int tile = (int)(i / cgn);
    const int c = NE * (int)(i - (long long)tile * cgn);
    const size_t plane = (size_t)T * C;
    const float *src = m + (size_t)tile * C + c;
    float t[6][4][NE];  // [xi][output column][channel]: M A, row by row
#pragma unroll
    for (int xi = 0; xi < 6; ++xi) {
        float mr[6][NE];
#pragma unroll
        for (int nu = 0; nu < 6; ++nu) ld_vec<NE>(src + (6 * xi + nu) * plane, mr[nu]);
#pragma unroll
        for (int e = 0; e < NE; ++e) wino4_at<NE, NE>(&mr[0][e], &t[xi][0][e]);
    }
    float y[4][4][NE];  // [output row][output column][channel]
#pragma unroll
    for (int cx = 0; cx < 4; ++cx)
#pragma unroll
        for (int e = 0; e < NE; ++e) wino4_at<4 * NE, 4 * NE>(&t[0][cx][e], &y[0][cx][e]);
    float bv[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) bv[e] = 0.f;
    if (bias) ld_vec<NE>(bias + c, bv);
    const int ty = tile / tw, tx = tile - (tile / tw) * tw;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int oy = 4 * ty + r;
        if (oy >= H) break;
#pragma unroll
        for (int cx = 0; cx < 4; ++cx) {
            const int ox = 4 * tx + cx;
            if (ox >= W) break;
            const size_t px = (size_t)oy * W + ox;
            float v[NE], rv[NE];
#pragma unroll
            for (int e = 0; e < NE; ++e) v[e] = y[r][cx][e] + bv[e];
            if (res) {
                ld_vec<NE>(res + px * ldr + c, rv);
#pragma unroll
                for (int e = 0; e < NE; ++e) v[e] += rv[e];
            }
            if (lrelu) {
#pragma unroll
                for (int e = 0; e < NE; ++e) v[e] = v[e] < 0.f ? v[e] * slope : v[e];
            }
            st_vec<NE>(out + px * ldo + c, v);
        }
    }
}

unsigned wino_out_grid(int H, int W, int C) {
    return (unsigned)(((long long)wino_tiles(H, W) * (C / WINO_OUT_NE) + 255) / 256);
}

hipError_t launch_wino_out(const float *m, const float *bias, const float *res, int ldr,
                           float *out, int ldo, int H, int W, int C, int lrelu, float slope,
                           hipStream_t st) {
    if (H < 1 || W < 1 || C % 4 || ldo % 4 || (res && ldr % 4)) return hipErrorInvalidValue;
    const int tw = (W + 3) / 4;
    const int T = (int)wino_tiles(H, W);
    hipLaunchKernelGGL(k_wino_out<WINO_OUT_NE>, dim3(wino_out_grid(H, W, C)), dim3(256), 0, st, m,
                       bias, res, ldr, out, ldo, H, W, C, T, tw, lrelu, slope);
    return hipGetLastError();
}

// F(2x2,5x5) output transform with the x4 head's finish: tile (ty, tx) of
// the 2x2 tiles covering Ho x Wo input pixels, channels n, n+1 of the 48 (in
// torch's pixel_shuffle(4) order n = 16k + 4a + b, b even): M[6 xi + nu][tile]
// [n] (row stride ldm) to Y = A^T M A with
//   A^T = [1  1    1    1    1   0]
//         [0 3/2 -3/2  2/3 -2/3  1]
// + bias. Input pixel (y, x) = (2ty + r, 2tx + c) holds image pixels
// (4y + a, 4x + b) and (4y + a, 4x + b + 1) of channel k, denormalised as
// v / img_range + mean[k] and cropped to oh x ow, into out [3][oh][ow].
__global__ __launch_bounds__(256) void k_wino5_finish(const float *__restrict__ m, int ldm,
                                                       const float *__restrict__ bias,
                                                       float *__restrict__ out, int T, int tw,
                                                       int Ho, int Wo, int oh, int ow,
                                                       float img_range, float mean0, float mean1,
                                                       float mean2) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)T * 24) return;
    const int tile = (int)(i / 24);
    const int n = 2 * (int)(i - (long long)tile * 24);
    const size_t plane = (size_t)T * ldm;
    const float *src = m + (size_t)tile * ldm + n;
    auto at2 = [](const float *v, int s, float &y0, float &y1) {
        const float s12 = v[s] + v[2 * s], d12 = v[s] - v[2 * s];
        const float s34 = v[3 * s] + v[4 * s], d34 = v[3 * s] - v[4 * s];
        y0 = v[0] + s12 + s34;
        y1 = fmaf(1.5f, d12, fmaf(2.f / 3.f, d34, v[5 * s]));
    };
    float t[6][2][2];  // [xi][output column][channel]
#pragma unroll
    for (int xi = 0; xi < 6; ++xi) {
        float mr[6][2];
#pragma unroll
        for (int nu = 0; nu < 6; ++nu) ld_vec<2>(src + (6 * xi + nu) * plane, mr[nu]);
#pragma unroll
        for (int e = 0; e < 2; ++e) at2(&mr[0][e], 2, t[xi][0][e], t[xi][1][e]);
    }
    float y[2][2][2];  // [output row][output column][channel]
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 2; ++e) at2(&t[0][c][e], 4, y[0][c][e], y[1][c][e]);
    const float b0 = bias[n], b1 = bias[n + 1];
    const int k = n >> 4, a = (n >> 2) & 3, b = n & 3;
    const float mk = k == 0 ? mean0 : (k == 1 ? mean1 : mean2);
    const int ty = tile / tw, tx = tile - (tile / tw) * tw;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int py = 2 * ty + r, px = 2 * tx + c;
            const int oy = 4 * py + a, ox = 4 * px + b;
            if (py >= Ho || px >= Wo || oy >= oh || ox >= ow) continue;
            float *dst = out + ((size_t)k * oh + oy) * ow + ox;
            const float v0 = (y[r][c][0] + b0) / img_range + mk;
            const float v1 = (y[r][c][1] + b1) / img_range + mk;
            if (ox + 1 < ow && !(ow & 1)) {
                *reinterpret_cast<float2 *>(dst) = make_float2(v0, v1);
            } else {
                dst[0] = v0;
                if (ox + 1 < ow) dst[1] = v1;
            }
        }
}

unsigned wino5_finish_grid(int Ho, int Wo) {
    return (unsigned)(((long long)wino5_tiles(Ho, Wo) * 24 + 255) / 256);
}

hipError_t launch_wino5_finish(const float *m, int ldm, const float *bias, float *out, int Ho,
                               int Wo, int oh, int ow, float img_range, const float *mean,
                               hipStream_t st) {
    if (Ho < 1 || Wo < 1 || ldm < 48 || ldm % 2 || !bias) return hipErrorInvalidValue;
    const int tw = (Wo + 1) / 2;
    const int T = (int)wino5_tiles(Ho, Wo);
    hipLaunchKernelGGL(k_wino5_finish, dim3(wino5_finish_grid(Ho, Wo)), dim3(256), 0, st, m, ldm,
                       bias, out, T, tw, Ho, Wo, oh, ow, img_range, mean[0], mean[1], mean[2]);
    return hipGetLastError();
}

// U = G5 g G5^T per (co, ci) for F(2x2,5x5) with the points above,
//   G5 = [1        0       0      0       0     ]
//        [8/65     12/65   18/65  27/65   81/130]
//        [8/65    -12/65   18/65 -27/65   81/130]
//        [-81/130 -27/65  -18/65 -12/65  -8/65  ]
//        [-81/130  27/65  -18/65  12/65  -8/65  ]
//        [0        0       0      0       1     ],
// from weights w [co][25][ci] (tap-major, in double) as [36][co][round4(ci)].
void wino5_weights(const double *w, int co, int ci, float *out) {
    static const double G[6][5] = {{1, 0, 0, 0, 0},
                                   {8.0 / 65, 12.0 / 65, 18.0 / 65, 27.0 / 65, 81.0 / 130},
                                   {8.0 / 65, -12.0 / 65, 18.0 / 65, -27.0 / 65, 81.0 / 130},
                                   {-81.0 / 130, -27.0 / 65, -18.0 / 65, -12.0 / 65, -8.0 / 65},
                                   {-81.0 / 130, 27.0 / 65, -18.0 / 65, 12.0 / 65, -8.0 / 65},
                                   {0, 0, 0, 0, 1}};
    const int cp = (ci + 3) / 4 * 4;
    for (size_t i = 0; i < (size_t)WINO_POS * co * cp; ++i) out[i] = 0.f;
    for (int o = 0; o < co; ++o)
        for (int i = 0; i < ci; ++i)
            for (int xi = 0; xi < 6; ++xi)
                for (int nu = 0; nu < 6; ++nu) {
                    double u = 0.0;
                    for (int a = 0; a < 5; ++a)
                        for (int b = 0; b < 5; ++b)
                            u += G[xi][a] * w[((size_t)o * 25 + 5 * a + b) * ci + i] * G[nu][b];
                    out[((size_t)(6 * xi + nu) * co + o) * cp + i] = (float)u;
                }
}

// U = G g G^T per (co, ci) with G above, accumulated in double and rounded
// once, as the GEMM's B: [36][co][round4(ci)] with batch b = 6 xi + nu.
void wino_weights(const float *w, int co, int ci, float *out) {
    static const double G[6][3] = {{1, 0, 0},
                                   {8.0 / 65, 12.0 / 65, 18.0 / 65},
                                   {8.0 / 65, -12.0 / 65, 18.0 / 65},
                                   {-81.0 / 130, -27.0 / 65, -18.0 / 65},
                                   {-81.0 / 130, 27.0 / 65, -18.0 / 65},
                                   {0, 0, 1}};
    const int cp = (ci + 3) / 4 * 4;
    for (size_t i = 0; i < (size_t)WINO_POS * co * cp; ++i) out[i] = 0.f;
    for (int o = 0; o < co; ++o)
        for (int i = 0; i < ci; ++i) {
            const float *g = w + ((size_t)o * ci + i) * 9;
            for (int xi = 0; xi < 6; ++xi)
                for (int nu = 0; nu < 6; ++nu) {
                    double u = 0.0;
                    for (int a = 0; a < 3; ++a)
                        for (int b = 0; b < 3; ++b) u += G[xi][a] * (double)g[3 * a + b] * G[nu][b];
                    out[((size_t)(6 * xi + nu) * co + o) * cp + i] = (float)u;
                }
        }
}

// A 3x3 conv (w [co][ci][3][3]) of the nearest-2x upsampling of a plane, as
// the four 2x2 convs of the plane itself that the ALOAD_SUB2 GEMM runs, one
// per output phase (a, b) (reference src/gpu.rs:641-669, the real-world head's
// conv_up1 / conv_up2: nearest upsampling, then the conv). Output row
// 2y + a, tap ky reads upsampled row 2y + a + ky - 1, i.e. plane row
// floor((2y + a + ky - 1) / 2) = y + a - 1 + i with i = 0 for ky in S(a, 0)
// and 1 for ky in S(a, 1): S(0, 0) = {0}, S(0, 1) = {1, 2}, S(1, 0) = {0, 1},
// S(1, 1) = {2}; the same for the columns. The phase's 2x2 weights are the
// sums of the 3x3 taps that land on the same plane pixel (in double, rounded
// once); the upsampled plane's zero padding is the plane's. Layout [4 phases]
// [co][4 taps (i, j)][ci_pad4], k = tap * ci_pad4 + ci: 16 co ci_pad4 floats at out.
void subpixel_weights(const float *w, int co, int ci, float *out) {
    const int cp = (ci + 3) / 4 * 4;
    std::fill(out, out + (size_t)4 * co * 4 * cp, 0.f);
    // whether tap k (0..2) of the 3x3 lands on tap i (0..1) of phase a's 2x2
    auto in_set = [](int a, int i, int k) {
        return a == 0 ? (i == 0 ? k == 0 : k >= 1) : (i == 0 ? k <= 1 : k == 2);
    };
    for (int ph = 0; ph < 4; ++ph) {
        const int a = ph >> 1, b = ph & 1;
        for (int o = 0; o < co; ++o)
            for (int c = 0; c < ci; ++c)
                for (int i = 0; i < 2; ++i)
                    for (int j = 0; j < 2; ++j) {
                        double sum = 0.0;
                        for (int ky = 0; ky < 3; ++ky)
                            for (int kx = 0; kx < 3; ++kx)
                                if (in_set(a, i, ky) && in_set(b, j, kx))
                                    sum += w[(((size_t)o * ci + c) * 3 + ky) * 3 + kx];
                        out[(((size_t)ph * co + o) * 4 + 2 * i + j) * cp + c] = (float)sum;
                    }
    }
}

hipError_t launch_bicubic4(const float *in, float *out, int h, int w, int oh, int ow,
                           hipStream_t st) {
    const int n = oh * ow;
    hipLaunchKernelGGL(k_bicubic4, dim3((n + 255) / 256), dim3(256), 0, st, in, out, h, w, oh, ow);
    return hipGetLastError();
}

hipError_t launch_window_map(int hp, int wp, int shift, int32_t *yx, uint8_t *reg,
                             hipStream_t st) {
    const int total = (hp / 8) * (wp / 8) * 64;
    hipLaunchKernelGGL(k_window_map, dim3((total + 255) / 256), dim3(256), 0, st, hp, wp, shift,
                       yx, reg);
    return hipGetLastError();
}
