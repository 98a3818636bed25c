// s2s_test_api.cpp - the per-op test entry points of include/swin2sr_hip.h
// (the device half of the reference's gpu::selftest, src/gpu.rs:889-1265).
// Each uploads host operands, runs ONE kernel of the production path on the
// null stream, downloads and synchronises. They reuse the production launchers
// so the tested code is the code the forward runs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "swin2sr_hip.h"
#include "s2s_kernels.h"

namespace {

// Scoped device allocations: everything is freed on return, success or not.
struct Dev {
    std::vector<void *> ptrs;
    ~Dev() {
        for (void *p : ptrs) (void)hipFree(p);
    }
    template <typename T>
    T *alloc(size_t n) {
        void *p = nullptr;
        if (hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)) != hipSuccess) return nullptr;
        ptrs.push_back(p);
        return static_cast<T *>(p);
    }
    template <typename T>
    T *up(const T *host, size_t n) {
        T *d = alloc<T>(n);
        if (d && host && hipMemcpy(d, host, n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
            return nullptr;
        return d;
    }
};

int round4(int v) { return (v + 3) / 4 * 4; }

// channel-pad [rows][c] -> [rows][cp] with zeros
std::vector<float> pad_rows(const float *x, size_t rows, int c, int cp) {
    std::vector<float> o(rows * (size_t)cp, 0.f);
    for (size_t r = 0; r < rows; ++r) std::memcpy(&o[r * cp], x + r * c, sizeof(float) * c);
    return o;
}

// nb weights of host rows [N][K] (each N*K apart) as the forward uploads
// them: in k_bsgemm's register order when that kernel takes the GEMM `g`
// (then g.b_packed and g.b_bstride are set), else unchanged.
std::vector<float> gemm_weights(GemmArgs &g, int aload, int epi, const float *rows, int nb) {
    const size_t raw = (size_t)g.N * g.K;
    if (!bs_takes(g, aload, epi)) return std::vector<float>(rows, rows + raw * nb);
    const size_t pf = bs_weight_floats(g.N, g.K, epi);
    std::vector<float> out(pf * nb);
    for (int b = 0; b < nb; ++b) bs_pack_weights(rows + b * raw, g.K, g.N, g.K, epi, out.data() + b * pf);
    g.b_packed = 1;
    if (nb > 1) g.b_bstride = pf;
    return out;
}

std::vector<float> conv_relayout(const float *w, int co, int ci, const std::vector<int> *perm) {
    const int cp = round4(ci);
    std::vector<float> out((size_t)co * 9 * cp, 0.f);
    for (int o = 0; o < co; ++o) {
        const int dst = perm ? (*perm)[o] : o;
        for (int i = 0; i < ci; ++i)
            for (int t = 0; t < 9; ++t)
                out[((size_t)dst * 9 + t) * cp + i] = w[((size_t)o * ci + i) * 9 + t];
    }
    return out;
}

}  // namespace

namespace {

int fail(const std::string &m) { return s2s_fail(m.c_str()); }

int finish(hipError_t e, const char *what) {
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail(std::string(what) + " failed: " + hipGetErrorString(e));
    return 0;
}

}  // namespace

extern "C" {

int s2s_test_window_map(int hp, int wp, int win, int shift, int32_t *yx, uint8_t *reg) {
    if (win != 8) return fail("the device window map is built for 8x8 windows");
    if (hp % 8 || wp % 8 || hp <= 0 || wp <= 0) return fail("plane must be a multiple of 8");
    if (shift < 0 || shift >= 8) return fail("shift must be in [0, 8)");
    const size_t n = (size_t)(hp / 8) * (wp / 8) * 64;
    Dev d;
    int32_t *dyx = d.alloc<int32_t>(2 * n);
    uint8_t *dreg = d.alloc<uint8_t>(2 * n);
    if (!dyx || !dreg) return fail("hipMalloc failed: out of memory");
    hipError_t e = launch_window_map(hp, wp, shift, dyx, dreg, 0);
    if (int rc = finish(e, "k_window_map")) return rc;
    if (hipMemcpy(yx, dyx, 2 * n * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(reg, dreg, 2 * n, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

int s2s_test_attention(int hp, int wp, int win, int heads, int head_dim, int shift,
                       const float *qkv, const float *logit_scale, const float *cpb, float *out) {
    if (win != 8) return fail("the device attention kernel is built for 8x8 windows");
    if (head_dim > 32 || head_dim <= 0) return fail("head_dim must be in [1, 32]");
    if (hp % 8 || wp % 8) return fail("plane must be a multiple of 8");
    const int c = heads * head_dim;
    if (c % 4) return fail("heads*head_dim must be a multiple of 4");
    const size_t P = (size_t)hp * wp;
    const int n = 64;
    std::vector<float> cpbt((size_t)heads * n * n);
    for (int q = 0; q < n; ++q)
        for (int k = 0; k < n; ++k)
            for (int h = 0; h < heads; ++h)
                cpbt[((size_t)h * n + q) * n + k] = ATTN_LOG2E * cpb[((size_t)q * n + k) * heads + h];
    // the shapes the unit-layout kernel takes get their qkv in that layout
    // (the qkv GEMM writes it in the forward; here the host lays it out)
    const bool unit = attn_unit_eligible(heads, head_dim, c);
    std::vector<float> ql;
    if (unit) {
        const int RS = attn_unit_stride(head_dim), HG = (heads + 1) / 2;
        const int nww = wp / 8, nw = (hp / 8) * nww;
        ql.assign(attn_unit_floats(hp, wp, heads, head_dim), 0.f);
        for (int wi = 0; wi < nw; ++wi)
            for (int t = 0; t < 64; ++t) {
                const int y = (8 * (wi / nww) + t / 8 + shift) % hp;
                const int x = (8 * (wi % nww) + t % 8 + shift) % wp;
                const float *src = qkv + ((size_t)y * wp + x) * 3 * c;
                for (int h = 0; h < heads; ++h)
                    for (int seg = 0; seg < 3; ++seg)
                        for (int dd = 0; dd < head_dim; ++dd)
                            ql[(((size_t)wi * HG + h / 2) * 64 + t) * RS +
                               (2 * seg + (h & 1)) * head_dim + dd] =
                                src[seg * c + h * head_dim + dd];
            }
    }
    Dev d;
    AttnArgs a{};
    a.unit = unit;
    a.qkv = unit ? d.up(ql.data(), ql.size()) : d.up(qkv, P * 3 * c);
    a.cpbt = d.up(cpbt.data(), cpbt.size());
    a.logit_scale = d.up(logit_scale, heads);
    a.out = d.alloc<float>(P * c);
    if (!a.qkv || !a.cpbt || !a.logit_scale || !a.out) return fail("hipMalloc failed: out of memory");
    a.hp = hp;
    a.wp = wp;
    a.nww = wp / 8;
    a.nw = (hp / 8) * (wp / 8);
    a.heads = heads;
    a.head_dim = head_dim;
    a.c = c;
    a.shift = shift;
    hipError_t e = launch_attention(a, 0, nullptr);
    if (int rc = finish(e, "k_attention")) return rc;
    if (hipMemcpy(out, a.out, P * c * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

// The block's qkv GEMM exactly as the forward launches it (qkv_gemm_args:
// the shifted-window gather into the unit layout), its raw output buffer
// downloaded. Unwritten floats (the padding) read back as NaN.
int s2s_test_qkv_windows(int hp, int wp, int heads, int head_dim, int shift, const float *x,
                         const float *wqkv, const float *bqkv, float *unit, size_t unit_cap) {
    const int c = heads * head_dim;
    if (!qkv_unit_layout(heads, head_dim, c))
        return fail("this head shape keeps qkv in the plane layout (no unit layout to probe)");
    if (hp % 8 || wp % 8 || hp <= 0 || wp <= 0) return fail("plane must be a multiple of 8");
    if (shift < 0 || shift >= 8) return fail("shift must be in [0, 8)");
    const size_t P = (size_t)hp * wp, nu = attn_unit_floats(hp, wp, heads, head_dim);
    if (unit_cap < nu) return fail("unit buffer too small: " + std::to_string(nu) + " floats needed");
    Dev d;
    const float *dx = d.up(x, P * c);
    const float *db = d.up(bqkv, (size_t)3 * c);
    float *dq = d.alloc<float>(nu);
    if (!dx || !db || !dq) return fail("hipMalloc failed: out of memory");
    if (hipMemset(dq, 0xff, nu * 4) != hipSuccess) return fail("hipMemset failed");
    GemmArgs g;
    const int epi = qkv_gemm_args(dx, nullptr, db, dq, hp, wp, shift, heads, head_dim, &g);
    const std::vector<float> wg = gemm_weights(g, ALOAD_ROWS, epi, wqkv, 1);
    if (!(g.B = d.up(wg.data(), wg.size()))) return fail("hipMalloc failed: out of memory");
    hipError_t e = launch_gemm(g, ALOAD_ROWS, epi, 0);
    if (int rc = finish(e, "k_bsgemm(qkv)")) return rc;
    if (hipMemcpy(unit, dq, nu * 4, hipMemcpyDeviceToHost) != hipSuccess) return fail("hipMemcpy failed");
    return 0;
}

// The block's attention half exactly as the forward launches it: the qkv
// GEMM (unit or plane layout by head shape), then the window attention whose
// output is scattered back to the plane [hp*wp][c]. `cpb` is [n*n][heads] in
// the checkpoint's (cpb_pre) layout.
int s2s_test_block_attention(int hp, int wp, int heads, int head_dim, int shift, const float *x,
                             const float *wqkv, const float *bqkv, const float *logit_scale,
                             const float *cpb, float *out) {
    const int c = heads * head_dim;
    if (head_dim > 32 || head_dim <= 0 || c % 4) return fail("unsupported head shape");
    if (hp % 8 || wp % 8 || hp <= 0 || wp <= 0) return fail("plane must be a multiple of 8");
    if (shift < 0 || shift >= 8) return fail("shift must be in [0, 8)");
    const size_t P = (size_t)hp * wp;
    const int n = 64;
    std::vector<float> cpbt((size_t)heads * n * n);
    for (int q = 0; q < n; ++q)
        for (int k = 0; k < n; ++k)
            for (int h = 0; h < heads; ++h)
                cpbt[((size_t)h * n + q) * n + k] = ATTN_LOG2E * cpb[((size_t)q * n + k) * heads + h];
    const size_t nq = qkv_unit_layout(heads, head_dim, c)
                          ? std::max(P * 3 * c, attn_unit_floats(hp, wp, heads, head_dim))
                          : P * 3 * c;
    Dev d;
    const float *dx = d.up(x, P * c);
    const float *db = d.up(bqkv, (size_t)3 * c), *dls = d.up(logit_scale, heads);
    const float *dcp = d.up(cpbt.data(), cpbt.size());
    float *dq = d.alloc<float>(nq), *dout = d.alloc<float>(P * c);
    if (!dx || !db || !dls || !dcp || !dq || !dout)
        return fail("hipMalloc failed: out of memory");
    hipError_t e;
    if (qkv_attn_fused(heads, head_dim)) {
        // the forward's fused kernel, with the weights in its order: each head
        // pair's q|k|v rows as the unit's columns, each pair's c x c rows in
        // k_bsgemm's register order
        std::vector<float> wp_((size_t)3 * c * c), bp_((size_t)3 * c);
        qkv_pair_weights(wqkv, bqkv, heads, head_dim, wp_.data(), bp_.data());
        const size_t pf = bs_weight_floats(c, c, EPI_STORE);
        std::vector<float> wk((size_t)(heads / 2) * pf);
        for (int pr = 0; pr < heads / 2; ++pr)
            bs_pack_weights(wp_.data() + (size_t)pr * c * c, c, c, c, EPI_STORE, wk.data() + pr * pf);
        const float *dwp = d.up(wk.data(), wk.size()), *dbp = d.up(bp_.data(), bp_.size());
        if (!dwp || !dbp) return fail("hipMalloc failed: out of memory");
        QkvAttnArgs a{};
        a.x = dx;
        a.w = dwp;
        a.bias = dbp;
        a.cpbt = dcp;
        a.logit_scale = dls;
        a.out = dout;
        a.hp = hp;
        a.wp = wp;
        a.shift = shift;
        e = launch_qkv_attention(a, 0, nullptr);
    } else {
        GemmArgs g;
        const int epi = qkv_gemm_args(dx, nullptr, db, dq, hp, wp, shift, heads, head_dim, &g);
        const std::vector<float> wg = gemm_weights(g, ALOAD_ROWS, epi, wqkv, 1);
        if (!(g.B = d.up(wg.data(), wg.size()))) return fail("hipMalloc failed: out of memory");
        e = launch_gemm(g, ALOAD_ROWS, epi, 0);
        if (e == hipSuccess)
            e = launch_attention(window_attn_args(dq, dcp, dls, dout, hp, wp, shift, heads, head_dim),
                                 0, nullptr);
    }
    if (int rc = finish(e, "qkv + window attention")) return rc;
    if (hipMemcpy(out, dout, P * c * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

int s2s_test_cpb_table(int win, int heads, const float *w0, const float *b0, const float *w2,
                       float *out) {
    if (win < 2) return fail("window must be >= 2");
    const int n = win * win, side = 2 * win - 1;
    Dev d;
    const float *dw0 = d.up(w0, 1024), *db0 = d.up(b0, 512), *dw2 = d.up(w2, (size_t)heads * 512);
    float *tab = d.alloc<float>((size_t)heads * side * side);
    float *cpbt = d.alloc<float>((size_t)heads * n * n);
    if (!dw0 || !db0 || !dw2 || !tab || !cpbt) return fail("hipMalloc failed: out of memory");
    hipError_t e = launch_cpb(dw0, db0, dw2, tab, cpbt, win, heads, 0);
    if (int rc = finish(e, "k_cpb")) return rc;
    std::vector<float> t((size_t)heads * n * n);
    if (hipMemcpy(t.data(), cpbt, t.size() * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    for (int q = 0; q < n; ++q)
        for (int k = 0; k < n; ++k)
            for (int h = 0; h < heads; ++h)
                out[((size_t)q * n + k) * heads + h] = t[((size_t)h * n + q) * n + k] / ATTN_LOG2E;
    return 0;
}

int s2s_test_linear(int rows, int c_in, int c_out, const float *x, const float *w,
                    const float *bias, int epilogue, const float *res, const float *ln_w,
                    const float *ln_b, float slope, float *out) {
    static const int map[6] = {EPI_STORE, EPI_GELU, EPI_RES, EPI_LN, EPI_LN_RES, EPI_LRELU};
    if (epilogue < 0 || epilogue > 5) return fail("epilogue must be 0..5");
    const int epi = map[epilogue];
    if ((epi == EPI_LN || epi == EPI_LN_RES) && c_out > 192)
        return fail("LayerNorm epilogues need c_out <= 192");
    if ((epi == EPI_RES || epi == EPI_LN_RES) && !res) return fail("residual epilogue needs res");
    if ((epi == EPI_LN || epi == EPI_LN_RES) && (!ln_w || !ln_b)) return fail("LN needs ln_w/ln_b");
    const int kp = round4(c_in);
    std::vector<float> xp = pad_rows(x, rows, c_in, kp), wp = pad_rows(w, c_out, c_in, kp);
    Dev d;
    GemmArgs g{};
    g.A = d.up(xp.data(), xp.size());
    g.lda = kp;
    g.ldb = kp;
    g.bias = bias ? d.up(bias, c_out) : nullptr;
    float *dout = d.alloc<float>((size_t)rows * c_out);
    g.out = dout;
    g.ldo = c_out;
    g.res = res ? d.up(res, (size_t)rows * c_out) : nullptr;
    g.ldr = c_out;
    g.ln_w = ln_w ? d.up(ln_w, c_out) : nullptr;
    g.ln_b = ln_b ? d.up(ln_b, c_out) : nullptr;
    g.slope = slope;
    g.M = rows;
    g.N = c_out;
    g.K = kp;
    // the weights as the forward holds them (register order for k_bsgemm)
    const std::vector<float> wg = gemm_weights(g, ALOAD_ROWS, epi, wp.data(), 1);
    g.B = d.up(wg.data(), wg.size());
    if (!g.A || !g.B || !dout) return fail("hipMalloc failed: out of memory");
    hipError_t e = launch_gemm(g, ALOAD_ROWS, epi, 0);
    if (int rc = finish(e, "k_gemm")) return rc;
    if (hipMemcpy(out, dout, (size_t)rows * c_out * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

int s2s_test_ln_residual(int hw, int c, const float *x, const float *ln_w, const float *ln_b,
                         const float *res, float *out) {
    if (c % 4 || c > 256) return fail("the LayerNorm kernel needs c % 4 == 0 and c <= 256");
    Dev d;
    const float *dx = d.up(x, (size_t)hw * c), *dw = d.up(ln_w, c), *db = d.up(ln_b, c);
    const float *dr = res ? d.up(res, (size_t)hw * c) : nullptr;
    float *dy = d.alloc<float>((size_t)hw * c);
    if (!dx || !dw || !db || !dy || (res && !dr)) return fail("hipMalloc failed: out of memory");
    hipError_t e = launch_layernorm(dx, dw, db, dr, dy, hw, c, 0);
    if (int rc = finish(e, "k_layernorm")) return rc;
    if (hipMemcpy(out, dy, (size_t)hw * c * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

int s2s_test_embed(int h, int w, int c, const float *x, const float *w_first, const float *b_first,
                   const float *w_fold, const float *b_fold, const float *ln_w, const float *ln_b,
                   float *body, float *cur) {
    if (c % 4 || c > 192 || c <= 0) return fail("the embed kernel needs c % 4 == 0 and c <= 192");
    if (h < 1 || w < 1) return fail("empty plane");
    const size_t P = (size_t)h * w;
    // the kernel's operands as s2s_create lays them out: the input with a
    // zero fourth channel, the weights [set][tap][ci < 4][c]
    std::vector<float> in4(P * 4, 0.f), wt((size_t)2 * 9 * 4 * c, 0.f);
    for (size_t i = 0; i < P; ++i)
        for (int ci = 0; ci < 3; ++ci) in4[i * 4 + ci] = x[i * 3 + ci];
    for (int o = 0; o < c; ++o)
        for (int ci = 0; ci < 3; ++ci)
            for (int t = 0; t < 9; ++t) {
                wt[((size_t)t * 4 + ci) * c + o] = w_first[(size_t)o * 27 + ci * 9 + t];
                wt[((size_t)(9 + t) * 4 + ci) * c + o] = w_fold[(size_t)o * 27 + ci * 9 + t];
            }
    Dev d;
    const float *di = d.up(in4.data(), in4.size()), *dw = d.up(wt.data(), wt.size());
    const float *b0 = d.up(b_first, c), *b1 = d.up(b_fold, c), *lw = d.up(ln_w, c), *lb = d.up(ln_b, c);
    float *db = d.alloc<float>(P * c), *dc = d.alloc<float>(P * c);
    if (!di || !dw || !b0 || !b1 || !lw || !lb || !db || !dc) return fail("hipMalloc failed: out of memory");
    hipError_t e = launch_embed(di, dw, b0, b1, lw, lb, db, dc, h, w, c, 0);
    if (int rc = finish(e, "k_embed")) return rc;
    if (hipMemcpy(body, db, P * c * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(cur, dc, P * c * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

int s2s_test_conv3x3(int h, int w, int c_in, int c_out, const float *x, const float *wgt,
                     const float *bias, int epilogue, const float *res, float slope, float *out) {
    int epi;
    if (epilogue == 0) epi = EPI_STORE;
    else if (epilogue == 2) epi = EPI_RES;
    else if (epilogue == 5) epi = EPI_LRELU;
    else return fail("conv3x3 epilogue must be 0, 2 or 5");
    if (epi == EPI_RES && !res) return fail("residual epilogue needs res");
    const int cp = round4(c_in);
    const size_t P = (size_t)h * w;
    std::vector<float> xp = pad_rows(x, P, c_in, cp);
    std::vector<float> wt = conv_relayout(wgt, c_out, c_in, nullptr);
    Dev d;
    GemmArgs g{};
    g.A = d.up(xp.data(), xp.size());
    g.H = h;
    g.W = w;
    g.cin = cp;
    g.B = d.up(wt.data(), wt.size());
    g.ldb = 9 * cp;
    g.bias = bias ? d.up(bias, c_out) : nullptr;
    float *dout = d.alloc<float>(P * c_out);
    g.out = dout;
    g.ldo = c_out;
    g.res = res ? d.up(res, P * c_out) : nullptr;
    g.ldr = c_out;
    g.slope = slope;
    g.M = (int)P;
    g.N = c_out;
    g.K = 9 * cp;
    if (!g.A || !g.B || !dout) return fail("hipMalloc failed: out of memory");
    hipError_t e = launch_gemm(g, ALOAD_IM2COL, epi, 0);
    if (int rc = finish(e, "k_gemm(conv3x3)")) return rc;
    if (hipMemcpy(out, dout, P * c_out * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

int s2s_test_conv3x3_winograd(int h, int w, int c_in, int c_out, const float *x, const float *wgt,
                              const float *bias, int epilogue, const float *res, float slope,
                              float *out) {
    if (epilogue != 0 && epilogue != 2 && epilogue != 5) return fail("winograd epilogue must be 0, 2 or 5");
    if (epilogue == 2 && !res) return fail("residual epilogue needs res");
    if (h <= 0 || w <= 0) return fail("the Winograd conv needs a non-empty plane");
    const bool body = c_out == c_in && wino_body(c_in);
    if (!body && !wino_head(c_in, c_out))
        return fail("the Winograd conv is the body's C -> C conv, C in {60, 120, 180}, or "
                    "conv_before_upsample's C -> F, F <= 64 and a multiple of 4");
    const size_t P = (size_t)h * w, T = wino_tiles(h, w);
    std::vector<float> u((size_t)WINO_POS * c_out * c_in);
    wino_weights(wgt, c_out, c_in, u.data());
    GemmArgs g{};
    g.lda = c_in;
    g.ldb = c_in;
    g.ldo = c_out;
    g.M = (int)T;
    g.N = c_out;
    g.K = c_in;
    g.nb = WINO_POS;
    g.a_bstride = T * c_in;
    g.o_bstride = T * c_out;
    g.b_bstride = (size_t)c_out * c_in;
    // U in the batched GEMM's register order, as the forward uploads it
    const std::vector<float> ug = gemm_weights(g, ALOAD_ROWS, EPI_STORE, u.data(), WINO_POS);
    Dev d;
    const float *dx = d.up(x, P * c_in), *du = d.up(ug.data(), ug.size());
    const float *db = bias ? d.up(bias, c_out) : nullptr;
    const float *dr = res ? d.up(res, P * c_out) : nullptr;
    // V [36][T][C_in], then M [36][T][C_out] - over V row for row for the
    // body's convs, in a buffer of its own for conv_before_upsample, as the
    // forward does
    float *dv = d.alloc<float>(WINO_POS * T * c_in), *dout = d.alloc<float>(P * c_out);
    float *dm = body ? dv : d.alloc<float>(WINO_POS * T * c_out);
    if (!dx || !du || !dv || !dm || !dout || (bias && !db) || (res && !dr))
        return fail("hipMalloc failed: out of memory");
    g.A = dv;
    g.B = du;
    g.out = dm;
    hipError_t e = launch_wino_in(dx, c_in, dv, h, w, c_in, 0);
    if (e == hipSuccess) e = launch_gemm(g, ALOAD_ROWS, EPI_STORE, 0);
    if (e == hipSuccess)
        e = launch_wino_out(dm, db, epilogue == 2 ? dr : nullptr, c_out, dout, c_out, h, w, c_out,
                            epilogue == 5, slope, 0);
    if (int rc = finish(e, "winograd conv3x3")) return rc;
    if (hipMemcpy(out, dout, P * c_out * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

int s2s_test_conv3x3_shuffle2(int h, int w, int c_in, int feat, const float *x,
                              const float *wgt, const float *bias, float *out) {
    const int cp = round4(c_in);
    const size_t P = (size_t)h * w;
    std::vector<int> perm(4 * feat);
    for (int co = 0; co < 4 * feat; ++co) perm[co] = (co % 4) * feat + co / 4;
    std::vector<float> xp = pad_rows(x, P, c_in, cp);
    std::vector<float> wt = conv_relayout(wgt, 4 * feat, c_in, &perm);
    std::vector<float> bp(4 * feat);
    for (int co = 0; co < 4 * feat; ++co) bp[perm[co]] = bias[co];
    Dev d;
    GemmArgs g{};
    g.A = d.up(xp.data(), xp.size());
    g.H = h;
    g.W = w;
    g.cin = cp;
    g.B = d.up(wt.data(), wt.size());
    g.ldb = 9 * cp;
    g.bias = d.up(bp.data(), bp.size());
    float *dout = d.alloc<float>(P * 4 * feat);
    g.out = dout;
    g.feat = feat;
    g.M = (int)P;
    g.N = 4 * feat;
    g.K = 9 * cp;
    if (!g.A || !g.B || !g.bias || !dout) return fail("hipMalloc failed: out of memory");
    hipError_t e = launch_gemm(g, ALOAD_IM2COL, EPI_SHUFFLE, 0);
    if (int rc = finish(e, "k_gemm(conv3x3_shuffle2)")) return rc;
    if (hipMemcpy(out, dout, P * 4 * feat * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

int s2s_test_conv3x3_nearest2(int h, int w, int c, const float *x, const float *wgt,
                              const float *bias, float slope, float *out) {
    if (h < 1 || w < 1 || c < 4 || c % 4) return fail("s2s_test_conv3x3_nearest2: bad shape");
    const size_t P = (size_t)h * w;
    std::vector<float> wt((size_t)16 * c * c);
    subpixel_weights(wgt, c, c, wt.data());
    Dev d;
    GemmArgs g{};
    g.A = d.up(x, P * c);
    g.H = h;
    g.W = w;
    g.cin = c;
    g.B = d.up(wt.data(), wt.size());
    g.ldb = 4 * c;
    g.bias = d.up(bias, c);
    float *dout = d.alloc<float>(4 * P * c);
    g.out = dout;
    g.ldo = c;
    g.M = (int)P;
    g.N = c;
    g.K = 4 * c;
    g.slope = slope;
    if (!g.A || !g.B || !g.bias || !dout) return fail("hipMalloc failed: out of memory");
    hipError_t e = launch_gemm(g, ALOAD_SUB2, EPI_LRELU, 0);
    if (int rc = finish(e, "k_gemm(conv_sub2)")) return rc;
    if (hipMemcpy(out, dout, 4 * P * c * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail("hipMemcpy failed");
    return 0;
}

int s2s_test_mfma_peak(int iters, int reps, double *ms, double *tflops, double *ghz) {
    if (iters <= 0 || reps <= 0 || !ms || !tflops || !ghz) return fail("s2s_test_mfma_peak: bad argument");
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return fail("s2s_test_mfma_peak: no device");
    Dev d;
    float *out = d.alloc<float>((size_t)cus * 512);
    if (!out) return fail("hipMalloc failed: out of memory");
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = launch_mfma_peak(out, cus, iters, 0);  // warm-up
    if (e == hipSuccess) e = hipEventRecord(e0, 0);
    for (int r = 0; r < reps && e == hipSuccess; ++r) e = launch_mfma_peak(out, cus, iters, 0);
    if (e == hipSuccess) e = hipEventRecord(e1, 0);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float t = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (e != hipSuccess) return fail(std::string("s2s_test_mfma_peak: ") + hipGetErrorString(e));
    *ms = (double)t / reps;
    // 8 waves per workgroup, 4 MFMAs per iteration, 2048 FLOPs each
    *tflops = (double)cus * 8 * 4 * (double)iters * 2048.0 / (*ms * 1e-3) / 1e12;
    // 4 SIMDs per CU, 64 fp32 matrix FLOPs per cycle each
    *ghz = *tflops * 1e12 / ((double)cus * 4 * 64) / 1e9;
    return 0;
}

int s2s_test_rstb(s2s_ctx *ctx, int stage, int hp, int wp, const float *x, float *out) {
    if (!ctx || !x || !out) return fail("s2s_test_rstb: null argument");
    const int c = s2s_ctx_embed(ctx);
    if (c <= 0 || hp <= 0 || wp <= 0) return fail("s2s_test_rstb: bad shape");
    const size_t n = (size_t)hp * wp * c;
    Dev d;
    float *dx = d.up(x, n);
    float *dy = d.alloc<float>(n);
    if (!dx || !dy) return fail("hipMalloc failed: out of memory");
    if (int rc = s2s_rstb_device(ctx, stage, hp, wp, dx, dy)) return rc;
    hipError_t e = hipStreamSynchronize((hipStream_t)s2s_stream(ctx));
    if (e != hipSuccess) return fail(std::string("hipStreamSynchronize failed: ") + hipGetErrorString(e));
    if (hipMemcpy(out, dy, n * 4, hipMemcpyDeviceToHost) != hipSuccess) return fail("hipMemcpy failed");
    return 0;
}

}  // extern "C"
