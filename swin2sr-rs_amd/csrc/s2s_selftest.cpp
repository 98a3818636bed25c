// s2s_selftest.cpp - s2s_selftest: every production kernel against its CPU
// definition, the device half of the crate's `--cuda-selftest`
// (reference gpu::selftest, src/gpu.rs:889-1265; CLI src/main.rs:180-192).
//
// Each check runs one kernel of the forward through its per-op test entry
// (which uses the production launchers) on a small deterministic input - the
// reference selftest's generator, x[i] = sin(0.7 i + phase) - and holds it
// against the operation's textbook definition evaluated here in double
// precision. The definitions are short and written for clarity, not speed;
// they exist only for this self-check and never produce a forward's output.
// Tolerance: the reference selftest's 2e-5 (src/gpu.rs:892), relative to the
// larger of 1 and the expected output's magnitude.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "swin2sr_hip.h"
#include "s2s_kernels.h"

namespace {

int fail(const std::string &m) { return s2s_fail(m.c_str()); }

std::vector<float> seq(size_t n, float phase) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = std::sin((float)i * 0.7f + phase);
    return v;
}

// The worst element against `tol * max(1, |want|max)`, reported with where it
// is and both values (reference close(), src/gpu.rs:1267-1289).
int close(const std::string &what, const std::vector<double> &want, const std::vector<float> &got,
          double tol) {
    if (want.size() != got.size())
        return fail(what + ": " + std::to_string(want.size()) + " elements expected, " +
                    std::to_string(got.size()) + " produced");
    double mag = 1.0, worst = 0.0;
    size_t at = 0;
    for (double w : want) mag = std::max(mag, std::fabs(w));
    for (size_t i = 0; i < want.size(); ++i) {
        const double d = std::fabs(want[i] - (double)got[i]);
        if (!(d <= worst)) {
            worst = d;
            at = i;
        }
    }
    if (!(worst <= tol * mag)) {
        char b[256];
        snprintf(b, sizeof b, "%s: max |diff| %.3e at %zu > %.1e (cpu %+.7f, hip %+.7f)", what.c_str(),
                 worst, at, tol * mag, want[at], (double)got[at]);
        return fail(b);
    }
    return 0;
}

double gelu(double x) { return 0.5 * x * (1.0 + std::erf(x / std::sqrt(2.0))); }

// 3x3, stride 1, zero padding 1, on channel-last planes; wgt [co][ci][3][3].
std::vector<double> conv3x3(const std::vector<float> &x, int h, int w, int ci, int co,
                            const std::vector<float> &wgt, const std::vector<float> &bias) {
    std::vector<double> y((size_t)h * w * co);
    for (int yy = 0; yy < h; ++yy)
        for (int xx = 0; xx < w; ++xx)
            for (int o = 0; o < co; ++o) {
                double acc = bias[o];
                for (int i = 0; i < ci; ++i)
                    for (int ky = 0; ky < 3; ++ky)
                        for (int kx = 0; kx < 3; ++kx) {
                            const int sy = yy + ky - 1, sx = xx + kx - 1;
                            if (sy < 0 || sy >= h || sx < 0 || sx >= w) continue;
                            acc += (double)wgt[(((size_t)o * ci + i) * 3 + ky) * 3 + kx] *
                                   x[((size_t)sy * w + sx) * ci + i];
                        }
                y[((size_t)yy * w + xx) * co + o] = acc;
            }
    return y;
}

// The window attention of the published network (network_swin2sr.py
// WindowAttention with the shift mask of calculate_mask), on plane-order q|k|v.
std::vector<double> attention(const std::vector<float> &qkv, int hp, int wp, int heads, int hd,
                              int shift, const std::vector<float> &ls, const std::vector<float> &cpb) {
    const int c = heads * hd, nww = wp / 8, nw = (hp / 8) * nww;
    std::vector<double> out((size_t)hp * wp * c);
    auto band = [&](int a, int p) { return a + 8 < p ? 0 : (a + shift < p ? 1 : 2); };
    std::vector<int> pix(64), by(64), bx(64);
    std::vector<double> s(64);
    for (int wi = 0; wi < nw; ++wi) {
        const int wh = wi / nww, ww = wi % nww;
        for (int t = 0; t < 64; ++t) {
            const int a = wh * 8 + t / 8, b = ww * 8 + t % 8;
            pix[t] = ((a + shift) % hp) * wp + (b + shift) % wp;
            by[t] = band(a, hp);
            bx[t] = band(b, wp);
        }
        for (int h = 0; h < heads; ++h) {
            const double temp = std::exp(std::min((double)ls[h], std::log(100.0)));
            for (int q = 0; q < 64; ++q) {
                const float *qv = &qkv[(size_t)pix[q] * 3 * c + h * hd];
                double qn = 0;
                for (int d = 0; d < hd; ++d) qn += (double)qv[d] * qv[d];
                qn = std::max(std::sqrt(qn), 1e-12);
                double mx = -1e300;
                for (int k = 0; k < 64; ++k) {
                    const float *kv = &qkv[(size_t)pix[k] * 3 * c + c + h * hd];
                    double kn = 0, dot = 0;
                    for (int d = 0; d < hd; ++d) {
                        kn += (double)kv[d] * kv[d];
                        dot += (double)qv[d] * kv[d];
                    }
                    kn = std::max(std::sqrt(kn), 1e-12);
                    double v = dot / (qn * kn) * temp + cpb[((size_t)q * 64 + k) * heads + h];
                    if (shift && (by[q] != by[k] || bx[q] != bx[k])) v -= 100.0;
                    s[k] = v;
                    mx = std::max(mx, v);
                }
                double den = 0;
                for (int k = 0; k < 64; ++k) den += (s[k] = std::exp(s[k] - mx));
                for (int d = 0; d < hd; ++d) {
                    double acc = 0;
                    for (int k = 0; k < 64; ++k)
                        acc += s[k] * qkv[(size_t)pix[k] * 3 * c + 2 * c + h * hd + d];
                    out[(size_t)pix[q] * c + h * hd + d] = acc / den;
                }
            }
        }
    }
    return out;
}

struct Counter {
    int checks = 0;
    int ok(int rc) {
        if (rc == 0) ++checks;
        return rc;
    }
};

#define CHECK(expr)               \
    do {                          \
        if (int rc_ = (expr)) return rc_; \
    } while (0)

const s2s_tensor *find(const s2s_tensor *t, size_t n, const std::string &name) {
    for (size_t i = 0; i < n; ++i)
        if (t[i].name && name == t[i].name) return &t[i];
    return nullptr;
}

}  // namespace

extern "C" int s2s_selftest(const s2s_arch *arch, const s2s_tensor *tensors, size_t n_tensors) {
    if (!arch) return fail("s2s_selftest: null architecture");
    if (arch->heads <= 0 || arch->embed % arch->heads) return fail("s2s_selftest: bad head count");
    const int wheads = arch->heads, whd = arch->embed / arch->heads;
    Counter cnt;
    const double tol = 2e-5;

    // the implicit-GEMM conv3x3 at the reference selftest's shapes (both its
    // direct and its winograd lists: a 7 x 9 plane and a 33 x 39 one, which is
    // not a multiple of any tile)
    {
        const int shapes[6][4] = {{7, 9, 4, 4}, {7, 9, 4, 12}, {7, 9, 12, 3},
                                  {33, 39, 3, 16}, {33, 39, 16, 3}, {33, 39, 16, 20}};
        for (auto &sh : shapes) {
            const int h = sh[0], w = sh[1], ci = sh[2], co = sh[3];
            std::vector<float> x = seq((size_t)h * w * ci, 0.3f), wgt = seq((size_t)co * ci * 9, 1.1f),
                               b = seq(co, 2.2f), got((size_t)h * w * co);
            CHECK(s2s_test_conv3x3(h, w, ci, co, x.data(), wgt.data(), b.data(), 0, nullptr, 0.f,
                                   got.data()));
            CHECK(cnt.ok(close("conv3x3 " + std::to_string(ci) + "->" + std::to_string(co) + " at " +
                                   std::to_string(h) + "x" + std::to_string(w),
                               conv3x3(x, h, w, ci, co, wgt, b), got, tol)));
        }
    }

    // the body's Winograd F(4x4,3x3) conv (the stage close, conv_after_body)
    // at the released widths and the checkpoint's own: a plane that is all
    // border, planes whose sides are not multiples of the 4x4 tile, planes
    // wider than one 64-lane wavefront
    {
        const int shapes[4][3] = {{2, 4, 60}, {34, 41, 120}, {17, 70, 180}, {8, 10, arch->embed}};
        for (auto &sh : shapes) {
            const int h = sh[0], w = sh[1], c = sh[2];
            if (!wino_body(c)) continue;
            std::vector<float> x = seq((size_t)h * w * c, 0.3f), wgt = seq((size_t)c * c * 9, 1.1f),
                               b = seq(c, 2.2f), res = seq((size_t)h * w * c, 0.9f), got((size_t)h * w * c);
            for (float &v : wgt) v /= std::sqrt(9.0f * c);
            CHECK(s2s_test_conv3x3_winograd(h, w, c, c, x.data(), wgt.data(), b.data(), 2, res.data(),
                                            0.f, got.data()));
            std::vector<double> want = conv3x3(x, h, w, c, c, wgt, b);
            for (size_t i = 0; i < want.size(); ++i) want[i] += res[i];
            CHECK(cnt.ok(close("winograd conv3x3 " + std::to_string(c) + "->" + std::to_string(c) +
                                   " + residual at " + std::to_string(h) + "x" + std::to_string(w),
                               want, got, tol)));
        }
    }

    // conv_before_upsample's Winograd conv (C -> F, then LeakyReLU) at the
    // checkpoint's width and a head of 64 features, on a plane ending in
    // partial tiles
    if (wino_head(arch->embed, 64)) {
        const int h = 11, w = 13, c = arch->embed, f = 64;
        std::vector<float> x = seq((size_t)h * w * c, 0.4f), wgt = seq((size_t)f * c * 9, 1.3f),
                           b = seq(f, 2.5f), got((size_t)h * w * f);
        for (float &v : wgt) v /= std::sqrt(9.0f * c);
        CHECK(s2s_test_conv3x3_winograd(h, w, c, f, x.data(), wgt.data(), b.data(), 5, nullptr, 0.01f,
                                        got.data()));
        std::vector<double> want = conv3x3(x, h, w, c, f, wgt, b);
        for (double &v : want) v = v < 0 ? v * 0.01 : v;
        CHECK(cnt.ok(close("winograd conv3x3 " + std::to_string(c) + "->64 + LeakyReLU at 11x13",
                           want, got, tol)));
    }

    // conv3x3 + pixel_shuffle(2) (the head's octave) at the reference's shapes
    {
        const int shapes[5][4] = {{4, 3, 5, 7}, {4, 3, 1, 6}, {6, 24, 4, 5}, {2, 2, 3, 61}, {2, 2, 1, 1025}};
        for (auto &sh : shapes) {
            const int ci = sh[0], feat = sh[1], h = sh[2], w = sh[3];
            std::vector<float> x = seq((size_t)h * w * ci, 0.35f), wgt = seq((size_t)4 * feat * ci * 9, 1.45f),
                               b = seq(4 * feat, 0.75f), got((size_t)4 * h * w * feat);
            CHECK(s2s_test_conv3x3_shuffle2(h, w, ci, feat, x.data(), wgt.data(), b.data(), got.data()));
            // conv to 4*feat channels, then channel 4c + 2dy + dx -> pixel (2y+dy, 2x+dx)
            const std::vector<double> y = conv3x3(x, h, w, ci, 4 * feat, wgt, b);
            std::vector<double> want(got.size());
            for (int yy = 0; yy < h; ++yy)
                for (int xx = 0; xx < w; ++xx)
                    for (int co = 0; co < 4 * feat; ++co) {
                        const int ch = co / 4, dy = (co / 2) % 2, dx = co % 2;
                        want[((size_t)(2 * yy + dy) * 2 * w + 2 * xx + dx) * feat + ch] =
                            y[((size_t)yy * w + xx) * 4 * feat + co];
                    }
            CHECK(cnt.ok(close("conv3x3_shuffle2 " + std::to_string(ci) + "->" + std::to_string(feat) +
                                   "x4 at " + std::to_string(h) + "x" + std::to_string(w),
                               want, got, tol)));
        }
    }

    // the token GEMM and every epilogue the forward uses, at the reference's
    // toy shape and at the checkpoint's width
    {
        const int C = arch->embed;
        const int shapes[3][3] = {{13, 6, 5}, {37, C, C}, {300, C, 3 * C}};
        for (auto &sh : shapes) {
            const int rows = sh[0], ci = sh[1], co = sh[2];
            std::vector<float> x = seq((size_t)rows * ci, 0.2f), wgt = seq((size_t)co * ci, 2.4f),
                               b = seq(co, 3.1f), res = seq((size_t)rows * co, 0.9f),
                               lw = seq(co, 0.7f), lb = seq(co, 0.8f);
            for (float &v : wgt) v /= std::sqrt((float)ci);
            std::vector<double> lin((size_t)rows * co);
            for (int r = 0; r < rows; ++r)
                for (int o = 0; o < co; ++o) {
                    double acc = b[o];
                    for (int i = 0; i < ci; ++i) acc += (double)x[(size_t)r * ci + i] * wgt[(size_t)o * ci + i];
                    lin[(size_t)r * co + o] = acc;
                }
            for (int epi = 0; epi <= 5; ++epi) {
                if ((epi == 3 || epi == 4) && co > 192) continue;
                std::vector<double> want = lin;
                for (int r = 0; r < rows; ++r) {
                    double *v = &want[(size_t)r * co];
                    if (epi == 1) for (int o = 0; o < co; ++o) v[o] = gelu(v[o]);
                    if (epi == 2) for (int o = 0; o < co; ++o) v[o] += res[(size_t)r * co + o];
                    if (epi == 5) for (int o = 0; o < co; ++o) v[o] = v[o] < 0 ? 0.2 * v[o] : v[o];
                    if (epi == 3 || epi == 4) {
                        double m = 0, q = 0;
                        for (int o = 0; o < co; ++o) m += v[o];
                        m /= co;
                        for (int o = 0; o < co; ++o) q += (v[o] - m) * (v[o] - m);
                        const double rs = 1.0 / std::sqrt(q / co + 1e-5);
                        for (int o = 0; o < co; ++o)
                            v[o] = (v[o] - m) * rs * lw[o] + lb[o] + (epi == 4 ? res[(size_t)r * co + o] : 0.0);
                    }
                }
                std::vector<float> got((size_t)rows * co);
                CHECK(s2s_test_linear(rows, ci, co, x.data(), wgt.data(), b.data(), epi,
                                      (epi == 2 || epi == 4) ? res.data() : nullptr, lw.data(), lb.data(),
                                      0.2f, got.data()));
                static const char *names[6] = {"store", "gelu", "residual", "layernorm",
                                               "residual + layernorm", "leaky_relu"};
                CHECK(cnt.ok(close("linear " + std::to_string(rows) + "x" + std::to_string(ci) + "->" +
                                       std::to_string(co) + " " + names[epi],
                                   want, got, tol)));
            }
        }
    }

    // the standalone channel LayerNorm (the final norm)
    {
        for (int c : {8, arch->embed}) {
            if (c % 4 || c > 256) continue;
            const int hw = 77;
            std::vector<float> x = seq((size_t)hw * c, 0.6f), w = seq(c, 0.7f), b = seq(c, 0.8f),
                               got((size_t)hw * c);
            CHECK(s2s_test_ln_residual(hw, c, x.data(), w.data(), b.data(), nullptr, got.data()));
            std::vector<double> want(got.size());
            for (int p = 0; p < hw; ++p) {
                double m = 0, q = 0;
                for (int i = 0; i < c; ++i) m += x[(size_t)p * c + i];
                m /= c;
                for (int i = 0; i < c; ++i) q += (x[(size_t)p * c + i] - m) * (x[(size_t)p * c + i] - m);
                const double rs = 1.0 / std::sqrt(q / c + 1e-5);
                for (int i = 0; i < c; ++i) want[(size_t)p * c + i] = (x[(size_t)p * c + i] - m) * rs * w[i] + b[i];
            }
            CHECK(cnt.ok(close("layernorm c=" + std::to_string(c), want, got, tol)));
        }
    }

    // the window index and mask-band maps, exactly (reference src/plan.rs:72-108)
    {
        const int cases[3][3] = {{16, 16, 0}, {16, 16, 4}, {16, 24, 4}};
        for (auto &cs : cases) {
            const int hp = cs[0], wp = cs[1], shift = cs[2], nww = wp / 8, n = (hp / 8) * nww * 64;
            std::vector<int32_t> yx(2 * n);
            std::vector<uint8_t> reg(2 * n);
            CHECK(s2s_test_window_map(hp, wp, 8, shift, yx.data(), reg.data()));
            auto band = [&](int a, int p) { return a + 8 < p ? 0 : (a + shift < p ? 1 : 2); };
            for (int i = 0; i < n; ++i) {
                const int wi = i / 64, t = i % 64, a = (wi / nww) * 8 + t / 8, b = (wi % nww) * 8 + t % 8;
                if (yx[2 * i] != (a + shift) % hp || yx[2 * i + 1] != (b + shift) % wp ||
                    reg[2 * i] != band(a, hp) || reg[2 * i + 1] != band(b, wp))
                    return fail("window map " + std::to_string(hp) + "x" + std::to_string(wp) + " shift " +
                                std::to_string(shift) + ": token " + std::to_string(i) + " differs");
            }
            ++cnt.checks;
        }
    }

    // window attention, plane-order qkv, at a toy head shape and the
    // checkpoint's own (reference: (2, 2) and (wt.heads, wt.head_dim))
    {
        const int shapes[2][2] = {{2, 2}, {wheads, whd}};
        for (auto &sh : shapes) {
            const int heads = sh[0], hd = sh[1], c = heads * hd, hp = 16, wp = 24;
            if (c % 4 || hd > 32) continue;
            for (int shift : {0, 4}) {
                std::vector<float> qkv = seq((size_t)hp * wp * 3 * c, 0.45f), ls(heads),
                                   cpb = seq((size_t)64 * 64 * heads, 0.05f), got((size_t)hp * wp * c);
                for (int h = 0; h < heads; ++h) ls[h] = 1.3f - 0.2f * h;
                CHECK(s2s_test_attention(hp, wp, 8, heads, hd, shift, qkv.data(), ls.data(), cpb.data(),
                                         got.data()));
                CHECK(cnt.ok(close("attention " + std::to_string(heads) + "x" + std::to_string(hd) +
                                       " shift=" + std::to_string(shift),
                                   attention(qkv, hp, wp, heads, hd, shift, ls, cpb), got, tol)));
            }
        }
    }

    // the block's qkv projection and window attention as the forward runs
    // them for 6 heads of 30 (one fused kernel): x -> x W^T + b -> attention
    if (qkv_attn_fused(wheads, whd)) {
        const int heads = wheads, hd = whd, c = heads * hd, hp = 16, wp = 24;
        const size_t P = (size_t)hp * wp;
        for (int shift : {0, 4}) {
            std::vector<float> x = seq(P * c, 0.35f), w = seq((size_t)3 * c * c, 0.6f),
                               b = seq((size_t)3 * c, 1.7f), ls(heads),
                               cpb = seq((size_t)64 * 64 * heads, 0.15f), got(P * c);
            for (float &v : w) v /= std::sqrt((float)c);
            for (int i = c; i < 2 * c; ++i) b[i] = 0.f;  // k has no bias
            for (int h = 0; h < heads; ++h) ls[h] = 1.3f - 0.2f * h;
            std::vector<float> qkv(P * 3 * c);
            for (size_t p = 0; p < P; ++p)
                for (int o = 0; o < 3 * c; ++o) {
                    double a = b[o];
                    for (int i = 0; i < c; ++i) a += (double)w[(size_t)o * c + i] * x[p * c + i];
                    qkv[p * 3 * c + o] = (float)a;
                }
            CHECK(s2s_test_block_attention(hp, wp, heads, hd, shift, x.data(), w.data(), b.data(),
                                           ls.data(), cpb.data(), got.data()));
            CHECK(cnt.ok(close("qkv + attention (fused) " + std::to_string(heads) + "x" +
                                   std::to_string(hd) + " shift=" + std::to_string(shift),
                               attention(qkv, hp, wp, heads, hd, shift, ls, cpb), got, tol)));
        }
    }

    // the qkv GEMM's shifted-window gather into the unit layout, exactly: an
    // identity weight carries each pixel's index into every q/k/v column
    {
        const int heads = wheads, hd = whd, c = heads * hd, hp = 16, wp = 24, HG = (heads + 1) / 2;
        if (qkv_unit_layout(heads, hd, c)) {
            for (int shift : {0, 4}) {
                std::vector<float> x((size_t)hp * wp * c), w((size_t)3 * c * c, 0.f), b((size_t)3 * c, 0.f);
                for (size_t p = 0; p < (size_t)hp * wp; ++p)
                    for (int i = 0; i < c; ++i) x[p * c + i] = (float)p;
                for (int s = 0; s < 3; ++s)
                    for (int i = 0; i < c; ++i) w[((size_t)s * c + i) * c + i] = 1.f;
                std::vector<float> unit(attn_unit_floats(hp, wp, heads, hd));
                CHECK(s2s_test_qkv_windows(hp, wp, heads, hd, shift, x.data(), w.data(), b.data(),
                                           unit.data(), unit.size()));
                const int nww = wp / 8, nw = (hp / 8) * nww, RS = attn_unit_stride(hd);
                for (int wi = 0; wi < nw; ++wi)
                    for (int t = 0; t < 64; ++t) {
                        const float want = (float)(((wi / nww * 8 + t / 8 + shift) % hp) * wp +
                                                   (wi % nww * 8 + t % 8 + shift) % wp);
                        for (int h = 0; h < heads; ++h)
                            for (int sg = 0; sg < 3; ++sg)
                                for (int d = 0; d < hd; ++d)
                                    if (unit[(((size_t)wi * HG + h / 2) * 64 + t) * RS +
                                             (2 * sg + (h & 1)) * hd + d] != want)
                                        return fail("qkv window gather shift " + std::to_string(shift) +
                                                    ": window " + std::to_string(wi) + " token " +
                                                    std::to_string(t) + " differs");
                    }
                ++cnt.checks;
            }
        }
    }

    // the checkpoint's CPB tables: the device MLP against the converter's
    // cpb_pre, where the set carries both
    if (tensors) {
        int blocks = 0;
        for (int s = 0; s < arch->n_stages && s < S2S_MAX_STAGES; ++s)
            for (int b = 0; b < arch->depths[s]; ++b) {
                const std::string p = "layers." + std::to_string(s) + ".residual_group.blocks." +
                                      std::to_string(b) + ".attn.";
                const s2s_tensor *w0 = find(tensors, n_tensors, p + "cpb_mlp.0.weight"),
                                 *b0 = find(tensors, n_tensors, p + "cpb_mlp.0.bias"),
                                 *w2 = find(tensors, n_tensors, p + "cpb_mlp.2.weight"),
                                 *pre = find(tensors, n_tensors, p + "cpb_pre");
                if (!w0 || !b0 || !w2 || !pre) continue;
                std::vector<float> got((size_t)64 * 64 * wheads);
                CHECK(s2s_test_cpb_table(arch->window, wheads, w0->data, b0->data, w2->data, got.data()));
                std::vector<double> want(pre->data, pre->data + got.size());
                CHECK(close("cpb table of " + p, want, got, tol));
                ++blocks;
            }
        if (blocks) ++cnt.checks;
    }

    printf("hip selftest: %d kernel/shape pairs checked against their CPU definitions\n", cnt.checks);
    fflush(stdout);
    return 0;
}
