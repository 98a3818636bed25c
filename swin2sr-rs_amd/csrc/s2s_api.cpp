// s2s_api.cpp - the C ABI of include/swin2sr_hip.h: context, weight upload,
// per-size buffer planning, the forward graph, the event profiler and the
// per-op test entry points.
//
// The graph is the reference's (src/gpu.rs:462-583 / src/cpu.rs:1437-1685) on
// channel-last planes, with the elementwise ops folded into the GEMM epilogues:
//   block (src/gpu.rs:485-522):  qkv = x Wqkv^T + [qb|0|vb]
//                                o   = window_attention(qkv, shift)
//                                x1  = x  + LN1(o Wp^T + bp)
//                                x2  = x1 + LN2(gelu(x1 W1^T + b1) W2^T + b2)
//   RSTB close (:526-528):       x   = conv1x1(conv3x3(blocks(x))) + x
//   frame (:471-542):            conv_first -> patch_embed(1x1 + LN) -> stages
//                                -> LN -> conv_after_body + conv_first output
//   classical head (:601-623):   conv+lrelu(0.01), (conv3x3 + shuffle2) per
//                                octave, conv_last + finish (denormalise, crop)
#include <hip/hip_runtime.h>
#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "swin2sr_hip.h"
#include "s2s_kernels.h"

namespace {

thread_local std::string g_err;

int fail(const std::string &m) {
    g_err = m;
    return -1;
}

std::string hip_msg(const char *what, hipError_t e) {
    std::string m = std::string(what) + " failed: " + hipGetErrorName(e) + " (" +
                    hipGetErrorString(e) + ")";
    // run_with_fallback retries only on "out of memory" (reference
    // src/main.rs:655-662); make sure the phrase is there for the OOM code.
    if (e == hipErrorOutOfMemory && m.find("out of memory") == std::string::npos)
        m += ": out of memory";
    return m;
}

#define HIPCHK(what, expr)                                        \
    do {                                                          \
        hipError_t e_ = (expr);                                   \
        if (e_ != hipSuccess) return fail(hip_msg((what), e_));   \
    } while (0)

int round4(int v) { return (v + 3) / 4 * 4; }

struct BlockW {
    float *wqkv = nullptr, *bqkv = nullptr, *wproj = nullptr, *bproj = nullptr;
    float *n1w = nullptr, *n1b = nullptr, *n2w = nullptr, *n2b = nullptr;
    float *w1 = nullptr, *b1 = nullptr, *w2 = nullptr, *b2 = nullptr;
    float *ls = nullptr, *cpbt = nullptr;
};

struct StageW {
    std::vector<BlockW> blocks;
    // the stage close: its 3x3 conv with the 1x1 patch_embed conv folded in
    float *conv_w = nullptr, *conv_b = nullptr;
};

struct ProfKey {
    std::string name;
    unsigned g[3], b[3];
    bool operator<(const ProfKey &o) const {
        return std::tie(name, g[0], g[1], g[2], b[0], b[1], b[2]) <
               std::tie(o.name, o.g[0], o.g[1], o.g[2], o.b[0], o.b[1], o.b[2]);
    }
};
struct ProfRow {
    int calls = 0;
    double ms = 0.0;
};
struct Pending {
    ProfKey key;
    hipEvent_t e0, e1;
};

}  // namespace

int s2s_fail(const char *msg) { return fail(msg ? msg : "unknown error"); }

// One device buffer of a forward's plan: where its pointer goes, its size in
// floats, its name (for error messages) and whether the kernels reach it only
// through per-task resources or 64-bit pointers ("wide": any size), as opposed
// to a 32-bit offset from its base (below the 2 GiB resource limit).
struct BufSpec {
    float **dst;
    size_t floats;
    const char *what;
    bool wide;
};

// Device allocations of one lifetime (weights, body plan, image plan) and
// their total size.
struct AllocList {
    std::vector<void *> ptrs;
    std::vector<size_t> floats;  // each allocation's size, in the plan's order
    uint64_t bytes = 0;
};

// Whether the buffers of `v` fit the allocations of `l` one for one (the
// same plan layout, each no larger than what is held).
static bool fits_in(const AllocList &l, const std::vector<BufSpec> &v) {
    if (l.floats.size() != v.size()) return false;
    for (size_t i = 0; i < v.size(); ++i)
        if (std::max<size_t>(v[i].floats, 1) > l.floats[i]) return false;
    return true;
}


struct s2s_ctx {
    s2s_arch arch{};
    int c = 0, hd = 0, hidden = 0, feat = 0, octaves = 0;
    bool cbu_wino = false;  // conv_before_upsample as Winograd (weights U [36][F][C])
    int device = 0;
    hipStream_t stream = nullptr;
    AllocList weight_allocs;
    uint64_t uploaded = 0;

    float *cf_b = nullptr;                   // conv_first's bias [C]
    // conv_first and patch_embed's 1x1 folded into it, for k_embed: weights
    // [2][9][4][C], the folded bias [C], patch_embed's LayerNorm
    float *emb_w = nullptr, *pe_b = nullptr, *pe_nw = nullptr, *pe_nb = nullptr;
    float *norm_w = nullptr, *norm_b = nullptr;
    float *cab_w = nullptr, *cab_b = nullptr;  // conv_after_body (body_conv_weights)
    std::vector<StageW> stages;
    float *cbu_w = nullptr, *cbu_b = nullptr;  // conv_before_upsample [F][9*C] or [36][F][C]
    std::vector<float *> up_w, up_b;           // octave convs, shuffle-permuted [4F][9*F]
    float *last_w = nullptr, *last_b = nullptr;  // conv_last [9][F][3]
    // pixelshuffle: the last octave's conv and conv_last composed (k_up_last):
    // interior weights [25][F][12] and bias [12], edge variants [4][12][25][F]
    // and [4][12]; the last octave's plane is then never materialised
    bool fuse_last = false;
    float *ul_w = nullptr, *ul_b = nullptr, *ul_we = nullptr, *ul_be = nullptr;
    // with two or more octaves the last two compose as well (a 5x5 conv GEMM
    // to 48 outputs, stored through pixel_shuffle(4)): [48][25F], [48],
    // [4][48][25][F], [4][48]; the last two octaves' planes are never made
    bool fuse2 = false;
    bool up2_wino = false;  // the composed 5x5 conv as Winograd F(2x2,5x5) (u2_w [36][48][F])
    float *u2_w = nullptr, *u2_b = nullptr, *u2_we = nullptr, *u2_be = nullptr;
    int fused_octaves() const { return fuse2 ? 2 : (fuse_last ? 1 : 0); }
    // pixelshuffle_aux: conv_bicubic [F][9*4], conv_aux [4][9*F] (its fourth
    // output row zero, so the conv writes channel 3 of the aux plane as 0),
    // conv_after_aux [F][9*4]
    float *ax_w = nullptr, *ax_b = nullptr;
    // the compressed head's bicubic branch through conv_last, composed:
    // [4][25][3][4], [4][3]
    float *bl_w = nullptr, *bl_b = nullptr;
    float *caa_w = nullptr, *caa_b = nullptr;
    // pixelshuffledirect: upsample.0 [3*s*s][9*C]
    float *psd_w = nullptr, *psd_b = nullptr;
    // nearest+conv: conv_up1, conv_up2, conv_hr [F][9*F]
    float *nu1_w = nullptr, *nu1_b = nullptr, *nu2_w = nullptr, *nu2_b = nullptr;
    float *hr_w = nullptr, *hr_b = nullptr;

    // buffers planned for one padded plane (hp, wp)
    int bhp = 0, bwp = 0;
    AllocList body_allocs;
    float *cur = nullptr, *wk = nullptr, *body = nullptr;
    float *qkv = nullptr, *o = nullptr, *hid = nullptr;
    // head / io buffers planned for one image (h, w)
    int ih = 0, iw = 0;
    AllocList head_allocs;
    float *in_dev = nullptr, *in4 = nullptr, *out_dev = nullptr;
    std::vector<float *> fplanes;  // the head's feature planes
    // pixelshuffle_aux: aux conv output [P][4], its planar image [3][P], the
    // bicubic input [(hp*s)*(wp*s)][4] and its conv (= the last head plane)
    float *aux4 = nullptr, *auxp = nullptr, *bic4 = nullptr;
    // the host path's pinned staging copies of the input and output images
    float *pin_in = nullptr, *pin_out = nullptr;
    size_t pin_in_floats = 0, pin_out_floats = 0;
    // a cap on the bytes of the body and image plans together (0 = none):
    // SWIN2SR_HIP_ALLOC_LIMIT at s2s_create, or s2s_set_alloc_limit
    uint64_t alloc_limit = 0;

    // The device forward as HIP graphs: the second time a call comes (image
    // size, input and output pointers, buffer plan) among the last few seen,
    // its launches are captured into a graph, which is replayed whenever that
    // call comes again (about 1.6 us less per kernel than stream launches on
    // MI355X); a call seen once launches eagerly. Up to kGraphs graphs are
    // kept, the least recently used replaced first (so a tiled image's few
    // crop shapes, or a lane's alternating images, each keep theirs). Off
    // while profiling, for s2s_forward_device_noalloc, while a caller captures
    // the context's stream itself, and with SWIN2SR_HIP_GRAPHS=0.
    struct GraphKey {
        int h = 0, w = 0;
        const float *in = nullptr;
        const float *out = nullptr;
        uint64_t plan = 0;
        bool operator==(const GraphKey &k) const {
            return h == k.h && w == k.w && in == k.in && out == k.out && plan == k.plan;
        }
    };
    static constexpr size_t kGraphs = 4;
    struct GraphEntry {
        GraphKey key;
        hipGraphExec_t exec = nullptr;
        uint64_t used = 0;
    };
    bool graphs = true;
    uint64_t plan_gen = 1;  // bumped whenever a plan's buffers change
    std::vector<GraphKey> seen;       // calls seen once, oldest first (at most kGraphs)
    std::vector<GraphEntry> gcache;   // captured calls (at most kGraphs)
    uint64_t gtick = 0;
    void drop_graph();
    void drop_graph_entry(size_t i);

    bool prof = false;
    std::string prof_only;  // bracket only launches of this name ("" = all)
    std::vector<Pending> pending;
    std::vector<hipEvent_t> free_events;
    std::map<ProfKey, ProfRow> rows;

    std::vector<float> aux_host;

    // A second execution lane for s2s_forward_device_batch: its own stream,
    // buffer plans and graphs over this context's weights (made on first
    // use; it owns none of the weights), and the events that fork it off this
    // context's stream and join it back.
    s2s_ctx *lane = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
    int make_lane();

    ~s2s_ctx();
    int upload(const std::vector<float> &host, float **dev);
    int alloc(AllocList &list, size_t floats, float **dev, const char *what, bool wide = false,
              bool planned = false);
    // qkv buffer floats: the plane layout, or the attention unit layout; it
    // also holds the body's Winograd convs' transform-domain products (36
    // planes of wino_tiles(hp, wp) tiles x C) between blocks, and the head's
    size_t qkv_floats(int hp, int wp) const {
        const size_t plane = (size_t)hp * wp * 3 * c;
        const size_t q = qkv_unit_layout(arch.heads, hd, c)
                             ? std::max(plane, attn_unit_floats(hp, wp, arch.heads, hd))
                             : plane;
        const size_t qb = wino_body(c) ? std::max(q, WINO_POS * wino_tiles(hp, wp) * c) : q;
        // the x4 head's Winograd 5x5 conv: V and M (stride F) at most the
        // whole plane's tiles
        return up2_wino ? std::max(qb, WINO_POS * wino5_tiles(hp, wp) * feat) : qb;
    }
    // MLP hidden buffer floats; it also holds conv_before_upsample's Winograd
    // products (36 planes of wino_tiles(hp, wp) tiles x F) in the head
    size_t hid_floats(int hp, int wp) const {
        const size_t h = (size_t)hp * wp * hidden;
        return cbu_wino ? std::max(h, WINO_POS * wino_tiles(hp, wp) * feat) : h;
    }
    // The buffers of a padded plane's body, and of an image's head (with the
    // host path's device copies of the input and output when `io`); `bind`
    // points the specs at the context's members (else dst is null).
    void body_specs(int hp, int wp, bool bind, std::vector<BufSpec> &v);
    void image_specs(int h, int w, bool io, bool bind, std::vector<BufSpec> &v);
    int plan_body(int hp, int wp);
    int plan_image(int h, int w);
    // whether the current plan is for (h, w)
    bool plan_fits(int h, int w) const {
        const int hp = (h / arch.window + 1) * arch.window, wp = (w / arch.window + 1) * arch.window;
        return h == ih && w == iw && hp == bhp && wp == bwp;
    }
    // whether the held buffers can serve a plane / an image of this size
    // without allocating (within the allocation limit, if one is set)
    bool held_within_limit() const {
        return !alloc_limit || body_allocs.bytes + head_allocs.bytes <= alloc_limit;
    }
    bool body_reusable(int hp, int wp) {
        if (!bhp || !held_within_limit()) return false;
        std::vector<BufSpec> v;
        body_specs(hp, wp, false, v);
        return fits_in(body_allocs, v);
    }
    bool image_reusable(int h, int w) {
        if (!ih || !held_within_limit()) return false;
        std::vector<BufSpec> v;
        image_specs(h, w, true, false, v);
        return fits_in(head_allocs, v);
    }
    // whether plan_image(h, w) would allocate (or synchronise the stream)
    bool plan_allocates(int h, int w) {
        const int hp = (h / arch.window + 1) * arch.window, wp = (w / arch.window + 1) * arch.window;
        return !plan_fits(h, w) && !(image_reusable(h, w) && body_reusable(hp, wp));
    }
    int stage_buffers(int h, int w);
    hipEvent_t event();
    int drain();
    template <typename F>
    int run(const char *name, dim3 grid, dim3 block, F &&launch);
    int gemm(const char *name, const GemmArgs &g, int aload, int epi);
    int block_fwd(const BlockW &b, int hp, int wp, int shift, const float *x_in, float *x_out);
    int stage_fwd(int s, int hp, int wp, const float *x_in, float *x_out);
    int conv_body(const char *name, const float *in, int H, int W, const float *u,
                  const float *bias, const float *res, float *out);
    int conv_wino(const char *name, const float *in, int H, int W, int ci, int co,
                  const float *u, const float *bias, const float *res, float *mbuf, float *out,
                  int lrelu, float slope);
    int forward_device(int h, int w, const float *d_in, float *d_out, bool may_graph = true);
    int forward_launches(int h, int w, const float *d_in, float *d_out);
    int head(int h, int w, float *d_out);
};

namespace {

// Whether a weight of N rows of K multiplied under epilogue `epi` is stored
// in k_bsgemm's register order (bs_pack_weights), and its floats as stored.
// The x4 head's K = 64 Winograd products keep rows: their GEMM is bound by
// HBM, not by its start, and measured 10% slower with packed weights.
bool bs_packs(int N, int K, int epi) { return K != 64 && bs_weight_floats(N, K, epi) > 0; }
size_t weight_floats(int N, int K, int epi) {
    return bs_packs(N, K, epi) ? bs_weight_floats(N, K, epi) : (size_t)N * K;
}

// nb weights of rows [N][K], one after another, as the GEMM that multiplies
// by them reads them: in register order when k_bsgemm takes the shape (each
// batch weight_floats apart), else unchanged.
std::vector<float> gemm_weights(const std::vector<float> &rows, int nb, int N, int K, int epi) {
    if (!bs_packs(N, K, epi)) return rows;
    const size_t pf = bs_weight_floats(N, K, epi);
    std::vector<float> out(pf * nb);
    for (int b = 0; b < nb; ++b)
        bs_pack_weights(rows.data() + (size_t)b * N * K, K, N, K, epi, out.data() + b * pf);
    return out;
}

void free_list(AllocList &l) {
    for (void *p : l.ptrs) (void)hipFree(p);
    l.ptrs.clear();
    l.floats.clear();
    l.bytes = 0;
}


}  // namespace

// An exec graph's last launch may still be queued on the stream: HIP does not
// promise to defer the destruction of an exec graph in flight, so the stream
// drains first (this runs only when a graph is evicted or a plan changes).
void s2s_ctx::drop_graph_entry(size_t i) {
    if (stream) (void)hipStreamSynchronize(stream);
    (void)hipGraphExecDestroy(gcache[i].exec);
    gcache.erase(gcache.begin() + (long)i);
}

void s2s_ctx::drop_graph() {
    if (!gcache.empty() && stream) (void)hipStreamSynchronize(stream);
    for (GraphEntry &e : gcache) (void)hipGraphExecDestroy(e.exec);
    gcache.clear();
    seen.clear();
}

s2s_ctx::~s2s_ctx() {
    delete lane;  // (its own stream drained, its plans freed; the weights are ours)
    if (fork_ev) (void)hipEventDestroy(fork_ev);
    if (join_ev) (void)hipEventDestroy(join_ev);
    if (stream) (void)hipStreamSynchronize(stream);
    drop_graph();
    for (auto &p : pending) {
        (void)hipEventDestroy(p.e0);
        (void)hipEventDestroy(p.e1);
    }
    for (auto e : free_events) (void)hipEventDestroy(e);
    free_list(head_allocs);
    free_list(body_allocs);
    free_list(weight_allocs);
    if (pin_in) (void)hipHostFree(pin_in);
    if (pin_out) (void)hipHostFree(pin_out);
    if (stream) (void)hipStreamDestroy(stream);
}

// The lane: a copy of this context's weights, architecture and switches, with
// every resource the context owns taken out (the weights' allocation list,
// plans, staging, graphs, profiler state) and a stream of its own.
int s2s_ctx::make_lane() {
    if (lane) return 0;
    s2s_ctx *L = new s2s_ctx(*this);
    L->weight_allocs = AllocList{};
    L->body_allocs = AllocList{};
    L->head_allocs = AllocList{};
    L->bhp = L->bwp = L->ih = L->iw = 0;
    L->cur = L->wk = L->body = L->qkv = L->o = L->hid = nullptr;
    L->in_dev = L->in4 = L->out_dev = nullptr;
    L->fplanes.clear();
    L->aux4 = L->auxp = L->bic4 = nullptr;
    L->pin_in = L->pin_out = nullptr;
    L->pin_in_floats = L->pin_out_floats = 0;
    L->plan_gen = 1;
    L->seen.clear();
    L->gcache.clear();
    L->gtick = 0;
    L->prof = false;
    L->prof_only.clear();
    L->pending.clear();
    L->free_events.clear();
    L->rows.clear();
    L->aux_host.clear();
    L->lane = nullptr;
    L->fork_ev = L->join_ev = nullptr;
    L->stream = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&L->stream, hipStreamNonBlocking);
    if (e == hipSuccess && !fork_ev) e = hipEventCreateWithFlags(&fork_ev, hipEventDisableTiming);
    if (e == hipSuccess && !join_ev) e = hipEventCreateWithFlags(&join_ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        delete L;
        return fail(hip_msg("s2s_forward_device_batch: the second lane", e));
    }
    lane = L;
    return 0;
}

int s2s_ctx::upload(const std::vector<float> &host, float **dev) {
    float *p = nullptr;
    HIPCHK("hipMalloc(weights)", hipMalloc(&p, std::max<size_t>(host.size(), 1) * sizeof(float)));
    weight_allocs.ptrs.push_back(p);
    HIPCHK("hipMemcpy(weights)",
           hipMemcpy(p, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice));
    uploaded += host.size() * sizeof(float);
    *dev = p;
    return 0;
}

// The kernels address buffers with raw buffer loads and stores: 32-bit byte
// offsets from a base, with the resource's bounds check as the out-of-range
// mechanism. The large buffers (qkv, the head's feature planes, the output)
// are only reached through resources based per task, tile or window, or
// through 64-bit pointers, so they may have any size ("wide"); the others
// (planes of C or 2C channels, read whole as GEMM operands) must stay below
// the resource limit, which holds for every plane up to 1.49 M pixels, above
// the crate's GPU_MAX_PLANE_PIXELS (65535 x 16, src/backend.rs:230). A plane
// that would pass it is refused like an allocation failure: the message says
// "out of memory", which is what the crate's tile-halving retry keys on
// (src/main.rs:655-662), and a smaller tile then fits. `planned` buffers (the
// body and image plans) also count against the context's allocation limit.
static constexpr size_t kMaxBufferBytes = 0x7fff0000u;  // BUF_MAX_BYTES of the kernels

// The workspace of the allocation-free forward (s2s_forward_device_noalloc):
// one static array per GPU, S2S_NOALLOC_SCRATCH_BYTES long, which every
// process that loads the library holds on each GPU it runs on until it ends.
// Host code never uses the name `scratch` as an address (on the host it is a
// stand-in for the device symbol): each device's address comes from
// hipGetSymbolAddress at s2s_create, with that device current, and is kept in
// g_scratch[device].
#define S2S_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)
static __device__ __align__(256) unsigned char scratch[S2S_NOALLOC_SCRATCH_BYTES];
static constexpr int kMaxDevices = 64;
static void *g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;
// The workspace's last user on each device: every eager allocation-free call
// makes its stream wait for this event before its first launch and records it
// after its last, under g_ws_mu[device], so calls from different contexts
// (different streams) take the workspace one after the other instead of
// racing on it. Created with the address, at s2s_create (an event, not an
// allocation on the call's path).
static hipEvent_t g_ws_event[kMaxDevices];
static std::mutex g_ws_mu[kMaxDevices];

// Looks up the current device's address of `scratch`, and creates its
// ordering event, once per device.
static int scratch_init(int dev) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (dev < 0 || dev >= kMaxDevices) return fail("device index out of range for the workspace table");
    if (g_scratch[dev]) return 0;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return fail(hip_msg("hipGetSymbolAddress(scratch)", e == hipSuccess ? hipErrorInvalidSymbol : e));
    }
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(hip_msg("hipEventCreate(workspace order)", e));
    }
    g_ws_event[dev] = ev;
    g_scratch[dev] = p;
    return 0;
}

int s2s_ctx::alloc(AllocList &list, size_t floats, float **dev, const char *what, bool wide,
                   bool planned) {
    const size_t bytes = std::max<size_t>(floats, 1) * sizeof(float);
    if (!wide && floats > kMaxBufferBytes / sizeof(float))
        return fail(std::string("hipMalloc(") + what + ", " + std::to_string(floats * sizeof(float)) +
                    " bytes) refused: above the 2 GiB limit of the kernels' 32-bit offsets into "
                    "this buffer (out of memory for one pass; tile the image)");
    if (planned && alloc_limit &&
        body_allocs.bytes + head_allocs.bytes + bytes > alloc_limit)
        return fail(std::string("hipMalloc(") + what + ", " + std::to_string(bytes) +
                    " bytes) refused: the context's allocation limit of " +
                    std::to_string(alloc_limit) + " bytes would be passed (" +
                    std::to_string(body_allocs.bytes + head_allocs.bytes) +
                    " already planned): out of memory");
    float *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(std::string("hipMalloc(") + what + ", " +
                    std::to_string(floats * sizeof(float)) + " bytes) failed: " +
                    hipGetErrorString(e) + (e == hipErrorOutOfMemory ? " (out of memory)" : ""));
    }
    list.ptrs.push_back(p);
    list.floats.push_back(std::max<size_t>(floats, 1));
    list.bytes += bytes;
    *dev = p;
    return 0;
}

// Body buffers for a padded plane: the activation, the in-stage working copy,
// conv_first's output (the body skip), qkv (also the Winograd convs'
// transform-domain products), the attention output (also the final norm's
// output) and the MLP hidden layer.
void s2s_ctx::body_specs(int hp, int wp, bool bind, std::vector<BufSpec> &v) {
    const size_t P = (size_t)hp * wp;
    auto d = [&](float **p) { return bind ? p : nullptr; };
    v.push_back({d(&cur), P * c, "cur", false});
    v.push_back({d(&wk), P * c, "work", false});
    v.push_back({d(&body), P * c, "body", false});
    v.push_back({d(&qkv), qkv_floats(hp, wp), "qkv", true});
    v.push_back({d(&o), P * c, "attn", false});
    v.push_back({d(&hid), hid_floats(hp, wp), "mlp", false});
}

// Image buffers: the padded input (and, for the host path, device copies of
// the input and the output), the head's feature planes - one per octave that
// is not composed away for the pixel-shuffle heads, P, 4P, 16P, 16P for
// nearest+conv, none for pixelshuffledirect - and the compressed head's aux
// and bicubic planes.
void s2s_ctx::image_specs(int h, int w, bool io, bool bind, std::vector<BufSpec> &v) {
    const int win = arch.window, s = arch.scale;
    const size_t P = (size_t)((h / win + 1) * win) * ((w / win + 1) * win);
    auto d = [&](float **p) { return bind ? p : nullptr; };
    if (io) {
        v.push_back({d(&in_dev), (size_t)3 * h * w, "input", false});
        v.push_back({d(&out_dev), (size_t)3 * h * s * w * s, "output", true});
    }
    v.push_back({d(&in4), P * 4, "padded input", false});
    std::vector<size_t> planes;
    if (arch.upsampler == S2S_PIXELSHUFFLE || arch.upsampler == S2S_PIXELSHUFFLE_AUX) {
        size_t px = P;
        for (int o_ = 0; o_ <= octaves - fused_octaves(); ++o_, px *= 4) planes.push_back(px);
    } else if (arch.upsampler == S2S_NEAREST_CONV) {
        planes = {P, 4 * P, 16 * P, 16 * P};
    }
    if (bind) fplanes.assign(planes.size(), nullptr);
    for (size_t i = 0; i < planes.size(); ++i)
        v.push_back({bind ? &fplanes[i] : nullptr, planes[i] * feat, "head plane", true});
    if (arch.upsampler == S2S_PIXELSHUFFLE_AUX) {
        v.push_back({d(&aux4), P * 4, "aux conv", false});
        v.push_back({d(&auxp), P * 3, "aux image", false});
        v.push_back({d(&bic4), P * s * s * 4, "bicubic input", true});
    }
}

// Reused while the plane size repeats (reference Gpu::forward rebuilds Acts
// only on a size change, src/gpu.rs:741-750), and also when a new plane's
// buffers each fit the ones held (a smaller tile after a larger one, or the
// same number of pixels transposed, as a tiled image alternates): the
// buffers stay where they are, nothing is freed or allocated and the stream
// is not synchronised. A plane that needs more is planned afresh at its own
// size.
int s2s_ctx::plan_body(int hp, int wp) {
    if (hp == bhp && wp == bwp) return 0;
    if (body_reusable(hp, wp)) {
        bhp = hp;
        bwp = wp;
        return 0;
    }
    if (stream) HIPCHK("hipStreamSynchronize", hipStreamSynchronize(stream));
    drop_graph();
    ++plan_gen;
    free_list(body_allocs);
    bhp = bwp = 0;
    std::vector<BufSpec> v;
    body_specs(hp, wp, true, v);
    for (const BufSpec &b : v)
        if (alloc(body_allocs, b.floats, b.dst, b.what, b.wide, true)) {
            free_list(body_allocs);
            return -1;
        }
    bhp = hp;
    bwp = wp;
    return 0;
}

int s2s_ctx::plan_image(int h, int w) {
    const int win = arch.window;
    const int hp = (h / win + 1) * win, wp = (w / win + 1) * win;
    if (plan_fits(h, w)) return 0;
    if (image_reusable(h, w) && body_reusable(hp, wp)) {
        bhp = hp;
        bwp = wp;
        ih = h;
        iw = w;
        return 0;
    }
    if (stream) HIPCHK("hipStreamSynchronize", hipStreamSynchronize(stream));
    drop_graph();
    ++plan_gen;
    // the image's buffers go first, so a size change never holds the old
    // image plan and the new body plan at once
    free_list(head_allocs);
    fplanes.clear();
    ih = iw = 0;
    if (plan_body(hp, wp)) return -1;
    std::vector<BufSpec> v;
    image_specs(h, w, true, true, v);
    for (const BufSpec &b : v)
        if (alloc(head_allocs, b.floats, b.dst, b.what, b.wide, true)) {
            free_list(head_allocs);
            fplanes.clear();
            return -1;
        }
    ih = h;
    iw = w;
    return 0;
}

// The host path's pinned staging images for an h x w image (page-locked, so
// the copies run as DMA at the link's rate and the host-side copies overlap
// them). Only s2s_forward uses them. Kept while an image fits them (pinning
// a fresh buffer costs milliseconds, and a tiled image alternates sizes).
int s2s_ctx::stage_buffers(int h, int w) {
    const int s = arch.scale;
    const size_t nin = (size_t)3 * h * w, nout = nin * s * s;
    if (pin_in && nin <= pin_in_floats && nout <= pin_out_floats) return 0;
    if (pin_in) (void)hipHostFree(pin_in);
    if (pin_out) (void)hipHostFree(pin_out);
    pin_in = pin_out = nullptr;
    pin_in_floats = pin_out_floats = 0;
    hipError_t e = hipHostMalloc((void **)&pin_in, nin * sizeof(float));
    if (e == hipSuccess) e = hipHostMalloc((void **)&pin_out, nout * sizeof(float));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (pin_in) (void)hipHostFree(pin_in);
        pin_in = nullptr;
        return fail(hip_msg("hipHostMalloc(staging)", e));
    }
    pin_in_floats = nin;
    pin_out_floats = nout;
    return 0;
}

hipEvent_t s2s_ctx::event() {
    if (!free_events.empty()) {
        hipEvent_t e = free_events.back();
        free_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

int s2s_ctx::drain() {
    if (pending.empty()) return 0;
    HIPCHK("hipStreamSynchronize", hipStreamSynchronize(stream));
    for (auto &p : pending) {
        float ms = 0.f;
        HIPCHK("hipEventElapsedTime", hipEventElapsedTime(&ms, p.e0, p.e1));
        ProfRow &r = rows[p.key];
        r.calls += 1;
        r.ms += ms;
        free_events.push_back(p.e0);
        free_events.push_back(p.e1);
    }
    pending.clear();
    return 0;
}

// One launch, bracketed by an event pair when profiling (reference
// Cuda::run, src/cuda.rs:109-140).
template <typename F>
int s2s_ctx::run(const char *name, dim3 grid, dim3 block, F &&launch) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    const bool timed = prof && (prof_only.empty() || prof_only == name);
    if (timed) {
        e0 = event();
        e1 = event();
        if (!e0 || !e1) return fail("hipEventCreate failed");
        HIPCHK("hipEventRecord", hipEventRecord(e0, stream));
    }
    hipError_t e = launch();
    if (e != hipSuccess) return fail(hip_msg(name, e));
    if (timed) {
        HIPCHK("hipEventRecord", hipEventRecord(e1, stream));
        pending.push_back(Pending{ProfKey{name, {grid.x, grid.y, grid.z}, {block.x, block.y, block.z}},
                                  e0, e1});
        if (pending.size() > 4096) return drain();
    }
    return 0;
}

int s2s_ctx::gemm(const char *name, const GemmArgs &g, int aload, int epi) {
    dim3 grid, block;
    gemm_geometry(g, aload, epi, &grid, &block);
    return run(name, grid, block, [&] { return launch_gemm(g, aload, epi, stream); });
}

namespace {

GemmArgs rows_gemm(const float *A, int lda, const float *B, int ldb, const float *bias, float *out,
                   int ldo, int M, int N, int K) {
    GemmArgs g{};
    g.A = A;
    g.lda = lda;
    g.B = B;
    g.ldb = ldb;
    g.bias = bias;
    g.out = out;
    g.ldo = ldo;
    g.M = M;
    g.N = N;
    g.K = K;
    return g;
}

GemmArgs conv_gemm(const float *in, int H, int W, int cin, const float *wt, const float *bias,
                   float *out, int ldo, int N) {
    GemmArgs g{};
    g.A = in;
    g.H = H;
    g.W = W;
    g.cin = cin;
    g.B = wt;
    g.ldb = 9 * cin;
    g.bias = bias;
    g.out = out;
    g.ldo = ldo;
    g.M = H * W;
    g.N = N;
    g.K = 9 * cin;
    return g;
}

// A 3x3 conv (F -> F) of the nearest-2x upsampling of the H x W plane `in`
// into the 2H x 2W plane `out`, as the ALOAD_SUB2 GEMM over its four phases
// (weights from subpixel_weights).
GemmArgs sub2_gemm(const float *in, int H, int W, int F, const float *wt, const float *bias,
                   float *out) {
    GemmArgs g = conv_gemm(in, H, W, F, wt, bias, out, F, F);
    g.ldb = 4 * F;
    g.K = 4 * F;
    return g;
}

}  // namespace

// One post-norm Swin V2 block (reference src/gpu.rs:485-522), x_in -> x_out
// (x_out may equal x_in).
int s2s_ctx::block_fwd(const BlockW &b, int hp, int wp, int shift, const float *x_in,
                       float *x_out) {
    const int P = hp * wp;
    GemmArgs g;
    if (qkv_attn_fused(arch.heads, hd)) {
        // 6 heads of 30: the qkv projection and the window attention as one
        // kernel (the head pair's q, k, v never leave the CU)
        QkvAttnArgs a{};
        a.x = x_in;
        a.w = b.wqkv;
        a.bias = b.bqkv;
        a.cpbt = b.cpbt;
        a.logit_scale = b.ls;
        a.out = o;
        a.hp = hp;
        a.wp = wp;
        a.shift = shift;
        if (run("qkv_window_attention", dim3(qkv_attention_grid(hp, wp)), dim3(256),
                [&] { return launch_qkv_attention(a, stream, nullptr); }))
            return -1;
    } else {
        // qkv straight into the window attention's unit layout where its
        // kernel takes the head shape, else the plane layout [P][3c]
        const int epi = qkv_gemm_args(x_in, b.wqkv, b.bqkv, qkv, hp, wp, shift, arch.heads, hd, &g);
        g.b_packed = bs_packs(3 * c, c, EPI_STORE);
        if (gemm("qkv", g, ALOAD_ROWS, epi)) return -1;
        const AttnArgs a = window_attn_args(qkv, b.cpbt, b.ls, o, hp, wp, shift, arch.heads, hd);
        const unsigned ag = attention_grid(a);
        if (run("window_attention", dim3(ag), dim3(256),
                [&] { return launch_attention(a, stream, nullptr); }))
            return -1;
    }

    g = rows_gemm(o, c, b.wproj, c, b.bproj, x_out, c, P, c, c);
    g.b_packed = bs_packs(c, c, EPI_LN_RES);
    g.res = x_in;
    g.ldr = c;
    g.ln_w = b.n1w;
    g.ln_b = b.n1b;
    if (gemm("proj_ln_res", g, ALOAD_ROWS, EPI_LN_RES)) return -1;

    g = rows_gemm(x_out, c, b.w1, c, b.b1, hid, hidden, P, hidden, c);
    g.b_packed = bs_packs(hidden, c, EPI_GELU);
    if (gemm("fc1_gelu", g, ALOAD_ROWS, EPI_GELU)) return -1;

    g = rows_gemm(hid, hidden, b.w2, hidden, b.b2, x_out, c, P, c, hidden);
    g.b_packed = bs_packs(c, hidden, EPI_LN_RES);
    g.res = x_out;
    g.ldr = c;
    g.ln_w = b.n2w;
    g.ln_b = b.n2b;
    return gemm("fc2_ln_res", g, ALOAD_ROWS, EPI_LN_RES);
}

// One RSTB stage (reference src/gpu.rs:481-529): blocks, conv3x3, 1x1, + x_in.
int s2s_ctx::stage_fwd(int s, int hp, int wp, const float *x_in, float *x_out) {
    const StageW &st = stages[s];
    const float *src = x_in;
    for (size_t bi = 0; bi < st.blocks.size(); ++bi) {
        const int shift = (bi % 2 == 1) ? arch.window / 2 : 0;
        if (block_fwd(st.blocks[bi], hp, wp, shift, src, wk)) return -1;
        src = wk;
    }
    // The stage close (reference src/gpu.rs:526-528: the 3x3 conv, the 1x1
    // patch_embed conv, the stage's residual) as one conv: the two
    // convolutions are folded into one at upload, and the residual is added
    // by the output transform element by element, so it may write over x_in
    // (the transform-domain GEMM has read all of its input before that).
    return conv_body("conv3x3_stage", src, hp, wp, st.conv_w, st.conv_b, x_in, x_out);
}

// A C -> C 3x3 conv of the body (the stage close, conv_after_body), + bias +
// residual. For the released widths (wino_body) as Winograd F(4x4,3x3): the
// input transform V of every 4x4 output tile into the qkv buffer (free
// between blocks), the 36 transform-position GEMMs M = V U^T as one batched
// launch of the weight-stationary kernel (M over V in place), then the output
// transform with the bias and the residual: 4x fewer multiplies than the
// direct conv, the same map to fp32 rounding (the reference's own CUDA backend
// runs these convs as Winograd with 6x6 tiles, src/gpu.rs:161-181). Other
// widths: the direct implicit-GEMM conv with the residual as its epilogue.
int s2s_ctx::conv_body(const char *name, const float *in, int H, int W, const float *u,
                       const float *bias, const float *res, float *out) {
    if (!wino_body(c)) {
        // the epilogue adds the residual element by element; only a conv that
        // reads the plane it writes (a stage with no blocks) goes through
        // `o` (free between blocks)
        float *dst = in == out ? o : out;
        GemmArgs g = conv_gemm(in, H, W, c, u, bias, dst, c, c);
        g.res = res;
        g.ldr = c;
        if (gemm(name, g, ALOAD_IM2COL, EPI_RES)) return -1;
        if (dst != out) {
            const hipError_t e = hipMemcpyAsync(out, dst, (size_t)H * W * c * 4, hipMemcpyDeviceToDevice, stream);
            if (e != hipSuccess) return fail(hip_msg("hipMemcpyAsync(stage)", e));
        }
        return 0;
    }
    return conv_wino(name, in, H, W, c, c, u, bias, res, qkv, out, 0, 0.f);
}

// A 3x3 conv ci -> co as Winograd F(4x4,3x3) on the qkv buffer (free outside
// the blocks): the input transform of `in` [H*W][ci] into V there, the 36
// transform-position GEMMs into M at `mbuf` (M over V in place when mbuf is
// the qkv buffer, which takes co == ci: every GEMM task then writes exactly
// the rows it has read), then the output transform with the bias, the
// residual `res` if set and LeakyReLU(slope) if `lrelu`, into out [H*W][co].
int s2s_ctx::conv_wino(const char *name, const float *in, int H, int W, int ci, int co,
                       const float *u, const float *bias, const float *res, float *mbuf,
                       float *out, int lrelu, float slope) {
    if (mbuf == qkv && co != ci) return fail(std::string(name) + ": in-place Winograd needs co == ci");
    const int T = (int)wino_tiles(H, W);
    const std::string in_name = std::string(name) + "_in", out_name = std::string(name) + "_out";
    if (run(in_name.c_str(), dim3(wino_in_grid(H, W, ci)), dim3(256),
            [&] { return launch_wino_in(in, ci, qkv, H, W, ci, stream); }))
        return -1;
    GemmArgs g = rows_gemm(qkv, ci, u, ci, nullptr, mbuf, co, T, co, ci);
    g.nb = WINO_POS;
    g.a_bstride = (size_t)T * ci;
    g.o_bstride = (size_t)T * co;
    g.b_packed = bs_packs(co, ci, EPI_STORE);
    g.b_bstride = weight_floats(co, ci, EPI_STORE);
    if (gemm(name, g, ALOAD_ROWS, EPI_STORE)) return -1;
    return run(out_name.c_str(), dim3(wino_out_grid(H, W, co)), dim3(256), [&] {
        return launch_wino_out(mbuf, bias, res, res ? co : 0, out, co, H, W, co, lrelu, slope, stream);
    });
}

int s2s_ctx::forward_device(int h, int w, const float *d_in, float *d_out, bool may_graph) {
    const int win = arch.window;
    if (h < win || w < win)
        return fail(std::to_string(h) + "x" + std::to_string(w) + " is smaller than one " +
                    std::to_string(win) + "x" + std::to_string(win) +
                    " window. The reference pads to the NEXT window multiple by concatenating "
                    "the image with its own mirror, which for an image shorter than a window "
                    "falls through to a different padding rule this engine does not implement.");
    // A caller capturing the context's stream into a graph of its own gets
    // the launches recorded there. A new buffer plan cannot be made then:
    // planning synchronises the stream and allocates, which would end the
    // caller's capture in an error; the call is refused instead and the
    // context stays as it was.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIPCHK("hipStreamIsCapturing", hipStreamIsCapturing(stream, &cs));
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (capturing && plan_allocates(h, w))
        return fail("s2s_forward_device: the context's stream is being captured into a graph and a " +
                    std::to_string(h) + "x" + std::to_string(w) +
                    " image needs a new buffer plan (planning allocates and synchronises the "
                    "stream, which a capture does not allow); run one call of this size before "
                    "capturing, or capture s2s_forward_device_noalloc");
    if (plan_image(h, w)) return -1;
    if (capturing) {
        // the launches go into the caller's graph; no profiler events there
        const bool p = prof;
        prof = false;
        const int rc = forward_launches(h, w, d_in, d_out);
        prof = p;
        return rc;
    }
    if (!may_graph || prof || !graphs) return forward_launches(h, w, d_in, d_out);
    const GraphKey k{h, w, d_in, d_out, plan_gen};
    for (GraphEntry &e : gcache)
        if (e.key == k) {
            e.used = ++gtick;
            HIPCHK("hipGraphLaunch", hipGraphLaunch(e.exec, stream));
            return 0;
        }
    const auto sk = std::find(seen.begin(), seen.end(), k);
    if (sk == seen.end()) {
        if (seen.size() >= kGraphs) seen.erase(seen.begin());
        seen.push_back(k);
        return forward_launches(h, w, d_in, d_out);
    }
    // the call's second sighting: capture its launches (nothing runs while
    // capturing), then launch the graph; the least recently used graph makes
    // room
    seen.erase(sk);
    if (gcache.size() >= kGraphs) {
        size_t lru = 0;
        for (size_t i = 1; i < gcache.size(); ++i)
            if (gcache[i].used < gcache[lru].used) lru = i;
        drop_graph_entry(lru);
    }
    HIPCHK("hipStreamBeginCapture", hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    const int rc = forward_launches(h, w, d_in, d_out);
    hipGraph_t gr = nullptr;
    const hipError_t ec = hipStreamEndCapture(stream, &gr);
    if (rc || ec != hipSuccess) {
        if (gr) (void)hipGraphDestroy(gr);
        (void)hipGetLastError();
        return rc ? rc : fail(hip_msg("hipStreamEndCapture", ec));
    }
    hipGraphExec_t ex = nullptr;
    const hipError_t ei = hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0);
    (void)hipGraphDestroy(gr);
    if (ei != hipSuccess) {
        // no graphs on this context from now on: the same launches, eagerly
        graphs = false;
        (void)hipGetLastError();
        drop_graph();
        return forward_launches(h, w, d_in, d_out);
    }
    gcache.push_back(GraphEntry{k, ex, ++gtick});
    HIPCHK("hipGraphLaunch", hipGraphLaunch(ex, stream));
    return 0;
}

// The device forward's launches on the context's stream (reference
// src/gpu.rs:462-583): pad, embed, the stages, norm, conv_after_body, head.
int s2s_ctx::forward_launches(int h, int w, const float *d_in, float *d_out) {
    const int win = arch.window;
    const int hp = (h / win + 1) * win, wp = (w / win + 1) * win;
    const int P = hp * wp;
    if (run("pad_input", dim3((P + 255) / 256), dim3(256),
            [&] { return launch_pad_input(d_in, in4, h, w, hp, wp, stream); }))
        return -1;
    // conv_first -> body, and patch_embed (1x1 conv + LayerNorm) on it -> cur,
    // the 1x1 folded into a second set of conv_first weights: one pass
    if (run("embed", dim3((P + 63) / 64), dim3(256), [&] {
            return launch_embed(in4, emb_w, cf_b, pe_b, pe_nw, pe_nb, body, cur, hp, wp, c, stream);
        }))
        return -1;
    for (int s = 0; s < arch.n_stages; ++s)
        if (stage_fwd(s, hp, wp, cur, cur)) return -1;
    if (run("layernorm", dim3((P + 15) / 16), dim3(256),
            [&] { return launch_layernorm(cur, norm_w, norm_b, nullptr, o, P, c, stream); }))
        return -1;
    // (the final norm lands in the attention output's plane, free after the blocks)
    if (conv_body("conv_after_body", o, hp, wp, cab_w, cab_b, body, cur)) return -1;
    return head(h, w, d_out);
}

// The reconstruction heads (reference src/gpu.rs:591-733 / src/cpu.rs:1701-1880)
// from `cur`, the body's output, into the planar, denormalised, cropped output.
int s2s_ctx::head(int h, int w, float *d_out) {
    const int win = arch.window, s = arch.scale;
    const int hp = (h / win + 1) * win, wp = (w / win + 1) * win;
    const int oh = h * s, ow = w * s;
    GemmArgs g{};
    // conv_before_upsample + LeakyReLU(0.01) into the first feature plane
    auto before_upsample = [&]() -> int {
        if (cbu_wino)
            return conv_wino("conv_before_upsample", cur, hp, wp, c, feat, cbu_w, cbu_b, nullptr,
                             hid, fplanes[0], 1, 0.01f);
        g = conv_gemm(cur, hp, wp, c, cbu_w, cbu_b, fplanes[0], feat, feat);
        g.slope = 0.01f;
        return gemm("conv_before_upsample", g, ALOAD_IM2COL, EPI_LRELU);
    };
    auto last = [&](const float *f, int H, int W) {
        return run("conv_last_finish", conv_last_grid(oh, ow), dim3(256), [&] {
            return launch_conv_last_finish(f, last_w, last_b, d_out, H, W, feat, oh, ow,
                                           arch.img_range, arch.mean, stream);
        });
    };
    switch (arch.upsampler) {
    case S2S_PIXELSHUFFLE:
    case S2S_PIXELSHUFFLE_AUX: {
        const bool aux = arch.upsampler == S2S_PIXELSHUFFLE_AUX;
        if (before_upsample()) return -1;
        if (aux) {
            // the aux image and its conv back to features (reference
            // network_swin2sr.py:948-958)
            // conv_aux (feat -> 3) on the VALU with the aux image's finish: the
            // conv's output to the aux plane (its channel 3 zero, which
            // conv_after_aux reads as zero padding) and the denormalised aux
            // image (an N = 3 GEMM would use 3 of its 64 columns)
            if (run("conv_aux", conv_last_grid(hp, wp), dim3(256), [&] {
                    return launch_conv_aux(fplanes[0], ax_w, ax_b, aux4, auxp, hp, wp, feat,
                                           arch.img_range, arch.mean, stream);
                }))
                return -1;
            g = conv_gemm(aux4, hp, wp, 4, caa_w, caa_b, fplanes[0], feat, feat);
            g.slope = 0.01f;
            if (gemm("conv_after_aux", g, ALOAD_IM2COL, EPI_LRELU)) return -1;
        }
        int H = hp, W = wp;
        for (int oc = 0; oc < octaves - fused_octaves(); ++oc) {
            g = conv_gemm(fplanes[oc], H, W, feat, up_w[oc], up_b[oc], fplanes[oc + 1], 0, 4 * feat);
            g.feat = feat;
            const std::string nm = "conv3x3_shuffle2_o" + std::to_string(oc);
            if (gemm(nm.c_str(), g, ALOAD_IM2COL, EPI_SHUFFLE)) return -1;
            H *= 2;
            W *= 2;
        }
        // the composed tail (the last octaves and conv_last, with the finish),
        // then for the compressed head its bicubic branch through conv_last,
        // composed, added into the finished image
        auto composed = [&]() -> int {
            if (fuse2 && up2_wino) {
                // the last two octaves and conv_last: one 5x5 conv to 48 channels
                // as Winograd F(2x2,5x5) over the pixels whose outputs survive the
                // crop (V, then M over it at a row stride of F, in the qkv
                // buffer), stored through pixel_shuffle(4), denormalised and
                // cropped by the output transform; then the input row 0 / column 0
                // outputs recomputed
                const int Ho = std::min(H, (oh + 3) / 4), Wo = std::min(W, (ow + 3) / 4);
                const int T = (int)wino5_tiles(Ho, Wo);
                const float *src = fplanes[octaves - 2];
                if (run("up2_last_in", dim3(wino5_in_grid(Ho, Wo, feat)), dim3(256),
                        [&] { return launch_wino5_in(src, feat, qkv, H, W, Ho, Wo, feat, stream); }))
                    return -1;
                g = rows_gemm(qkv, feat, u2_w, feat, nullptr, qkv, feat, T, 48, feat);
                g.nb = WINO_POS;
                g.a_bstride = g.o_bstride = (size_t)T * feat;
                g.b_packed = bs_packs(48, feat, EPI_STORE);
                g.b_bstride = weight_floats(48, feat, EPI_STORE);
                if (gemm("up2_last", g, ALOAD_ROWS, EPI_STORE)) return -1;
                if (run("up2_last_out", dim3(wino5_finish_grid(Ho, Wo)), dim3(256), [&] {
                        return launch_wino5_finish(qkv, feat, u2_b, d_out, Ho, Wo, oh, ow, arch.img_range,
                                                   arch.mean, stream);
                    }))
                    return -1;
                const int nb = (ow + 3) / 4 + (oh + 3) / 4 - 1;
                return run("up2_last_edge", dim3(nb), dim3(256), [&] {
                    return launch_up2_last_edge(src, u2_we, u2_be, d_out, H, W, feat, oh, ow,
                                                arch.img_range, arch.mean, stream);
                });
            }
            if (fuse2) {
                // the last two octaves and conv_last: one 5x5 conv to 48 channels
                // stored through pixel_shuffle(4), denormalised and cropped, then
                // the input row 0 / column 0 outputs recomputed
                g = conv_gemm(fplanes[octaves - 2], H, W, feat, u2_w, u2_b, d_out, 0, 48);
                g.ldb = 25 * feat;
                g.K = 25 * feat;
                // only the rows whose outputs survive the crop (the loader still
                // reads the rows below them as the footprint needs)
                g.M = std::min(H, (oh + 3) / 4) * W;
                g.scale = 4;
                g.oh = oh;
                g.ow = ow;
                g.img_range = arch.img_range;
                for (int i = 0; i < 3; ++i) g.mean[i] = arch.mean[i];
                if (gemm("up2_last", g, ALOAD_IM2COL5, EPI_SHUFFLE_FINISH)) return -1;
                const int nb = (ow + 3) / 4 + (oh + 3) / 4 - 1;
                return run("up2_last_edge", dim3(nb), dim3(256), [&] {
                    return launch_up2_last_edge(fplanes[octaves - 2], u2_we, u2_be, d_out, H, W, feat,
                                                oh, ow, arch.img_range, arch.mean, stream);
                });
            }
            return run("up_last", up_last_grid(oh, ow), dim3(256), [&] {
                return launch_up_last(fplanes[octaves - 1], ul_w, ul_b, ul_we, ul_be, d_out, H, W,
                                      feat, oh, ow, arch.img_range, arch.mean, stream);
            });
        };
        if (!fuse_last) return last(fplanes[octaves], H, W);
        if (composed()) return -1;
        if (!aux) return 0;
        // the compressed head's bicubic branch: the padded input resampled to
        // the output grid, then through conv_last o conv_bicubic into the image
        const int qh = hp * s, qw = wp * s, Q = qh * qw;
        if (run("bicubic", dim3((Q + 255) / 256), dim3(256),
                [&] { return launch_bicubic4(in4, bic4, hp, wp, qh, qw, stream); }))
            return -1;
        return run("bic_last_add", dim3((ow + 63) / 64, (oh + 3) / 4), dim3(256), [&] {
            return launch_bic_last_add(bic4, qh, qw, bl_w, bl_b, d_out, oh, ow, arch.img_range, stream);
        });
    }
    case S2S_PIXELSHUFFLE_DIRECT: {
        // one conv to 3*s^2 channels, stored through pixel_shuffle(s) straight
        // into the denormalised, cropped output
        g = conv_gemm(cur, hp, wp, c, psd_w, psd_b, d_out, 0, 3 * s * s);
        g.scale = s;
        g.oh = oh;
        g.ow = ow;
        g.img_range = arch.img_range;
        for (int i = 0; i < 3; ++i) g.mean[i] = arch.mean[i];
        return gemm("conv_shuffle_finish", g, ALOAD_IM2COL, EPI_SHUFFLE_FINISH);
    }
    case S2S_NEAREST_CONV: {
        if (before_upsample()) return -1;
        // two nearest-2x steps, each read by the next conv's operand loader
        g = sub2_gemm(fplanes[0], hp, wp, feat, nu1_w, nu1_b, fplanes[1]);
        g.slope = 0.2f;
        if (gemm("conv_up1", g, ALOAD_SUB2, EPI_LRELU)) return -1;
        g = sub2_gemm(fplanes[1], 2 * hp, 2 * wp, feat, nu2_w, nu2_b, fplanes[2]);
        g.slope = 0.2f;
        if (gemm("conv_up2", g, ALOAD_SUB2, EPI_LRELU)) return -1;
        g = conv_gemm(fplanes[2], 4 * hp, 4 * wp, feat, hr_w, hr_b, fplanes[3], feat, feat);
        g.slope = 0.2f;
        if (gemm("conv_hr", g, ALOAD_IM2COL, EPI_LRELU)) return -1;
        return last(fplanes[3], 4 * hp, 4 * wp);
    }
    default:
        return fail("unknown upsampler " + std::to_string(arch.upsampler));
    }
}

// ---------------------------------------------------------------------------
// Weight set: lookup, validation and re-layout.
// ---------------------------------------------------------------------------

namespace {

struct TensorSet {
    const s2s_tensor *t;
    size_t n;
    const s2s_tensor *find(const std::string &name) const {
        for (size_t i = 0; i < n; ++i)
            if (t[i].name && name == t[i].name) return &t[i];
        return nullptr;
    }
    size_t numel(const s2s_tensor *x) const {
        size_t v = 1;
        for (int d = 0; d < x->ndim; ++d) v *= (size_t)x->shape[d];
        return v;
    }
    // The tensor, or an error naming it and the shape expected (the reference
    // refuses a checkpoint the same way, src/weights.rs:142-235).
    int get(const std::string &name, std::vector<int64_t> shape, const s2s_tensor **out) const {
        const s2s_tensor *x = find(name);
        if (!x) return fail("weight `" + name + "` is missing from the tensor set");
        bool ok = x->ndim == (int)shape.size();
        for (int d = 0; ok && d < x->ndim; ++d) ok = x->shape[d] == shape[d];
        if (!ok) {
            std::string got, want;
            for (int d = 0; d < x->ndim; ++d) got += (d ? "," : "") + std::to_string(x->shape[d]);
            for (size_t d = 0; d < shape.size(); ++d)
                want += (d ? "," : "") + std::to_string(shape[d]);
            return fail("weight `" + name + "` is [" + got + "], the architecture implies [" +
                        want + "]");
        }
        *out = x;
        return 0;
    }
};

std::vector<float> vec_of(const s2s_tensor *x, size_t n) { return std::vector<float>(x->data, x->data + n); }

// [co][ci][3][3] -> [co][tap][ci_pad] (tap = ky*3+kx, ci zero-padded to 4)
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

// A body C -> C conv's weights [co][ci][3][3] as its kernels read them: the
// Winograd transform [36][C][C] for the released widths (in the batched
// GEMM's order), else the implicit GEMM's [co][tap][ci_pad4].
std::vector<float> body_conv_weights(const float *w, int C) {
    if (!wino_body(C)) return conv_relayout(w, C, C, nullptr);
    std::vector<float> u((size_t)WINO_POS * C * C);
    wino_weights(w, C, C, u.data());
    return gemm_weights(u, WINO_POS, C, C, EPI_STORE);
}

// co = 4ch + 2dy + dx  ->  row (2dy+dx)*feat + ch, so a 32-column tile of the
// GEMM is 32 consecutive output channels of one sub-pixel (coalesced stores).
std::vector<int> shuffle_perm(int feat) {
    std::vector<int> p(4 * feat);
    for (int co = 0; co < 4 * feat; ++co) p[co] = (co % 4) * feat + co / 4;
    return p;
}

// The last pixel-shuffle octave (conv3x3 F -> 4F, PixelShuffle(2); Wo, bo) and
// conv_last (conv3x3 F -> 3; Wl, bl) composed into one linear map from the
// octave's input plane (reference src/gpu.rs:601-623). Output (2y + sy,
// 2x + sx), channel k (s = (2 sy + sx) * 3 + k) reads conv_last's tap (ky, kx)
// at shuffled position (2y + sy + ky - 1, ...), which is channel
// 4c + 2 dy' + dx' of the octave's pixel (y + fy, ...), u = sy + ky - 1,
// fy = floor(u / 2), dy' = u - 2 fy; that in turn reads input pixel
// (y + fy + ty - 1, ...): offsets -2..2, a 5 x 5 footprint. Variant (ey, ex)
// drops conv_last's kernel row 0 for sy = 0 (ey) and column 0 for sx = 0 (ex):
// the taps that fall on conv_last's zero padding at output row 0 / column 0.
// Accumulated in double, rounded once. wi [25][F][12], bi [12] (variant 0);
// we [4][12][25][F], be [4][12].
void compose_up_last(const float *Wo, const float *bo, const float *Wl, const float *bl, int F,
                     std::vector<float> &wi, std::vector<float> &bi, std::vector<float> &we,
                     std::vector<float> &be) {
    std::vector<double> W((size_t)4 * 12 * 25 * F, 0.0), B(4 * 12, 0.0);
    for (int var = 0; var < 4; ++var) {
        const bool ey = var >> 1, ex = var & 1;
        for (int sy = 0; sy < 2; ++sy)
            for (int sx = 0; sx < 2; ++sx)
                for (int k = 0; k < 3; ++k) {
                    const int s = (2 * sy + sx) * 3 + k;
                    double b = bl[k];
                    double *w = &W[(size_t)(var * 12 + s) * 25 * F];
                    for (int ky = 0; ky < 3; ++ky)
                        for (int kx = 0; kx < 3; ++kx) {
                            if ((ey && sy == 0 && ky == 0) || (ex && sx == 0 && kx == 0)) continue;
                            const int u = sy + ky - 1, v = sx + kx - 1;
                            const int fy = (u + 2) / 2 - 1, fx = (v + 2) / 2 - 1;
                            const int dyp = u - 2 * fy, dxp = v - 2 * fx;
                            for (int c = 0; c < F; ++c) {
                                const double wl = Wl[(((size_t)k * F + c) * 3 + ky) * 3 + kx];
                                const int co = 4 * c + 2 * dyp + dxp;
                                b += wl * bo[co];
                                for (int ci = 0; ci < F; ++ci)
                                    for (int ty = 0; ty < 3; ++ty)
                                        for (int tx = 0; tx < 3; ++tx) {
                                            const int tap = (fy + ty + 1) * 5 + (fx + tx + 1);
                                            w[(size_t)tap * F + ci] +=
                                                wl * Wo[(((size_t)co * F + ci) * 3 + ty) * 3 + tx];
                                        }
                            }
                        }
                    B[var * 12 + s] = b;
                }
    }
    wi.assign((size_t)25 * F * 12, 0.f);
    for (int s = 0; s < 12; ++s)
        for (int tap = 0; tap < 25; ++tap)
            for (int ci = 0; ci < F; ++ci)
                wi[((size_t)tap * F + ci) * 12 + s] = (float)W[((size_t)s * 25 + tap) * F + ci];
    bi.assign(B.begin(), B.begin() + 12);
    we.assign(W.begin(), W.end());
    be.assign(B.begin(), B.end());
}

// The last two octaves and conv_last composed, from the composition of the
// last one with conv_last (compose_up_last's edge variants ue [4][12][25][F],
// ub [4][12]) and the octave before it (Wo, bo: conv3x3 F -> 4F,
// PixelShuffle(2)). Output (4y + a, 4x + b), channel k is up_last's output
// s12 = (2(a%2) + b%2)*3 + k at pixel (y1, x1) = (2y + a/2, 2x + b/2) of the
// middle plane Z1, which reads Z1 at (y1 + oy, x1 + ox), |oy|, |ox| <= 2;
// Z1 there is channel 4c + 2((a/2 + oy) & 1) + ((b/2 + ox) & 1) of the octave's
// pixel (y + floor((a/2 + oy)/2), ...), which reads input pixel offsets
// floor((a/2 + oy)/2) + ty - 1 in -2..2: a 5 x 5 footprint again. Variant
// (ey, ex) is for input row 0 / column 0: up_last's own variant there (its
// pixel y1 = 0 with sub-row 0, i.e. a = 0) and the Z1 positions above / left of
// the plane dropped (o1's zero padding). Output s48 = k*16 + a*4 + b (torch's
// pixel_shuffle(4) channel order); w48 and b48 [4][48] in
// double, rounded once; wg [48][25*F] (variant 0, the GEMM's [n][k] with
// k = tap*F + ci) and bg [48]; w48 [4][48][25][F]; with u5, variant 0 also as
// Winograd F(2x2,5x5) weights [36][48][F] (wino5_weights).
void compose_up2_last(const std::vector<float> &ue, const std::vector<float> &ub, const float *Wo,
                      const float *bo, int F, std::vector<float> &wg, std::vector<float> &bg,
                      std::vector<float> &w48, std::vector<float> &b48, std::vector<float> *u5) {
    const size_t kk = (size_t)25 * F;
    std::vector<double> W((size_t)4 * 48 * kk, 0.0), B(4 * 48, 0.0);
    for (int var = 0; var < 4; ++var) {
        const bool ey = var >> 1, ex = var & 1;
        for (int k = 0; k < 3; ++k)
            for (int a = 0; a < 4; ++a)
                for (int b = 0; b < 4; ++b) {
                    const int s48 = k * 16 + a * 4 + b;
                    const int s12 = (2 * (a % 2) + b % 2) * 3 + k;
                    const int vu = 2 * (ey && a == 0) + (ex && b == 0);
                    const float *uw = &ue[(size_t)(vu * 12 + s12) * kk];
                    double bias = ub[vu * 12 + s12];
                    double *w = &W[(size_t)(var * 48 + s48) * kk];
                    for (int oy = -2; oy <= 2; ++oy)
                        for (int ox = -2; ox <= 2; ++ox) {
                            const int zy = a / 2 + oy, zx = b / 2 + ox;
                            if ((ey && zy < 0) || (ex && zx < 0)) continue;
                            const int fy = zy >= 0 ? zy / 2 : -((1 - zy) / 2);
                            const int fx = zx >= 0 ? zx / 2 : -((1 - zx) / 2);
                            const int dyp = zy - 2 * fy, dxp = zx - 2 * fx;
                            const int ut = (oy + 2) * 5 + (ox + 2);
                            for (int c = 0; c < F; ++c) {
                                const double u = uw[(size_t)ut * F + c];
                                if (u == 0.0) continue;
                                const int co = 4 * c + 2 * dyp + dxp;
                                bias += u * bo[co];
                                for (int ci = 0; ci < F; ++ci)
                                    for (int ty = 0; ty < 3; ++ty)
                                        for (int tx = 0; tx < 3; ++tx) {
                                            const int tap = (fy + ty + 1) * 5 + (fx + tx + 1);
                                            w[(size_t)tap * F + ci] +=
                                                u * Wo[(((size_t)co * F + ci) * 3 + ty) * 3 + tx];
                                        }
                            }
                        }
                    B[var * 48 + s48] = bias;
                }
    }
    wg.assign((size_t)48 * kk, 0.f);
    for (size_t i = 0; i < (size_t)48 * kk; ++i) wg[i] = (float)W[i];
    if (u5) {
        // variant 0 as Winograd F(2x2,5x5) weights, from the double sums
        u5->assign((size_t)WINO_POS * 48 * round4(F), 0.f);
        wino5_weights(W.data(), 48, F, u5->data());
    }
    bg.assign(B.begin(), B.begin() + 48);
    w48.assign(W.begin(), W.end());
    b48.assign(B.begin(), B.end());
}

// The compressed head's bicubic branch through conv_last (reference
// src/gpu.rs:678-730: conv_last(octaves(x) + conv_bicubic(B))): conv_last
// (Wl [3][F][3][3], without its bias, which the octaves' composition carries)
// after conv_bicubic (Wb [F][3][3][3], bb [F]) as one 5x5 conv of the bicubic
// image B: output (Y, X), channel k reads conv_last's tap (ky, kx) at
// (Y + ky - 1, X + kx - 1) of conv_bicubic's output, which reads B at a further
// (dy - 1, dx - 1): tap t = (ky + dy) * 5 + (kx + dx) of the 5x5 footprint.
// Variant (ey, ex) drops conv_last's kernel row 0 (ey) / column 0 (ex) - with
// the bias they carry - for output row 0 / column 0, where those taps read
// conv_last's zero padding. Accumulated in double, rounded once: w [4][25][3][4]
// (input channel 3 zero), b [4][3].
void compose_bic_last(const float *Wb, const float *bb, const float *Wl, int F,
                      std::vector<float> &w, std::vector<float> &b) {
    std::vector<double> W((size_t)4 * 25 * 3 * 4, 0.0), B(12, 0.0);
    for (int var = 0; var < 4; ++var) {
        const bool ey = var >> 1, ex = var & 1;
        for (int k = 0; k < 3; ++k)
            for (int ky = 0; ky < 3; ++ky)
                for (int kx = 0; kx < 3; ++kx) {
                    if ((ey && ky == 0) || (ex && kx == 0)) continue;
                    for (int f = 0; f < F; ++f) {
                        const double wl = Wl[(((size_t)k * F + f) * 3 + ky) * 3 + kx];
                        B[var * 3 + k] += wl * bb[f];
                        for (int c = 0; c < 3; ++c)
                            for (int dy = 0; dy < 3; ++dy)
                                for (int dx = 0; dx < 3; ++dx) {
                                    const int t = (ky + dy) * 5 + (kx + dx);
                                    W[((size_t)(var * 25 + t) * 3 + k) * 4 + c] +=
                                        wl * Wb[(((size_t)f * 3 + c) * 3 + dy) * 3 + dx];
                                }
                    }
                }
    }
    w.assign(W.begin(), W.end());
    b.assign(B.begin(), B.end());
}

// The head's feature width: conv_before_upsample's output channels.
int head_feat_of(const TensorSet &ts, int C, int *F) {
    const s2s_tensor *cb = ts.find("conv_before_upsample.0.weight");
    if (!cb || cb->ndim != 4 || cb->shape[0] <= 0 || cb->shape[0] % 32 != 0)
        return fail("weight `conv_before_upsample.0.weight` is missing or not [feat][C][3][3] "
                    "with feat a multiple of 32");
    if (ts.get("conv_before_upsample.0.weight", {cb->shape[0], C, 3, 3}, &cb)) return -1;
    *F = (int)cb->shape[0];
    return 0;
}

int octaves_of(int scale) {
    int oct = 0;
    while ((1 << oct) < scale) ++oct;
    return oct;
}

// The bytes s2s_create uploads for an architecture and tensor set: the
// weights as the kernels read them (re-laid-out, padded to 4 input channels,
// folded and composed) and one CPB table per block. Written out term by term
// from s2s_create's uploads; s2s_create checks its own count against it, so
// the two cannot drift apart.
int weights_device_bytes(const s2s_arch &A, const TensorSet &ts, uint64_t *bytes) {
    const uint64_t C = A.embed, C4 = round4(A.embed), H2 = (uint64_t)A.mlp_ratio * A.embed;
    const uint64_t NH = A.heads, n = (uint64_t)A.window * A.window;
    uint64_t f = 0;
    f += C;                     // conv_first's bias (the body skip)
    f += 2 * 9 * 4 * C + C;     // k_embed's two weight sets, the folded bias
    f += 4 * C;                 // patch_embed's LayerNorm, the final LayerNorm
    // the body's C -> C convs: Winograd weights [36][C][C] (in the batched
    // GEMM's register order) or direct [C][9][C4]
    const uint64_t body_conv = wino_body(A.embed) ? WINO_POS * weight_floats(C, C, EPI_STORE) : C * 9 * C4;
    f += body_conv + C;         // conv_after_body
    for (int s = 0; s < A.n_stages; ++s) {
        f += body_conv + C;     // the stage close (3x3 with the 1x1 folded in)
        // the fused qkv (per head pair when the qkv + attention kernel takes
        // the head shape), proj, fc1, fc2 in their GEMMs' layouts
        const uint64_t wqkv = qkv_attn_fused(A.heads, A.embed / A.heads)
                                  ? (uint64_t)(A.heads / 2) * weight_floats(C, C, EPI_STORE)
                                  : weight_floats(3 * C, C, EPI_STORE);
        const uint64_t per_block = wqkv + 3 * C                               // fused qkv, its bias
                                   + NH                                       // logit scale
                                   + weight_floats(C, C, EPI_LN_RES) + C      // proj
                                   + 4 * C                                    // norm1, norm2
                                   + weight_floats(H2, C, EPI_GELU) + H2      // fc1
                                   + weight_floats(C, H2, EPI_LN_RES) + C     // fc2
                                   + NH * n * n;                              // the CPB table
        f += per_block * (uint64_t)A.depths[s];
    }
    const int up = A.upsampler;
    if (up == S2S_PIXELSHUFFLE || up == S2S_PIXELSHUFFLE_AUX || up == S2S_NEAREST_CONV) {
        int F = 0;
        if (head_feat_of(ts, A.embed, &F)) return -1;
        const uint64_t F_ = F, F4 = round4(F);
        // conv_before_upsample: Winograd weights [36][F][C4] or direct [F][9][C4]
        f += (wino_head(A.embed, F) ? WINO_POS * weight_floats(F, C4, EPI_STORE) : F_ * 9 * C4) + F_;
        f += 9 * F_ * 3 + 3;            // conv_last
        if (up == S2S_NEAREST_CONV) {
            f += 2 * (4 * F_ * 4 * F4 + F_) + (F_ * 9 * F4 + F_);  // conv_up1, conv_up2 (by phase), conv_hr
        } else {
            const int oct = octaves_of(A.scale);
            f += (uint64_t)oct * (4 * F_ * 9 * F4 + 4 * F_);  // the octave convs
            if (F % 8 == 0) {
                if (oct >= 2 && F == 64)     // two octaves and conv_last composed (the
                    f += (wino_up2(oct, F) ? WINO_POS * weight_floats(48, F4, EPI_STORE) : 48 * 25 * F_)  // GEMM's,
                         + 4 * 48 * 25 * F_ + 5 * 48;                           // the edges')
                else
                    f += 5 * 12 * 25 * F_ + 5 * 12;  // the last octave and conv_last composed
            }
            if (up == S2S_PIXELSHUFFLE_AUX)
                f += (4 * 25 * 3 * 4 + 12)                     // conv_last o conv_bicubic composed,
                     + (9 * F_ * 3 + 3) + (F_ * 9 * 4 + F_);  // aux, after_aux
        }
    } else if (up == S2S_PIXELSHUFFLE_DIRECT) {
        const uint64_t n3 = 3 * (uint64_t)A.scale * A.scale;
        f += n3 * 9 * C4 + n3;
    }
    *bytes = f * sizeof(float);
    return 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// Exported ABI
// ---------------------------------------------------------------------------

int s2s_ctx_embed(s2s_ctx *ctx) { return ctx ? ctx->arch.embed : 0; }

extern "C" {

const char *s2s_last_error(void) { return g_err.c_str(); }

const char *s2s_name(void) { return "hip"; }

int s2s_create(const s2s_arch *arch, const s2s_tensor *tensors, size_t n_tensors, s2s_ctx **out) {
    if (!arch || !tensors || !out) return fail("s2s_create: null argument");
    *out = nullptr;
    const s2s_arch &A = *arch;
    if (A.embed <= 0 || A.heads <= 0 || A.embed % A.heads != 0)
        return fail("embed_dim must be a positive multiple of num_heads");
    if (A.embed % 4 != 0) return fail("embed_dim must be a multiple of 4 for the device kernels");
    if (A.window != 8)
        return fail("window " + std::to_string(A.window) +
                    ": the device attention kernel is built for 8x8 windows (64 tokens), the "
                    "size of every released checkpoint");
    if (A.embed / A.heads > 32)
        return fail("head_dim " + std::to_string(A.embed / A.heads) +
                    " exceeds the attention kernel's 32 (every released checkpoint has <= 30)");
    if (A.n_stages < 0 || A.n_stages > S2S_MAX_STAGES) return fail("bad stage count");
    if (A.upsampler != S2S_PIXELSHUFFLE && A.upsampler != S2S_PIXELSHUFFLE_DIRECT &&
        A.upsampler != S2S_NEAREST_CONV && A.upsampler != S2S_PIXELSHUFFLE_AUX)
        return fail("unknown upsampler " + std::to_string(A.upsampler));

    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev == 0)
        return fail(std::string("no HIP device: ") + (e == hipSuccess ? "count 0" : hipGetErrorString(e)));

    int dev = 0;
    HIPCHK("hipGetDevice", hipGetDevice(&dev));
    if (scratch_init(dev)) return -1;
    s2s_ctx *ctx = new s2s_ctx();
    ctx->arch = A;
    ctx->c = A.embed;
    ctx->hd = A.embed / A.heads;
    ctx->hidden = A.mlp_ratio * A.embed;
    ctx->device = dev;
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return fail(hip_msg("hipStreamCreate", e));
    }
    const char *pe = getenv("SWIN2SR_PROFILE_GPU");
    ctx->prof = pe && *pe && strcmp(pe, "0") != 0;
    const char *ge = getenv("SWIN2SR_HIP_GRAPHS");
    ctx->graphs = !(ge && strcmp(ge, "0") == 0);

    TensorSet ts{tensors, n_tensors};
    const int C = A.embed, H2 = A.mlp_ratio * C, NH = A.heads, win = A.window, n = win * win;
    const s2s_tensor *x;
    int rc = 0;
    auto up = [&](const std::string &name, std::vector<int64_t> shape, float **dst) -> int {
        if (ts.get(name, shape, &x)) return -1;
        return ctx->upload(vec_of(x, ts.numel(x)), dst);
    };
    auto upconv = [&](const std::string &name, int co, int ci, float **dst,
                      const std::vector<int> *perm) -> int {
        if (ts.get(name, {co, ci, 3, 3}, &x)) return -1;
        return ctx->upload(conv_relayout(x->data, co, ci, perm), dst);
    };
    // a conv of a nearest-2x upsampling [F][F][3][3], as its four phases' 2x2 convs
    auto up_sub2 = [&](const std::string &name, int F, float **dst) -> int {
        if (ts.get(name, {F, F, 3, 3}, &x)) return -1;
        std::vector<float> w((size_t)16 * F * round4(F));
        subpixel_weights(x->data, F, F, w.data());
        return ctx->upload(w, dst);
    };
    // conv_before_upsample [F][C][3][3]: the Winograd transform [36][F][C]
    // when wino_head takes it, else the implicit GEMM's layout
    auto up_before_upsample = [&](int F) -> int {
        ctx->cbu_wino = wino_head(C, F);
        if (!ctx->cbu_wino) return upconv("conv_before_upsample.0.weight", F, C, &ctx->cbu_w, nullptr);
        if (ts.get("conv_before_upsample.0.weight", {F, C, 3, 3}, &x)) return -1;
        std::vector<float> u((size_t)WINO_POS * F * round4(C));
        wino_weights(x->data, F, C, u.data());
        return ctx->upload(gemm_weights(u, WINO_POS, F, round4(C), EPI_STORE), &ctx->cbu_w);
    };

    rc = rc || up("conv_first.bias", {C}, &ctx->cf_b);
    {
        // patch_embed's 1x1 conv (reference src/gpu.rs:474-478) reads nothing
        // but conv_first's output, so it is uploaded folded into conv_first:
        // W[o][i][t] = sum_m P[o][m] Wcf[m][i][t], b[o] = sum_m P[o][m] bcf[m]
        // + bpe[o] (double accumulation, rounded once); k_embed computes both
        // convs (conv_first's output is the body's long skip) in one pass
        const s2s_tensor *wcf, *bcf, *wpe, *bpe;
        rc = rc || ts.get("conv_first.weight", {C, 3, 3, 3}, &wcf);
        rc = rc || ts.get("conv_first.bias", {C}, &bcf);
        rc = rc || ts.get("patch_embed.proj.weight", {C, C, 1, 1}, &wpe);
        rc = rc || ts.get("patch_embed.proj.bias", {C}, &bpe);
        if (!rc) {
            std::vector<float> wf((size_t)C * 27), bf(C);
            for (int o = 0; o < C; ++o) {
                double acc[27] = {0.0};
                double ab = bpe->data[o];
                for (int m = 0; m < C; ++m) {
                    const double pm = wpe->data[(size_t)o * C + m];
                    ab += pm * bcf->data[m];
                    for (int k = 0; k < 27; ++k) acc[k] += pm * wcf->data[(size_t)m * 27 + k];
                }
                for (int k = 0; k < 27; ++k) wf[(size_t)o * 27 + k] = (float)acc[k];
                bf[o] = (float)ab;
            }
            // k_embed's [set][tap][ci][C]: set 0 conv_first, set 1 the fold
            std::vector<float> emb((size_t)2 * 9 * 4 * C, 0.f);
            for (int o = 0; o < C; ++o)
                for (int ci = 0; ci < 3; ++ci)
                    for (int t = 0; t < 9; ++t) {
                        emb[((size_t)t * 4 + ci) * C + o] = wcf->data[(size_t)o * 27 + ci * 9 + t];
                        emb[((size_t)(9 + t) * 4 + ci) * C + o] = wf[(size_t)o * 27 + ci * 9 + t];
                    }
            rc = ctx->upload(emb, &ctx->emb_w) || ctx->upload(bf, &ctx->pe_b);
        }
    }
    rc = rc || up("patch_embed.norm.weight", {C}, &ctx->pe_nw);
    rc = rc || up("patch_embed.norm.bias", {C}, &ctx->pe_nb);
    rc = rc || up("norm.weight", {C}, &ctx->norm_w);
    rc = rc || up("norm.bias", {C}, &ctx->norm_b);
    {
        const s2s_tensor *cw;
        rc = rc || ts.get("conv_after_body.weight", {C, C, 3, 3}, &cw);
        if (!rc) rc = ctx->upload(body_conv_weights(cw->data, C), &ctx->cab_w);
    }
    rc = rc || up("conv_after_body.bias", {C}, &ctx->cab_b);

    // cpb scratch: the [heads][(2w-1)^2] MLP output before the gather
    float *cpb_tab = nullptr;
    if (!rc) rc = ctx->alloc(ctx->weight_allocs, (size_t)NH * (2 * win - 1) * (2 * win - 1),
                             &cpb_tab, "cpb table");

    ctx->stages.resize(A.n_stages);
    for (int s = 0; !rc && s < A.n_stages; ++s) {
        StageW &st = ctx->stages[s];
        const std::string sp = "layers." + std::to_string(s) + ".";
        {
            // The stage close is the 3x3 conv, then the 1x1 patch_embed conv,
            // then the stage residual, with nothing between the two
            // convolutions (reference src/gpu.rs:526-528, src/cpu.rs:1577-1581):
            // one linear map, uploaded as a single 3x3 conv with
            //   W[o][i][t] = sum_m P[o][m] W3[m][i][t],
            //   b[o]       = sum_m P[o][m] b3[m] + b1[o],
            // accumulated in double and rounded once.
            const s2s_tensor *w3, *b3, *w1, *b1;
            rc = rc || ts.get(sp + "conv.weight", {C, C, 3, 3}, &w3);
            rc = rc || ts.get(sp + "conv.bias", {C}, &b3);
            rc = rc || ts.get(sp + "patch_embed.proj.weight", {C, C, 1, 1}, &w1);
            rc = rc || ts.get(sp + "patch_embed.proj.bias", {C}, &b1);
            if (rc) break;
            const size_t kk = (size_t)C * 9;
            std::vector<float> wf((size_t)C * kk), bf(C);
            std::vector<double> acc(kk);
            for (int o = 0; o < C; ++o) {
                std::fill(acc.begin(), acc.end(), 0.0);
                double ab = b1->data[o];
                for (int m = 0; m < C; ++m) {
                    const double pm = w1->data[(size_t)o * C + m];
                    ab += pm * b3->data[m];
                    const float *w3m = w3->data + (size_t)m * kk;
                    for (size_t k = 0; k < kk; ++k) acc[k] += pm * w3m[k];
                }
                for (size_t k = 0; k < kk; ++k) wf[(size_t)o * kk + k] = (float)acc[k];
                bf[o] = (float)ab;
            }
            rc = rc || ctx->upload(body_conv_weights(wf.data(), C), &st.conv_w);
            rc = rc || ctx->upload(bf, &st.conv_b);
        }
        st.blocks.resize(A.depths[s]);
        for (int b = 0; !rc && b < A.depths[s]; ++b) {
            BlockW &bw = st.blocks[b];
            const std::string p = sp + "residual_group.blocks." + std::to_string(b) + ".";
            const s2s_tensor *wq, *wk_, *wv, *qb, *vb;
            rc = rc || ts.get(p + "attn.qkv.wq", {C, C}, &wq);
            rc = rc || ts.get(p + "attn.qkv.wk", {C, C}, &wk_);
            rc = rc || ts.get(p + "attn.qkv.wv", {C, C}, &wv);
            rc = rc || ts.get(p + "attn.qkv.q_bias", {C}, &qb);
            rc = rc || ts.get(p + "attn.qkv.v_bias", {C}, &vb);
            if (rc) break;
            // the fused [3C][C] projection and its [q_bias | 0 | v_bias] bias
            // (reference tools/convert.py:122-138; k has no bias)
            std::vector<float> wqkv((size_t)3 * C * C), bqkv((size_t)3 * C, 0.f);
            std::copy(wq->data, wq->data + (size_t)C * C, wqkv.begin());
            std::copy(wk_->data, wk_->data + (size_t)C * C, wqkv.begin() + (size_t)C * C);
            std::copy(wv->data, wv->data + (size_t)C * C, wqkv.begin() + (size_t)2 * C * C);
            std::copy(qb->data, qb->data + C, bqkv.begin());
            std::copy(vb->data, vb->data + C, bqkv.begin() + 2 * C);
            if (qkv_attn_fused(NH, C / NH)) {
                // the fused qkv + attention kernel's order: each head pair's
                // q|k|v rows as the attention unit's columns, each pair's
                // C x C rows in register order
                std::vector<float> wp(wqkv.size()), bp(bqkv.size());
                qkv_pair_weights(wqkv.data(), bqkv.data(), NH, C / NH, wp.data(), bp.data());
                wqkv = gemm_weights(wp, NH / 2, C, C, EPI_STORE);
                bqkv.swap(bp);
            } else {
                wqkv = gemm_weights(wqkv, 1, 3 * C, C, EPI_STORE);
            }
            rc = rc || ctx->upload(wqkv, &bw.wqkv) || ctx->upload(bqkv, &bw.bqkv);
            const s2s_tensor *lsx;
            rc = rc || ts.get(p + "attn.logit_scale", {NH, 1, 1}, &lsx);
            if (rc) break;
            rc = ctx->upload(vec_of(lsx, NH), &bw.ls);
            auto up_gemm = [&](const std::string &name, int N, int K, int epi, float **dst) -> int {
                if (ts.get(name, {N, K}, &x)) return -1;
                return ctx->upload(gemm_weights(vec_of(x, ts.numel(x)), 1, N, K, epi), dst);
            };
            rc = rc || up_gemm(p + "attn.proj.weight", C, C, EPI_LN_RES, &bw.wproj);
            rc = rc || up(p + "attn.proj.bias", {C}, &bw.bproj);
            rc = rc || up(p + "norm1.weight", {C}, &bw.n1w);
            rc = rc || up(p + "norm1.bias", {C}, &bw.n1b);
            rc = rc || up(p + "norm2.weight", {C}, &bw.n2w);
            rc = rc || up(p + "norm2.bias", {C}, &bw.n2b);
            rc = rc || up_gemm(p + "mlp.fc1.weight", H2, C, EPI_GELU, &bw.w1);
            rc = rc || up(p + "mlp.fc1.bias", {H2}, &bw.b1);
            rc = rc || up_gemm(p + "mlp.fc2.weight", C, H2, EPI_LN_RES, &bw.w2);
            rc = rc || up(p + "mlp.fc2.bias", {C}, &bw.b2);
            if (rc) break;
            // The bias table, stored [head][query][key] and scaled by log2(e)
            // for the base-2 softmax. From the converter's cpb_pre when the
            // set carries it - the table the crate itself reads
            // (src/gpu.rs:780-790, src/cpu.rs:1276-1284) - otherwise from the
            // MLP (16*sigmoid of Linear-ReLU-Linear on the log-spaced
            // coordinates, gathered, computed on the device).
            rc = ctx->alloc(ctx->weight_allocs, (size_t)NH * n * n, &bw.cpbt, "cpb");
            if (rc) break;
            ctx->uploaded += (uint64_t)NH * n * n * sizeof(float);
            if (ts.find(p + "attn.cpb_pre")) {
                const s2s_tensor *cp;
                rc = ts.get(p + "attn.cpb_pre", {(int64_t)n * n, NH}, &cp);
                if (rc) break;
                std::vector<float> t((size_t)NH * n * n);
                for (int q = 0; q < n; ++q)
                    for (int k = 0; k < n; ++k)
                        for (int hh = 0; hh < NH; ++hh)
                            t[((size_t)hh * n + q) * n + k] =
                                ATTN_LOG2E * cp->data[((size_t)q * n + k) * NH + hh];
                if (hipMemcpy(bw.cpbt, t.data(), t.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
                    rc = fail("hipMemcpy(cpb) failed");
            } else {
                const s2s_tensor *w0, *b0, *w2;
                rc = rc || ts.get(p + "attn.cpb_mlp.0.weight", {512, 2}, &w0);
                rc = rc || ts.get(p + "attn.cpb_mlp.0.bias", {512}, &b0);
                rc = rc || ts.get(p + "attn.cpb_mlp.2.weight", {NH, 512}, &w2);
                if (rc) break;
                float *dw0, *db0, *dw2;
                AllocList tmpl;
                rc = ctx->alloc(tmpl, 1024, &dw0, "cpb w0") || ctx->alloc(tmpl, 512, &db0, "cpb b0") ||
                     ctx->alloc(tmpl, (size_t)NH * 512, &dw2, "cpb w2");
                if (!rc) {
                    hipError_t le = hipMemcpy(dw0, w0->data, 1024 * 4, hipMemcpyHostToDevice);
                    if (le == hipSuccess)
                        le = hipMemcpy(db0, b0->data, 512 * 4, hipMemcpyHostToDevice);
                    if (le == hipSuccess)
                        le = hipMemcpy(dw2, w2->data, (size_t)NH * 512 * 4, hipMemcpyHostToDevice);
                    if (le == hipSuccess)
                        le = launch_cpb(dw0, db0, dw2, cpb_tab, bw.cpbt, win, NH, ctx->stream);
                    if (le == hipSuccess) le = hipStreamSynchronize(ctx->stream);
                    if (le != hipSuccess) rc = fail(hip_msg("cpb table", le));
                }
                free_list(tmpl);
            }
        }
    }

    // ---- the reconstruction head (reference src/gpu.rs:801-872, network_swin2sr.py:790-860)
    auto head_feat = [&]() -> int { return head_feat_of(ts, C, &ctx->feat); };
    auto conv_last = [&](int F) -> int {
        const s2s_tensor *lw;
        if (ts.get("conv_last.weight", {3, F, 3, 3}, &lw)) return -1;
        std::vector<float> t((size_t)9 * F * 3);
        for (int co = 0; co < 3; ++co)
            for (int ci = 0; ci < F; ++ci)
                for (int tap = 0; tap < 9; ++tap)
                    t[((size_t)tap * F + ci) * 3 + co] = lw->data[((size_t)co * F + ci) * 9 + tap];
        return ctx->upload(t, &ctx->last_w) || up("conv_last.bias", {3}, &ctx->last_b);
    };
    if (!rc && (A.upsampler == S2S_PIXELSHUFFLE || A.upsampler == S2S_PIXELSHUFFLE_AUX)) {
        if (A.scale < 2 || (A.scale & (A.scale - 1)))
            rc = fail("the pixel-shuffle head needs a power-of-two scale, got " + std::to_string(A.scale));
        rc = rc || head_feat();
        if (!rc) {
            const int F = ctx->feat;
            const int oct = octaves_of(A.scale);
            ctx->octaves = oct;
            rc = rc || up_before_upsample(F);
            rc = rc || up("conv_before_upsample.0.bias", {F}, &ctx->cbu_b);
            const std::vector<int> perm = shuffle_perm(F);
            // the head's last octave (two, at x4 and above) composed with
            // conv_last; the compressed head's bicubic branch, which the
            // reference adds before conv_last, then goes through its own
            // composition with conv_last (compose_bic_last)
            ctx->fuse_last = F % 8 == 0;
            for (int o = 0; !rc && o < oct; ++o) {
                const s2s_tensor *uw, *ub;
                const std::string base = "upsample." + std::to_string(2 * o);
                rc = rc || ts.get(base + ".weight", {4 * F, F, 3, 3}, &uw);
                rc = rc || ts.get(base + ".bias", {4 * F}, &ub);
                if (rc) break;
                float *dw, *db;
                std::vector<float> bb(4 * F);
                for (int co = 0; co < 4 * F; ++co) bb[perm[co]] = ub->data[co];
                rc = ctx->upload(conv_relayout(uw->data, 4 * F, F, &perm), &dw) || ctx->upload(bb, &db);
                ctx->up_w.push_back(dw);
                ctx->up_b.push_back(db);
            }
            rc = rc || conv_last(F);
            if (!rc && ctx->fuse_last) {
                const s2s_tensor *uw, *ub, *lw, *lb;
                const std::string base = "upsample." + std::to_string(2 * (oct - 1));
                rc = rc || ts.get(base + ".weight", {4 * F, F, 3, 3}, &uw);
                rc = rc || ts.get(base + ".bias", {4 * F}, &ub);
                rc = rc || ts.get("conv_last.weight", {3, F, 3, 3}, &lw);
                rc = rc || ts.get("conv_last.bias", {3}, &lb);
                if (!rc) {
                    std::vector<float> wi, bi, we, be;
                    compose_up_last(uw->data, ub->data, lw->data, lb->data, F, wi, bi, we, be);
                    if (oct >= 2 && F == 64) {  // (the edge kernel's channel count)
                        const s2s_tensor *u0w, *u0b;
                        const std::string b0 = "upsample." + std::to_string(2 * (oct - 2));
                        rc = rc || ts.get(b0 + ".weight", {4 * F, F, 3, 3}, &u0w);
                        rc = rc || ts.get(b0 + ".bias", {4 * F}, &u0b);
                        if (!rc) {
                            std::vector<float> wg, bg, w48, b48, u5;
                            ctx->up2_wino = wino_up2(oct, F);
                            compose_up2_last(we, be, u0w->data, u0b->data, F, wg, bg, w48, b48,
                                             ctx->up2_wino ? &u5 : nullptr);
                            rc = ctx->upload(ctx->up2_wino ? gemm_weights(u5, WINO_POS, 48, F, EPI_STORE) : wg,
                                             &ctx->u2_w) ||
                                 ctx->upload(bg, &ctx->u2_b) || ctx->upload(w48, &ctx->u2_we) ||
                                 ctx->upload(b48, &ctx->u2_be);
                            ctx->fuse2 = true;
                        }
                    } else {
                        rc = ctx->upload(wi, &ctx->ul_w) || ctx->upload(bi, &ctx->ul_b) ||
                             ctx->upload(we, &ctx->ul_we) || ctx->upload(be, &ctx->ul_be);
                    }
                }
            }
            if (A.upsampler == S2S_PIXELSHUFFLE_AUX && !ctx->fuse_last)
                rc = rc || fail("internal: the compressed head composes its octaves with conv_last");
            if (!rc && A.upsampler == S2S_PIXELSHUFFLE_AUX) {
                const s2s_tensor *bw, *bb, *lw;
                rc = rc || ts.get("conv_bicubic.weight", {F, 3, 3, 3}, &bw);
                rc = rc || ts.get("conv_bicubic.bias", {F}, &bb);
                rc = rc || ts.get("conv_last.weight", {3, F, 3, 3}, &lw);
                if (!rc) {
                    std::vector<float> w, b;
                    compose_bic_last(bw->data, bb->data, lw->data, F, w, b);
                    rc = ctx->upload(w, &ctx->bl_w) || ctx->upload(b, &ctx->bl_b);
                }
            }
            if (A.upsampler == S2S_PIXELSHUFFLE_AUX) {
                // conv_aux in conv_last's layout [tap][ci][3] (the same kernel)
                const s2s_tensor *aw;
                rc = rc || ts.get("conv_aux.weight", {3, F, 3, 3}, &aw);
                if (!rc) {
                    std::vector<float> t((size_t)9 * F * 3);
                    for (int co = 0; co < 3; ++co)
                        for (int ci = 0; ci < F; ++ci)
                            for (int tap = 0; tap < 9; ++tap)
                                t[((size_t)tap * F + ci) * 3 + co] = aw->data[((size_t)co * F + ci) * 9 + tap];
                    rc = ctx->upload(t, &ctx->ax_w);
                }
                rc = rc || up("conv_aux.bias", {3}, &ctx->ax_b);
                rc = rc || upconv("conv_after_aux.0.weight", F, 3, &ctx->caa_w, nullptr);
                rc = rc || up("conv_after_aux.0.bias", {F}, &ctx->caa_b);
            }
        }
    } else if (!rc && A.upsampler == S2S_PIXELSHUFFLE_DIRECT) {
        const int n = 3 * A.scale * A.scale;
        rc = rc || upconv("upsample.0.weight", n, C, &ctx->psd_w, nullptr);
        rc = rc || up("upsample.0.bias", {n}, &ctx->psd_b);
    } else if (!rc && A.upsampler == S2S_NEAREST_CONV) {
        if (A.scale != 4)
            rc = fail("the nearest+conv head upsamples by exactly 4 (two nearest-2x steps), got scale " +
                      std::to_string(A.scale));
        rc = rc || head_feat();
        if (!rc) {
            const int F = ctx->feat;
            rc = rc || up_before_upsample(F);
            rc = rc || up("conv_before_upsample.0.bias", {F}, &ctx->cbu_b);
            rc = rc || up_sub2("conv_up1.weight", F, &ctx->nu1_w);
            rc = rc || up("conv_up1.bias", {F}, &ctx->nu1_b);
            rc = rc || up_sub2("conv_up2.weight", F, &ctx->nu2_w);
            rc = rc || up("conv_up2.bias", {F}, &ctx->nu2_b);
            rc = rc || upconv("conv_hr.weight", F, F, &ctx->hr_w, nullptr);
            rc = rc || up("conv_hr.bias", {F}, &ctx->hr_b);
            rc = rc || conv_last(F);
        }
    }
    uint64_t planned = 0;
    if (!rc && weights_device_bytes(A, ts, &planned)) rc = -1;
    if (!rc && planned != ctx->uploaded)
        rc = fail("internal: s2s_create uploaded " + std::to_string(ctx->uploaded) +
                  " bytes where s2s_uploaded_bytes_for plans " + std::to_string(planned));
    if (!rc) {
        // an allocation cap on the per-image plans, for callers (and tests)
        // that reserve device memory: "out of memory" past it
        const char *lim = getenv("SWIN2SR_HIP_ALLOC_LIMIT");
        if (lim && *lim) ctx->alloc_limit = strtoull(lim, nullptr, 10);
    }
    if (rc) {
        std::string keep = g_err;
        delete ctx;
        g_err = keep;
        return -1;
    }
    *out = ctx;
    return 0;
}

int s2s_uploaded_bytes_for(const s2s_arch *arch, const s2s_tensor *tensors, size_t n_tensors,
                           uint64_t *bytes) {
    if (!arch || !tensors || !bytes) return fail("s2s_uploaded_bytes_for: null argument");
    if (arch->embed <= 0 || arch->heads <= 0 || arch->n_stages < 0 ||
        arch->n_stages > S2S_MAX_STAGES)
        return fail("s2s_uploaded_bytes_for: bad architecture");
    TensorSet ts{tensors, n_tensors};
    return weights_device_bytes(*arch, ts, bytes);
}

int s2s_plan_bytes(s2s_ctx *ctx, int h, int w, uint64_t *bytes) {
    if (!ctx || !bytes) return fail("s2s_plan_bytes: null argument");
    if (h < ctx->arch.window || w < ctx->arch.window) return fail("image smaller than one window");
    const int win = ctx->arch.window;
    std::vector<BufSpec> v;
    ctx->body_specs((h / win + 1) * win, (w / win + 1) * win, false, v);
    ctx->image_specs(h, w, true, false, v);
    uint64_t b = 0;
    for (const BufSpec &x : v) b += std::max<size_t>(x.floats, 1) * sizeof(float);
    *bytes = b;
    return 0;
}

int s2s_set_alloc_limit(s2s_ctx *ctx, uint64_t bytes) {
    if (!ctx) return fail("null context");
    ctx->alloc_limit = bytes;
    if (ctx->lane) ctx->lane->alloc_limit = bytes;
    return 0;
}

void s2s_destroy(s2s_ctx *ctx) { delete ctx; }

uint64_t s2s_uploaded_bytes(const s2s_ctx *ctx) { return ctx ? ctx->uploaded : 0; }

int s2s_forward_device(s2s_ctx *ctx, int h, int w, const float *d_in, float *d_out) {
    if (!ctx) return fail("null context");
    HIPCHK("hipSetDevice", hipSetDevice(ctx->device));
    return ctx->forward_device(h, w, d_in, d_out);
}

// n independent images of one size, alternating between the context's stream
// and a second lane's (its own stream, plans and graphs over the same
// weights), so that one image's kernel boundaries (each launch's start and
// tail, which leave CUs idle) overlap the other's kernels. The lane waits for
// the work already on the context's stream and the context's stream then
// waits for the lane, so ordering and synchronisation through s2s_stream /
// s2s_sync stay as for s2s_forward_device.
int s2s_forward_device_batch(s2s_ctx *ctx, int n, int h, int w, const float *const *d_in,
                             float *const *d_out) {
    if (!ctx || n < 0 || (n > 0 && (!d_in || !d_out)))
        return fail("s2s_forward_device_batch: null argument");
    for (int i = 0; i < n; ++i)
        if (!d_in[i] || !d_out[i]) return fail("s2s_forward_device_batch: null image pointer");
    HIPCHK("hipSetDevice", hipSetDevice(ctx->device));
    if (n <= 1) return n == 1 ? ctx->forward_device(h, w, d_in[0], d_out[0]) : 0;
    if (ctx->make_lane()) return -1;
    s2s_ctx *L = ctx->lane;
    HIPCHK("hipEventRecord(fork)", hipEventRecord(ctx->fork_ev, ctx->stream));
    HIPCHK("hipStreamWaitEvent(fork)", hipStreamWaitEvent(L->stream, ctx->fork_ev, 0));
    int rc = 0;
    for (int i = 0; i < n && !rc; ++i) rc = ((i & 1) ? L : ctx)->forward_device(h, w, d_in[i], d_out[i]);
    // joined after a failure too, so that whatever the lane launched is covered
    hipError_t e = hipEventRecord(ctx->join_ev, L->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(ctx->stream, ctx->join_ev, 0);
    if (rc) return rc;
    if (e != hipSuccess) return fail(hip_msg("s2s_forward_device_batch: joining the lane", e));
    return 0;
}

// The forward with every intermediate buffer carved out of this GPU's static
// workspace instead of the context's planned allocations: no hipMalloc,
// hipFree or other allocating call (and no profiler events). The context's
// own plan is left as it was. Calls that overlap on one GPU (other contexts,
// other streams) share the one workspace and race.
int s2s_forward_device_noalloc(s2s_ctx *ctx, int h, int w, const float *d_in, float *d_out) {
    if (!ctx || !d_in || !d_out) return fail("s2s_forward_device_noalloc: null argument");
    const int win = ctx->arch.window;
    if (h < win || w < win) return ctx->forward_device(h, w, d_in, d_out);  // its error message
    HIPCHK("hipSetDevice", hipSetDevice(ctx->device));
    char *base = ctx->device >= 0 && ctx->device < kMaxDevices ? (char *)g_scratch[ctx->device] : nullptr;
    if (!base) return fail("s2s_forward_device_noalloc: no workspace address for this device");
    const int hp = (h / win + 1) * win, wp = (w / win + 1) * win;

    // the context's plan, restored on every return
    struct Saved {
        s2s_ctx *c;
        int bhp, bwp, ih, iw;
        bool prof;
        float *cur, *wk, *body, *qkv, *o, *hid, *in_dev, *in4, *out_dev;
        float *aux4, *auxp, *bic4;
        std::vector<float *> fplanes;
        ~Saved() {
            c->bhp = bhp; c->bwp = bwp; c->ih = ih; c->iw = iw; c->prof = prof;
            c->cur = cur; c->wk = wk; c->body = body; c->qkv = qkv; c->o = o;
            c->hid = hid; c->in_dev = in_dev; c->in4 = in4; c->out_dev = out_dev;
            c->aux4 = aux4; c->auxp = auxp; c->bic4 = bic4;
            c->fplanes.swap(fplanes);
        }
    } saved{ctx, ctx->bhp, ctx->bwp, ctx->ih, ctx->iw, ctx->prof, ctx->cur, ctx->wk,
            ctx->body, ctx->qkv, ctx->o, ctx->hid, ctx->in_dev, ctx->in4, ctx->out_dev,
            ctx->aux4, ctx->auxp, ctx->bic4, {}};
    saved.fplanes.swap(ctx->fplanes);

    std::vector<BufSpec> v;
    ctx->body_specs(hp, wp, true, v);
    ctx->image_specs(h, w, false, true, v);
    size_t off = 0;
    for (const BufSpec &b : v) off += (std::max<size_t>(b.floats, 1) * sizeof(float) + 255) / 256 * 256;
    if (off > S2S_NOALLOC_SCRATCH_BYTES)
        return fail("s2s_forward_device_noalloc: a " + std::to_string(h) + "x" + std::to_string(w) +
                    " image needs " + std::to_string(off) + " bytes of workspace, above this "
                    "entry's maximum of " + std::to_string(S2S_NOALLOC_SCRATCH_BYTES) +
                    " bytes (use s2s_forward_device, or a smaller tile)");
    off = 0;
    for (const BufSpec &b : v) {
        *b.dst = (float *)(base + off);
        off += (std::max<size_t>(b.floats, 1) * sizeof(float) + 255) / 256 * 256;
    }
    // the carved plan is the current one for this call (plan_image keeps it)
    ctx->bhp = hp;
    ctx->bwp = wp;
    ctx->ih = h;
    ctx->iw = w;
    ctx->prof = false;
    // An eager call waits on the stream for the workspace's previous user
    // (any context on this GPU) and marks itself its last. A call captured
    // into a caller's graph is not ordered here: its replays run when the
    // caller launches them, so overlapping replays and calls still race.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIPCHK("hipStreamIsCapturing", hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone) return ctx->forward_device(h, w, d_in, d_out, false);
    std::lock_guard<std::mutex> lock(g_ws_mu[ctx->device]);
    HIPCHK("hipStreamWaitEvent(workspace)", hipStreamWaitEvent(ctx->stream, g_ws_event[ctx->device], 0));
    const int rc = ctx->forward_device(h, w, d_in, d_out, false);
    // recorded after a failed call too: whatever it launched is then waited for
    const hipError_t e = hipEventRecord(g_ws_event[ctx->device], ctx->stream);
    if (rc) return rc;
    if (e != hipSuccess) return fail(hip_msg("hipEventRecord(workspace)", e));
    return 0;
}

// Host copy out of the pinned staging image into the caller's buffer with
// streaming (non-temporal) stores: the destination lines are written whole
// without first being read into the cache, which roughly halves the memory
// traffic of a plain copy of a buffer this size. AVX2 where the CPU has it,
// memcpy otherwise.
__attribute__((target("avx2"))) static void stream_copy_avx2(float *dst, const float *src, size_t n) {
    size_t i = 0;
    while (i < n && ((uintptr_t)(dst + i) & 31)) {
        dst[i] = src[i];
        ++i;
    }
    for (; i + 32 <= n; i += 32) {
        const __m256 a = _mm256_loadu_ps(src + i), b = _mm256_loadu_ps(src + i + 8);
        const __m256 c = _mm256_loadu_ps(src + i + 16), d = _mm256_loadu_ps(src + i + 24);
        _mm256_stream_ps(dst + i, a);
        _mm256_stream_ps(dst + i + 8, b);
        _mm256_stream_ps(dst + i + 16, c);
        _mm256_stream_ps(dst + i + 24, d);
    }
    for (; i < n; ++i) dst[i] = src[i];
    _mm_sfence();
}

static void copy_out(float *dst, const float *src, size_t n) {
    static const bool avx2 = __builtin_cpu_supports("avx2");
    if (avx2 && n >= 1024)
        stream_copy_avx2(dst, src, n);
    else
        std::memcpy(dst, src, n * sizeof(float));
}

// The host path: the caller's pageable input is copied into the context's
// pinned staging image and uploaded as one DMA; the output comes back in
// chunks, each copied out of the pinned image while the next is still in
// flight, so the host copy overlaps the link.
// One image through the host path, in two halves so that a batch can keep two
// lanes busy: `host_enqueue` copies the caller's pageable input into the
// pinned staging image, uploads it as one DMA, enqueues the forward and the
// output's download in 2 MiB chunks, each with an event; `host_complete`
// touches every page of the caller's output once (a freshly allocated array
// takes its page faults while the device runs), then copies each finished
// chunk out of the pinned image with streaming stores while the next is in
// flight, and downloads the compressed head's aux image.
struct HostJob {
    int h = 0, w = 0;
    size_t nout = 0;
    std::vector<hipEvent_t> done;
};

static int host_enqueue(s2s_ctx *ctx, int h, int w, const float *in_adjusted, HostJob &job) {
    if (ctx->plan_image(h, w) || ctx->stage_buffers(h, w)) return -1;
    const int s = ctx->arch.scale;
    const size_t nin = (size_t)3 * h * w, nout = (size_t)3 * h * s * w * s;
    job.h = h;
    job.w = w;
    job.nout = nout;
    std::memcpy(ctx->pin_in, in_adjusted, nin * 4);
    HIPCHK("hipMemcpyAsync(input)", hipMemcpyAsync(ctx->in_dev, ctx->pin_in, nin * 4,
                                                   hipMemcpyHostToDevice, ctx->stream));
    if (ctx->forward_device(h, w, ctx->in_dev, ctx->out_dev)) return -1;
    constexpr size_t kChunk = (size_t)1 << 19;  // floats per download chunk (2 MiB)
    const size_t nchunks = (nout + kChunk - 1) / kChunk;
    job.done.assign(nchunks, nullptr);
    for (size_t i = 0; i < nchunks; ++i) {
        const size_t off = i * kChunk, len = std::min(kChunk, nout - off);
        hipError_t e = hipMemcpyAsync(ctx->pin_out + off, ctx->out_dev + off, len * 4,
                                      hipMemcpyDeviceToHost, ctx->stream);
        if (e == hipSuccess) e = (job.done[i] = ctx->event()) ? hipSuccess : hipErrorOutOfMemory;
        if (e == hipSuccess) e = hipEventRecord(job.done[i], ctx->stream);
        if (e != hipSuccess) return fail(hip_msg("hipMemcpyAsync(output)", e));
    }
    return 0;
}

// (returns the job's events to the context whatever happens)
static int host_complete(s2s_ctx *ctx, HostJob &job, float *out) {
    constexpr size_t kChunk = (size_t)1 << 19;
    int rc = 0;
    for (hipEvent_t e : job.done)
        if (!e) rc = -1;  // (host_enqueue failed part-way; its error is set)
    if (rc == 0)
        for (size_t i = 0; i < job.nout; i += 1024) out[i] = 0.f;
    for (size_t i = 0; i < job.done.size(); ++i) {
        if (!job.done[i]) continue;
        if (rc == 0) {
            const hipError_t e = hipEventSynchronize(job.done[i]);
            if (e != hipSuccess) {
                rc = fail(hip_msg("hipEventSynchronize(output)", e));
            } else {
                const size_t off = i * kChunk, len = std::min(kChunk, job.nout - off);
                copy_out(out + off, ctx->pin_out + off, len);
            }
        }
        ctx->free_events.push_back(job.done[i]);
    }
    job.done.clear();
    if (rc) return rc;
    ctx->aux_host.clear();
    if (ctx->arch.upsampler == S2S_PIXELSHUFFLE_AUX) {
        // the compressed head's second image, at the padded geometry
        // (reference src/gpu.rs:752-758)
        const int win = ctx->arch.window;
        const size_t P = (size_t)(job.h / win + 1) * win * ((job.w / win + 1) * win);
        ctx->aux_host.resize(3 * P);
        HIPCHK("hipMemcpyAsync(aux)", hipMemcpyAsync(ctx->aux_host.data(), ctx->auxp, 3 * P * 4,
                                                     hipMemcpyDeviceToHost, ctx->stream));
    }
    HIPCHK("hipStreamSynchronize", hipStreamSynchronize(ctx->stream));
    return 0;
}

int s2s_forward(s2s_ctx *ctx, int h, int w, const float *in_adjusted, float *out) {
    if (!ctx || !in_adjusted || !out) return fail("s2s_forward: null argument");
    HIPCHK("hipSetDevice", hipSetDevice(ctx->device));
    if (h < ctx->arch.window || w < ctx->arch.window) return ctx->forward_device(h, w, nullptr, nullptr);
    HostJob job;
    const int rc = host_enqueue(ctx, h, w, in_adjusted, job);
    const int rc2 = host_complete(ctx, job, out);
    return rc ? rc : rc2;
}

// n host images (sizes may differ: a tiled image's crops) through the host
// path, alternating between the context and its second lane (s2s_forward_device_batch's),
// pipelined: while one lane's image is copied out on the host, the other lane
// computes. Each image's result equals s2s_forward's; aux_out[i], if given,
// receives image i's aux image (the compressed head's, at its padded geometry),
// and s2s_aux afterwards returns the last image's.
int s2s_forward_batch(s2s_ctx *ctx, int n, const int *h, const int *w, const float *const *in_adjusted,
                      float *const *out, float *const *aux_out) {
    if (!ctx || n < 0 || (n > 0 && (!h || !w || !in_adjusted || !out)))
        return fail("s2s_forward_batch: null argument");
    for (int i = 0; i < n; ++i) {
        if (!in_adjusted[i] || !out[i]) return fail("s2s_forward_batch: null image pointer");
        if (h[i] < ctx->arch.window || w[i] < ctx->arch.window)
            return ctx->forward_device(h[i], w[i], nullptr, nullptr);  // its error message
    }
    HIPCHK("hipSetDevice", hipSetDevice(ctx->device));
    if (n > 1 && ctx->make_lane()) return -1;
    s2s_ctx *lanes[2] = {ctx, ctx->lane};
    HostJob jobs[2];
    auto lane_aux = [&](int i) -> int {
        s2s_ctx *L = lanes[i & 1];
        if (!aux_out || !aux_out[i] || L->aux_host.empty()) return 0;
        std::memcpy(aux_out[i], L->aux_host.data(), L->aux_host.size() * 4);
        return 0;
    };
    // enqueue 0 (and 1); then complete i and enqueue i + 2 on the same lane
    int rc = 0, last = -1;
    for (int i = 0; i < n && i < 2 && !rc; ++i) rc = host_enqueue(lanes[i], h[i], w[i], in_adjusted[i], jobs[i]);
    for (int i = 0; i < n; ++i) {
        const int rc_c = host_complete(lanes[i & 1], jobs[i & 1], out[i]);
        if (rc || rc_c) {
            rc = rc ? rc : rc_c;
            // drain the other lane's outstanding job (its events back to it)
            if (i + 1 < n && !jobs[(i + 1) & 1].done.empty()) {
                std::vector<float> scratch(jobs[(i + 1) & 1].nout);
                (void)host_complete(lanes[(i + 1) & 1], jobs[(i + 1) & 1], scratch.data());
            }
            break;
        }
        lane_aux(i);
        last = i;
        if (i + 2 < n) rc = host_enqueue(lanes[i & 1], h[i + 2], w[i + 2], in_adjusted[i + 2], jobs[i & 1]);
    }
    if (rc) return rc;
    if (last >= 1 && (last & 1)) ctx->aux_host = ctx->lane->aux_host;
    return 0;
}

int s2s_aux(s2s_ctx *ctx, const float **ptr, size_t *n) {
    if (!ctx || !ptr || !n) return fail("s2s_aux: null argument");
    if (ctx->aux_host.empty()) {
        *ptr = nullptr;
        *n = 0;
    } else {
        *ptr = ctx->aux_host.data();
        *n = ctx->aux_host.size();
    }
    return 0;
}

int s2s_rstb_device(s2s_ctx *ctx, int stage, int hp, int wp, const float *d_in, float *d_out) {
    if (!ctx) return fail("null context");
    if (stage < 0 || stage >= ctx->arch.n_stages) return fail("stage out of range");
    if (hp % ctx->arch.window || wp % ctx->arch.window || hp <= 0 || wp <= 0)
        return fail("the plane must be a positive multiple of the window in both directions");
    HIPCHK("hipSetDevice", hipSetDevice(ctx->device));
    if (ctx->plan_body(hp, wp)) return -1;
    return ctx->stage_fwd(stage, hp, wp, d_in, d_out);
}

int s2s_device_info(char *name, size_t name_cap, char *arch, size_t arch_cap) {
    int dev = 0;
    HIPCHK("hipGetDevice", hipGetDevice(&dev));
    hipDeviceProp_t p;
    HIPCHK("hipGetDeviceProperties", hipGetDeviceProperties(&p, dev));
    if (name && name_cap) snprintf(name, name_cap, "%s", p.name);
    if (arch && arch_cap) snprintf(arch, arch_cap, "%s", p.gcnArchName);
    return 0;
}

int s2s_vram(uint64_t *free_bytes, uint64_t *total_bytes) {
    size_t f = 0, t = 0;
    HIPCHK("hipMemGetInfo", hipMemGetInfo(&f, &t));
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return 0;
}

int s2s_sync(void) {
    HIPCHK("hipDeviceSynchronize", hipDeviceSynchronize());
    return 0;
}

void *s2s_stream(s2s_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int s2s_profile_enable(s2s_ctx *ctx, int on) {
    if (!ctx) return fail("null context");
    if (!on && ctx->drain()) return -1;
    ctx->prof = on != 0;
    return 0;
}

int s2s_profile_reset(s2s_ctx *ctx) {
    if (!ctx) return fail("null context");
    if (ctx->drain()) return -1;
    ctx->rows.clear();
    return 0;
}

int s2s_profile_report(s2s_ctx *ctx, float wall_ms) {
    if (!ctx) return fail("null context");
    if (ctx->drain()) return -1;
    std::vector<std::pair<ProfKey, ProfRow>> v(ctx->rows.begin(), ctx->rows.end());
    std::sort(v.begin(), v.end(), [](const auto &a, const auto &b) { return a.second.ms > b.second.ms; });
    double total = 0;
    for (auto &r : v) total += r.second.ms;
    fprintf(stderr, "gpu profile (%zu rows, %.3f ms in kernels, wall %.3f ms):\n", v.size(), total,
            wall_ms);
    fprintf(stderr, "  %-24s %-16s %-12s %7s %11s %10s %6s\n", "kernel", "grid", "block", "calls",
            "total ms", "avg ms", "%wall");
    for (auto &r : v) {
        char g[48], b[48];
        snprintf(g, sizeof g, "%u,%u,%u", r.first.g[0], r.first.g[1], r.first.g[2]);
        snprintf(b, sizeof b, "%u,%u,%u", r.first.b[0], r.first.b[1], r.first.b[2]);
        fprintf(stderr, "  %-24s %-16s %-12s %7d %11.3f %10.4f %6.1f\n", r.first.name.c_str(), g, b,
                r.second.calls, r.second.ms, r.second.ms / r.second.calls,
                wall_ms > 0 ? 100.0 * r.second.ms / wall_ms : 0.0);
    }
    return 0;
}

int s2s_profile_only(s2s_ctx *ctx, const char *kernel) {
    if (!ctx) return fail("null context");
    ctx->prof_only = kernel ? kernel : "";
    return 0;
}

int s2s_profile_query(s2s_ctx *ctx, const char *kernel, double *total_ms, int *launches) {
    if (!ctx || !kernel) return fail("null argument");
    if (ctx->drain()) return -1;
    double ms = 0;
    int calls = 0;
    for (auto &r : ctx->rows)
        if (r.first.name == kernel) {
            ms += r.second.ms;
            calls += r.second.calls;
        }
    if (total_ms) *total_ms = ms;
    if (launches) *launches = calls;
    return 0;
}

}  // extern "C"
