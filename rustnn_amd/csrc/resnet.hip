// Device-resident CIFAR ResNet train step (model.rs, nn.rs) on one MI355X.
//
// Reference: ResNet / BasicBlock (model.rs:10-209) over Conv2d, BatchNorm2d,
// gap, the classifier Linear, softmax_ce and Param::step (nn.rs), driven as in
// train.rs:686-699 / bench.rs:128-140: forward, softmax-CE, backward, SGD.
//
// Everything stays in HBM for the whole step: parameters, gradients and
// momenta in three flat arrays (weight-decayed parameters first, so the SGD
// step is one launch), BN running statistics in one array, and every
// activation the backward needs, planned once per input shape.  No tensor is
// copied between layers: BN writes its output next to its input (the input is
// kept so the backward recomputes xhat bit for bit instead of storing it), the
// second BN of a block, the shortcut (identity or 1x1 conv + BN), the residual
// add and the ReLU are one kernel, and each ReLU's backward is folded into the
// BN backward / residual add that consume its gradient.
//
// rnn_resnet_train_step records the step into a hipGraph the second time it
// is called for a shape and replays it from then on (RNN_GRAPH=0 disables
// this).  Step scalars (lr, momentum, wd, label smoothing) live in device
// memory written by a one-thread kernel before each replay; inputs are copied
// into the network's own input slots (or written there by the caller through
// rnn_resnet_inputs), so the graph never sees caller pointers.
#include "rnn_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

// rng.rs (Rng::new, next_u64, uniform, normal): splitmix64-seeded
// xoshiro256++ and Box-Muller on 24-bit uniforms, used for the Kaiming
// initialisation of ResNet::new.
struct HostRng {
    uint64_t s[4];
    explicit HostRng(uint64_t seed) {
        uint64_t z = seed + 0x9E3779B97F4A7C15ull;
        for (auto &w : s) {
            z += 0x9E3779B97F4A7C15ull;
            uint64_t x = z;
            x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
            x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
            w = x ^ (x >> 31);
        }
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        const uint64_t r = rotl(s[0] + s[3], 23) + s[0];
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    float uniform() { return (float)(next() >> 40) * (1.0f / 16777216.0f); }
    float normal() {
        float u1 = uniform();
        if (!(u1 > 1e-7f)) u1 = 1e-7f;
        const float u2 = uniform();
        return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958647692f * u2);
    }
};

struct ParamSlot {
    size_t off = 0, len = 0;
    bool decay = false;
};

struct NetConv {
    uint32_t cin = 0, cout = 0, k = 0, stride = 1, pad = 0;
    int w = -1;  // parameter index
    // dW partial slabs of the last backward (per plan); null: dW is added
    // straight into the gradient instead
    float *slabs = nullptr;
    int nz = 0;
    // dW in a grouped launch of the backward (group gset, member gidx)
    // instead of a launch of its own
    bool grouped = false;
    int gset = -1, gidx = -1;
    // weights packed for the forward / dX kernels (per plan); null: unpacked
    float *wp_f = nullptr, *wp_x = nullptr;
    // this conv's output gradient in the backward (per plan): its own buffer,
    // so the dW reading it on the side stream overlaps the work after it
    float *dyb = nullptr;
    // Side-stream slab sums (per plan): this conv's gradient segment in the
    // side table, or -1 (summed with the rest).
    int fseg = -1;
    long long fblk = 0;
    // Partials per channel of the batch statistics taken by this conv's
    // forward store pass (per plan); -1: they run as a pass of their own.
    int epf = -1;
    rnn_conv_spec spec(uint32_t h, uint32_t w_) const {
        rnn_conv_spec sp;
        rnn_conv_spec_init(&sp, cin, cout, k, stride, pad, h, w_);
        return sp;
    }
};

struct NetBn {
    uint32_t c = 0;
    int g = -1, b = -1;  // parameter indices
    size_t buf = 0;      // rm at buf, rv at buf + c in the buffer array
    float *coef = nullptr;   // device [2c]: batch mean, invstd of the last train forward
    double *part = nullptr;  // device: partial sums of the batch statistics (per plan)
    // partials per channel of the last forward's statistics in part (0: the
    // per-image-range split of the separate pass)
    int pf = 0;
};

struct NetBlock {
    NetConv c1, c2, cd;
    NetBn b1, b2, bd;
    bool down = false;
    uint32_t hin = 0, win = 0, hout = 0, wout = 0;
    float *in = nullptr;  // block input (previous output), not owned
    float *y1 = nullptr, *h = nullptr, *y2 = nullptr, *ys = nullptr, *out = nullptr;
};

}  // namespace

struct rnn_resnet {
    rnn_ctx *ctx = nullptr;
    uint32_t depth = 0, width = 0, nclass = 0;
    NetConv stem;
    NetBn stem_bn;
    std::vector<NetBlock> blocks;
    uint32_t fc_w = 0, fc_b = 0, fin = 0;  // parameter indices, classifier width
    std::vector<ParamSlot> params;         // for_each_param order
    size_t np = 0, ndecay = 0, nbuf = 0;
    float *pv = nullptr, *pg = nullptr, *pm = nullptr, *bufs = nullptr, *coefs = nullptr;
    // Activation plan for (n, h, w).
    size_t n = 0, H = 0, W = 0;
    void *arena = nullptr;
    float *x = nullptr, *y0 = nullptr, *s0 = nullptr, *pooled = nullptr, *logits = nullptr;
    float *dlogits = nullptr, *dpool = nullptr, *d0 = nullptr, *d1 = nullptr, *t1 = nullptr,
          *t2 = nullptr, *t3 = nullptr, *scal = nullptr, *loss = nullptr;
    // Gradient finalisation: one segment per parameter tensor in flat order.
    GradSeg *segs = nullptr;
    int nseg = 0;
    long long nseg_blocks = 0;
    // With the side stream: each conv's segment alone (fsegs, blk0 = 0),
    // its slabs summed into g on the side stream right after its dW; the
    // other segments with slabs (the stem) in rsegs after the join, then the
    // SGD step over every parameter.
    GradSeg *fsegs = nullptr, *rsegs = nullptr;
    int nrseg = 0;
    long long nrseg_blocks = 0;
    uint32_t *labels = nullptr, *correct = nullptr;
    // softmax-CE over several blocks: the last block's ticket (0 between
    // steps) and the row losses / hits
    uint32_t *ce_ticket = nullptr;
    float *ce_rows = nullptr;
    double *part = nullptr;
    // Packed conv weights: one segment per (conv, direction), refreshed by
    // the pass after every SGD step inside the step; packs_dirty marks
    // weights changed outside it (initialisation, copies in, rnn_resnet_step).
    PackSeg *psegs = nullptr;
    int npseg = 0, npblk = 0;
    bool packs_dirty = true;
    // the values last written to scal (lr, momentum, wd, smoothing)
    float scal_host[4] = {0, 0, 0, 0};
    bool scal_valid = false;
    size_t fh = 0, fw = 0;  // feature map at the pooling layer
    bool fwd_train = false;  // last forward saved the backward's activations
    // Graph of the train step for the current plan.
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    hipStream_t rec_stream = nullptr;  // default priority, used only to record
    // Weight gradients run on a second stream (default priority) beside the
    // dX chain: one event per fork (dy ready) and one for the join.
    hipStream_t side = nullptr;
    std::vector<hipEvent_t> events;
    bool overlap = true;
    // batch statistics in the forward convs' store passes
    // (RNN_BN_PASSES=separate: in passes of their own)
    bool fuse_bn = true;
    bool capturing = false;  // recording the step graph: no side stream there
    // The 3x3 stride-1 convs' weight gradients in grouped launches
    // (RNN_DW_GROUP): 1 = one launch after the dX chain; 2 = one per stage
    // (the blocks of one width), on the side stream once the stage's
    // output gradients exist; 0 = each conv's on its own, as the others'.
    int group_dw = 1;
    struct DwGroup {
        DwGroupLaunch L;
        std::vector<DwGroupMember> m;
        std::vector<NetConv *> convs;
        size_t first_block = 0;  // launched once this block's backward is done
        size_t table_off = 0;
    };
    std::vector<DwGroup> dwgs;
    int step_calls = 0;
    bool use_graph = true;
    char graph_err[160] = {0};
};

namespace {

float *pv_of(rnn_resnet *r, int p) { return r->pv + r->params[p].off; }
float *pg_of(rnn_resnet *r, int p) { return r->pg + r->params[p].off; }

void drop_graph(rnn_resnet *r) {
    if (r->gexec) (void)hipGraphExecDestroy(r->gexec);
    if (r->graph) (void)hipGraphDestroy(r->graph);
    r->gexec = nullptr;
    r->graph = nullptr;
    r->step_calls = 0;
}

int add_param(rnn_resnet *r, size_t len, bool decay) {
    ParamSlot s;
    s.len = len;
    s.decay = decay;
    r->params.push_back(s);
    return (int)r->params.size() - 1;
}

NetConv make_conv(uint32_t cin, uint32_t cout, uint32_t k, uint32_t stride, uint32_t pad) {
    NetConv c;
    c.cin = cin;
    c.cout = cout;
    c.k = k;
    c.stride = stride;
    c.pad = pad;
    return c;
}

// Plans the activations for (n, h, w) in one device block.
int plan(rnn_resnet *r, size_t n, size_t H, size_t W) {
    rnn_ctx *ctx = r->ctx;
    if (r->arena && r->n == n && r->H == H && r->W == W) return RNN_OK;
    drop_graph(r);
    if (r->arena) {
        RNN_HIP(ctx, hipStreamSynchronize(ctx->stream));
        RNN_HIP(ctx, hipFree(r->arena));
        r->arena = nullptr;
    }
    WsCarve cv;
    std::vector<std::pair<float **, size_t>> f32;
    const size_t w0 = r->width;
    size_t maxact = n * w0 * H * W, maxpart = rnn_bn_scratch_doubles(n, w0);
    f32.push_back({&r->x, n * 3 * H * W});
    f32.push_back({&r->y0, n * w0 * H * W});
    f32.push_back({&r->s0, n * w0 * H * W});
    size_t h = H, w = W;
    for (auto &b : r->blocks) {
        b.hin = (uint32_t)h;
        b.win = (uint32_t)w;
        rnn_conv_spec sp = b.c1.spec((uint32_t)h, (uint32_t)w);
        b.hout = sp.oh;
        b.wout = sp.ow;
        const size_t a = n * b.c1.cout * sp.oh * sp.ow;
        f32.push_back({&b.y1, a});
        f32.push_back({&b.h, a});
        f32.push_back({&b.y2, a});
        if (b.down) f32.push_back({&b.ys, a});
        f32.push_back({&b.out, a});
        maxact = std::max(maxact, a);
        maxpart = std::max(maxpart, rnn_bn_scratch_doubles(n, b.c1.cout));
        h = sp.oh;
        w = sp.ow;
    }
    r->fh = h;
    r->fw = w;
    f32.push_back({&r->pooled, n * r->fin});
    f32.push_back({&r->dpool, n * r->fin});
    f32.push_back({&r->logits, n * r->nclass});
    f32.push_back({&r->dlogits, n * r->nclass});
    f32.push_back({&r->d0, maxact});
    f32.push_back({&r->d1, maxact});
    f32.push_back({&r->t1, maxact});
    f32.push_back({&r->t2, maxact});
    f32.push_back({&r->t3, maxact});
    f32.push_back({&r->scal, 4});
    f32.push_back({&r->loss, 1});
    for (auto &b : r->blocks) {
        const size_t a = n * b.c1.cout * b.hout * b.wout;
        f32.push_back({&b.c1.dyb, a});
        f32.push_back({&b.c2.dyb, a});
        if (b.down) f32.push_back({&b.cd.dyb, a});
    }
    std::vector<size_t> offs;
    for (auto &e : f32) offs.push_back(cv.take(e.second * sizeof(float)));
    const size_t o_part = cv.take(maxpart * sizeof(double));
    // Store-pass batch statistics: partials per channel of each conv's forward.
    auto ep = [&](NetConv &c, size_t hh, size_t ww) -> int {
        if (!r->fuse_bn) return -1;
        rnn_conv_spec sp = c.spec((uint32_t)hh, (uint32_t)ww);
        return rnn_conv_fast_parts(&sp, n);
    };
    r->stem.epf = ep(r->stem, H, W);
    for (auto &b : r->blocks) {
        b.c1.epf = ep(b.c1, b.hin, b.win);
        b.c2.epf = ep(b.c2, b.hout, b.wout);
        b.cd.epf = b.down ? ep(b.cd, b.hin, b.win) : -1;
    }
    std::vector<std::pair<NetBn *, size_t>> bnparts;
    auto bnpart = [&](NetBn &bn, int pa) {
        const size_t d = std::max(rnn_bn_scratch_doubles(n, bn.c),
                                  (size_t)2 * bn.c * (size_t)std::max(pa, 0));
        bnparts.push_back({&bn, cv.take(d * sizeof(double))});
    };
    bnpart(r->stem_bn, r->stem.epf);
    for (auto &b : r->blocks) {
        bnpart(b.b1, b.c1.epf);
        bnpart(b.b2, b.c2.epf);
        if (b.down) bnpart(b.bd, b.cd.epf);
    }
    // The grouped weight gradients: the 3x3 stride-1 convs but the stem,
    // all in one group or one group per stage (blocks of one width).
    r->dwgs.clear();
    r->stem.grouped = false;
    for (auto &b : r->blocks) b.c1.grouped = b.c2.grouped = b.cd.grouped = false;
    if (r->group_dw) {
        for (size_t i = 0; i < r->blocks.size(); i++) {
            NetBlock &b = r->blocks[i];
            if (r->dwgs.empty() ||
                (r->group_dw == 2 && b.c2.cout != r->blocks[i - 1].c2.cout)) {
                r->dwgs.emplace_back();
                r->dwgs.back().first_block = i;  // its lowest block: the backward's last
            }
            auto &G = r->dwgs.back();
            for (auto pr : {std::make_pair(&b.c1, std::make_pair(b.hin, b.win)),
                            std::make_pair(&b.c2, std::make_pair(b.hout, b.wout))}) {
                DwGroupMember mm;
                mm.sp = pr.first->spec(pr.second.first, pr.second.second);
                if (mm.sp.k != 3 || mm.sp.stride != 1) continue;
                G.m.push_back(mm);
                G.convs.push_back(pr.first);
            }
        }
        for (size_t gi = 0; gi < r->dwgs.size(); gi++) {
            auto &G = r->dwgs[gi];
            if (G.convs.size() < 2 ||
                rnn_conv_dw_group_plan(ctx, n, G.m.data(), (int)G.m.size(), &G.L) != RNN_OK) {
                G.L = DwGroupLaunch();
                continue;
            }
            for (size_t i = 0; i < G.convs.size(); i++) {
                G.convs[i]->grouped = true;
                G.convs[i]->gset = (int)gi;
                G.convs[i]->gidx = (int)i;
            }
        }
    }
    // dW slabs of every conv, and the gradient segment table.
    std::vector<std::pair<NetConv *, size_t>> slabs;
    auto slab = [&](NetConv &c, uint32_t h, uint32_t w) {
        rnn_conv_spec sp = c.spec(h, w);
        const size_t len = (size_t)c.cout * c.cin * c.k * c.k;
        const size_t f = c.grouped ? (size_t)r->dwgs[c.gset].m[c.gidx].nz * len
                                   : rnn_conv_dw_slab_floats(ctx, &sp, n);
        c.nz = f ? (int)(f / len) : 0;
        if (f) slabs.push_back({&c, cv.take(f * sizeof(float))});
    };
    slab(r->stem, (uint32_t)H, (uint32_t)W);
    for (auto &b : r->blocks) {
        slab(b.c1, b.hin, b.win);
        slab(b.c2, b.hout, b.wout);
        if (b.down) slab(b.cd, b.hin, b.win);
    }
    // Packed weights: forward for every conv, dX for all but the stem (whose
    // input gradient is not needed).
    struct PackPlan {
        float **dst;
        PackSeg seg;
        size_t off;
    };
    std::vector<PackPlan> packs;
    auto pack = [&](NetConv &c, uint32_t h, uint32_t w, int dx, float **dst) {
        *dst = nullptr;
        rnn_conv_spec sp = c.spec(h, w);
        PackSeg sg;
        if (rnn_conv_pack_geo(&sp, dx, &sg.geo) != RNN_OK) return;
        packs.push_back({dst, sg, cv.take(sg.geo.floats() * sizeof(float))});
    };
    pack(r->stem, (uint32_t)H, (uint32_t)W, 0, &r->stem.wp_f);
    r->stem.wp_x = nullptr;
    for (auto &b : r->blocks) {
        pack(b.c1, b.hin, b.win, 0, &b.c1.wp_f);
        pack(b.c1, b.hin, b.win, 1, &b.c1.wp_x);
        pack(b.c2, b.hout, b.wout, 0, &b.c2.wp_f);
        pack(b.c2, b.hout, b.wout, 1, &b.c2.wp_x);
        if (b.down) {
            pack(b.cd, b.hin, b.win, 0, &b.cd.wp_f);
            pack(b.cd, b.hin, b.win, 1, &b.cd.wp_x);
        }
    }
    const size_t o_psegs = cv.take(std::max<size_t>(packs.size(), 1) * sizeof(PackSeg));
    const size_t o_segs = cv.take(r->params.size() * sizeof(GradSeg));
    const size_t o_fsegs = cv.take(r->params.size() * sizeof(GradSeg));
    const size_t o_rsegs = cv.take(r->params.size() * sizeof(GradSeg));
    const size_t o_lab = cv.take(n * sizeof(uint32_t));
    const size_t o_cor = cv.take(sizeof(uint32_t));
    const size_t o_tick = cv.take(sizeof(uint32_t));
    const size_t o_cer = cv.take(2 * n * sizeof(float));
    for (auto &G : r->dwgs) G.table_off = cv.take(std::max<size_t>(G.L.table_bytes, 1));
    void *mem = nullptr;
    hipError_t e = hipMalloc(&mem, cv.off);
    if (e != hipSuccess)
        return rnn_fail(ctx, RNN_E_NOMEM, "resnet activations hipMalloc(%zu): %s", cv.off,
                        hipGetErrorString(e));
    r->arena = mem;
    char *base = (char *)mem;
    for (size_t i = 0; i < f32.size(); i++) *f32[i].first = (float *)(base + offs[i]);
    r->part = (double *)(base + o_part);
    for (auto &e : bnparts) e.first->part = (double *)(base + e.second);
    r->stem.slabs = nullptr;
    for (auto &b : r->blocks) b.c1.slabs = b.c2.slabs = b.cd.slabs = nullptr;
    for (auto &e : slabs) e.first->slabs = (float *)(base + e.second);
    // Pack segments: source = the conv's weights in pv, destination relative
    // to the arena.
    std::vector<PackSeg> psegs;
    uint32_t pblk = 0;
    auto conv_of_dst = [&](float **dst) -> const NetConv * {
        if (dst == &r->stem.wp_f) return &r->stem;
        for (auto &b : r->blocks) {
            if (dst == &b.c1.wp_f || dst == &b.c1.wp_x) return &b.c1;
            if (dst == &b.c2.wp_f || dst == &b.c2.wp_x) return &b.c2;
            if (dst == &b.cd.wp_f || dst == &b.cd.wp_x) return &b.cd;
        }
        return nullptr;
    };
    for (auto &pp : packs) {
        *pp.dst = (float *)(base + pp.off);
        PackSeg sg = pp.seg;
        sg.src = r->params[conv_of_dst(pp.dst)->w].off;
        sg.dst = pp.off / sizeof(float);
        sg.blk0 = pblk;
        sg.nblk = (uint32_t)std::min(sg.geo.slabs(), 512);
        pblk += sg.nblk;
        psegs.push_back(sg);
    }
    r->psegs = (PackSeg *)(base + o_psegs);
    r->npseg = (int)psegs.size();
    r->npblk = (int)pblk;
    r->packs_dirty = true;
    r->scal_valid = false;
    if (!psegs.empty()) {
        hipError_t pe = hipMemcpy(r->psegs, psegs.data(), psegs.size() * sizeof(PackSeg),
                                  hipMemcpyHostToDevice);
        if (pe != hipSuccess) {
            (void)hipFree(r->arena);
            r->arena = nullptr;
            return rnn_fail(ctx, RNN_E_HIP, "resnet plan upload: %s", hipGetErrorString(pe));
        }
    }
    // Segment table: parameters in flat order, conv weights with their slabs.
    std::vector<GradSeg> segs(r->params.size());
    std::vector<const NetConv *> conv_of(r->params.size(), nullptr);
    conv_of[r->stem.w] = &r->stem;
    for (auto &b : r->blocks) {
        conv_of[b.c1.w] = &b.c1;
        conv_of[b.c2.w] = &b.c2;
        if (b.down) conv_of[b.cd.w] = &b.cd;
    }
    std::vector<int> order(r->params.size());
    for (size_t i = 0; i < order.size(); i++) order[i] = (int)i;
    std::sort(order.begin(), order.end(),
              [&](int a, int b) { return r->params[a].off < r->params[b].off; });
    long long blk = 0;
    for (size_t k = 0; k < order.size(); k++) {
        const ParamSlot &ps = r->params[order[k]];
        const NetConv *c = conv_of[order[k]];
        GradSeg g;
        g.off = (long long)ps.off;
        g.len = (long long)ps.len;
        g.blk0 = blk;
        g.slabs = c && c->slabs ? c->slabs : nullptr;
        g.nz = g.slabs ? c->nz : 0;
        g.decay = ps.decay ? 1 : 0;
        segs[k] = g;
        blk += (long long)rnn_div_up(ps.len, 32);
    }
    // the segments with slabs split: each conv's but the stem's alone, the rest
    std::vector<GradSeg> fsv, rsv;
    long long rblk = 0;
    for (size_t k = 0; k < order.size(); k++) {
        NetConv *c = const_cast<NetConv *>(conv_of[order[k]]);
        GradSeg g = segs[k];
        if (c) c->fseg = -1;
        if (c && c != &r->stem && !c->grouped && g.slabs) {
            g.blk0 = 0;
            c->fseg = (int)fsv.size();
            c->fblk = (long long)rnn_div_up((size_t)g.len, (size_t)32);
            fsv.push_back(g);
        } else if (g.slabs) {
            g.blk0 = rblk;
            rblk += (long long)rnn_div_up((size_t)g.len, (size_t)32);
            rsv.push_back(g);
        }
    }
    r->fsegs = (GradSeg *)(base + o_fsegs);
    r->rsegs = (GradSeg *)(base + o_rsegs);
    r->nrseg = (int)rsv.size();
    r->nrseg_blocks = rblk;
    for (auto *tab : {&fsv, &rsv}) {
        if (tab->empty()) continue;
        hipError_t fe = hipMemcpy(tab == &fsv ? r->fsegs : r->rsegs, tab->data(),
                                  tab->size() * sizeof(GradSeg), hipMemcpyHostToDevice);
        if (fe != hipSuccess) {
            (void)hipFree(r->arena);
            r->arena = nullptr;
            return rnn_fail(ctx, RNN_E_HIP, "resnet plan upload: %s", hipGetErrorString(fe));
        }
    }
    r->segs = (GradSeg *)(base + o_segs);
    r->nseg = (int)segs.size();
    r->nseg_blocks = blk;
    hipError_t ce = hipMemcpy(r->segs, segs.data(), segs.size() * sizeof(GradSeg),
                              hipMemcpyHostToDevice);
    if (ce != hipSuccess) {
        (void)hipFree(r->arena);
        r->arena = nullptr;
        return rnn_fail(ctx, RNN_E_HIP, "resnet plan upload: %s", hipGetErrorString(ce));
    }
    r->labels = (uint32_t *)(base + o_lab);
    r->correct = (uint32_t *)(base + o_cor);
    r->ce_ticket = (uint32_t *)(base + o_tick);
    r->ce_rows = (float *)(base + o_cer);
    hipError_t te = hipMemset(r->ce_ticket, 0, sizeof(uint32_t));
    if (te != hipSuccess) {
        (void)hipFree(r->arena);
        r->arena = nullptr;
        return rnn_fail(ctx, RNN_E_HIP, "resnet plan: %s", hipGetErrorString(te));
    }
    float *prev = r->s0;
    for (auto &b : r->blocks) {
        b.in = prev;
        prev = b.out;
    }
    // each grouped conv's output gradient buffer, input and slabs
    for (auto &b : r->blocks)
        for (auto pr : {std::make_pair(&b.c1, (const float *)b.in),
                        std::make_pair(&b.c2, (const float *)b.h)}) {
            NetConv &c = *pr.first;
            if (!c.grouped) continue;
            DwGroupMember &mm = r->dwgs[c.gset].m[c.gidx];
            mm.dy = c.dyb;
            mm.x = pr.second;
            mm.slabs = c.slabs;
        }
    for (auto &G : r->dwgs) {
        if (!G.L.njobs) continue;
        G.L.table = base + G.table_off;
        const int ue = rnn_conv_dw_group_upload(ctx, G.m.data(), &G.L);
        if (ue != RNN_OK) {
            (void)hipFree(r->arena);
            r->arena = nullptr;
            return ue;
        }
    }
    r->n = n;
    r->H = H;
    r->W = W;
    r->fwd_train = false;
    return RNN_OK;
}

// The RnnBn view of a layer: parameters, gradients, running statistics,
// batch statistics and partial sums.
RnnBn bn_state(rnn_resnet *r, const NetBn &bn) {
    RnnBn s;
    s.part = bn.part;
    s.mom = 0.1f;
    s.eps = 1e-5f;
    s.mean = bn.coef;
    s.invstd = bn.coef + bn.c;
    s.rm = r->bufs + bn.buf;
    s.rv = s.rm + bn.c;
    s.gamma = pv_of(r, bn.g);
    s.beta = pv_of(r, bn.b);
    s.dgamma = pg_of(r, bn.g);
    s.dbeta = pg_of(r, bn.b);
    return s;
}

// The same view with the partial count of the last forward's statistics.
RnnBn bn_fwd(rnn_resnet *r, const NetBn &bn) {
    RnnBn s = bn_state(r, bn);
    s.P = bn.pf;
    return s;
}

#define TRY(expr)                 \
    do {                          \
        int st_ = (expr);         \
        if (st_ != RNN_OK) return st_; \
    } while (0)

// Re-packs every conv's weights from pv (one launch).
int pack_all(rnn_resnet *r) {
    r->packs_dirty = false;
    return rnn_conv_pack_multi_launch(r->ctx, r->psegs, r->npseg, r->npblk, r->pv,
                                      (float *)r->arena);
}

// ResNet::forward (model.rs:138-150) with BasicBlock::forward (model.rs:39-57).
// The packed weights must be current (callers run pack_all when
// packs_dirty).
// Train mode: each BN's partial sums are taken right after its conv and
// finalised inside the kernel that applies the BN.
int forward(rnn_resnet *r, bool train) {
    rnn_ctx *ctx = r->ctx;
    const size_t n = r->n;
    const bool ev = !train;
    // conv c of src into y, with (train) the batch statistics' partial sums of
    // bn: in the conv's store pass, or by a pass of their own
    auto conv_bn = [&](NetConv &c, const rnn_conv_spec &sp, const float *src, float *y,
                       NetBn &bn) -> int {
        if (train && c.epf > 0) {
            bn.pf = c.epf;
            return rnn_conv2d_forward_stats(ctx, &sp, n, src, pv_of(r, c.w), c.wp_f, y, bn.part);
        }
        TRY(rnn_conv2d_forward_wp(ctx, &sp, n, src, pv_of(r, c.w), c.wp_f, y));
        bn.pf = 0;
        if (train) return rnn_bn_stats_launch(ctx, n, bn.c, (size_t)sp.oh * sp.ow, y, bn.part);
        return RNN_OK;
    };
    rnn_conv_spec sp = r->stem.spec((uint32_t)r->H, (uint32_t)r->W);
    const size_t hw0 = (size_t)sp.oh * sp.ow;
    TRY(conv_bn(r->stem, sp, r->x, r->y0, r->stem_bn));
    TRY(rnn_bn_apply_launch(ctx, n, r->stem_bn.c, hw0, r->y0, bn_fwd(r, r->stem_bn), ev, 1, 0,
                            nullptr, nullptr, r->s0));
    for (auto &b : r->blocks) {
        const size_t hw = (size_t)b.hout * b.wout;
        rnn_conv_spec s1 = b.c1.spec(b.hin, b.win);
        TRY(conv_bn(b.c1, s1, b.in, b.y1, b.b1));
        TRY(rnn_bn_apply_launch(ctx, n, b.b1.c, hw, b.y1, bn_fwd(r, b.b1), ev, 1, 0, nullptr,
                                nullptr, b.h));
        rnn_conv_spec s2 = b.c2.spec(b.hout, b.wout);
        TRY(conv_bn(b.c2, s2, b.h, b.y2, b.b2));
        if (b.down) {
            rnn_conv_spec sd = b.cd.spec(b.hin, b.win);
            TRY(conv_bn(b.cd, sd, b.in, b.ys, b.bd));
            const RnnBn sd_bn = bn_fwd(r, b.bd);
            TRY(rnn_bn_apply_launch(ctx, n, b.b2.c, hw, b.y2, bn_fwd(r, b.b2), ev, 1, 2, b.ys,
                                    &sd_bn, b.out));
        } else {
            TRY(rnn_bn_apply_launch(ctx, n, b.b2.c, hw, b.y2, bn_fwd(r, b.b2), ev, 1, 1, b.in,
                                    nullptr, b.out));
        }
    }
    const float *feat = r->blocks.empty() ? r->s0 : r->blocks.back().out;
    TRY(rnn_gap_fc_forward_launch(ctx, n, r->fin, r->fh * r->fw, r->nclass, feat,
                                  pv_of(r, r->fc_w), pv_of(r, r->fc_b), r->pooled, r->logits));
    r->fwd_train = train;
    return RNN_OK;
}

// dW of one conv: into its slabs (summed at the end of the backward), or
// straight into the gradient when the shape has no slab plan.
int conv_dw(rnn_resnet *r, const NetConv &c, const rnn_conv_spec &sp, const float *dy,
            const float *x) {
    if (c.slabs) return rnn_conv_dw_slabs(r->ctx, &sp, r->n, dy, x, c.slabs, nullptr);
    return rnn_conv2d_backward_w(r->ctx, &sp, r->n, dy, x, pg_of(r, c.w));
}

// The starting gradient of the BN layers that consume activation `a` of the
// backward: the second BN of the block before block i, plus its shortcut BN
// (i == 0: the stem BN).  resid_bwd computes their partial sums in the pass
// that produces that gradient.
struct ResidTarget {
    const NetBn *b1, *b2;
    const float *x1, *x2;
};

ResidTarget resid_target(rnn_resnet *r, size_t i) {
    if (i == 0) return {&r->stem_bn, nullptr, r->y0, nullptr};
    const NetBlock &p = r->blocks[i - 1];
    return {&p.b2, p.down ? &p.bd : nullptr, p.y2, p.down ? p.ys : nullptr};
}

int resid(rnn_resnet *r, size_t i, size_t c, size_t hw, float *a, const float *add,
          const float *mask, const float *gsrc) {
    const ResidTarget t = resid_target(r, i);
    const RnnBn s1 = bn_state(r, *t.b1);
    RnnBn s2;
    if (t.b2) s2 = bn_state(r, *t.b2);
    return rnn_resid_bwd_launch(r->ctx, r->n, c, hw, a, add, mask, gsrc, s1, t.x1, t.b1->part,
                                t.b2 ? &s2 : nullptr, t.x2, t.b2 ? t.b2->part : nullptr);
}

// ResNet::backward (model.rs:152-162) with BasicBlock::backward
// (model.rs:59-77).  A block's starting gradient d = relu_back_(.., out) is
// produced by one pass that also takes the partial sums of the BN backwards
// reading d (the block's second BN and its shortcut BN): for the last block
// the GAP backward, for the others the pass after the next block's first dX
// that adds the shortcut term (the residual add_) and masks by that block's
// input -- the previous block's output, or the stem's ReLU output, whose BN
// is then the one summed.  Those BN backwards then only apply dx.
// relu_back_ by h is folded into the first BN backward that reads c2's dX.
// The conv weight gradients are left as slabs; the finalisation adds them
// into pg (Param::g) -- and with `sgd` also takes the Nesterov step -- in one
// pass over all parameters.
// dW of conv c on the side stream once dy (written just before on the main
// stream) is ready; dy stays untouched until the join.
bool use_side(const rnn_resnet *r) { return r->overlap && !r->capturing; }

// The side stream waits for the work issued so far on the main stream.
int fork_side(rnn_resnet *r, size_t &ev) {
    rnn_ctx *ctx = r->ctx;
    if (!r->side) RNN_HIP(ctx, hipStreamCreateWithFlags(&r->side, hipStreamNonBlocking));
    if (ev == r->events.size()) {
        hipEvent_t e;
        RNN_HIP(ctx, hipEventCreateWithFlags(&e, hipEventDisableTiming));
        r->events.push_back(e);
    }
    hipEvent_t e = r->events[ev++];
    RNN_HIP(ctx, hipEventRecord(e, ctx->stream));
    RNN_HIP(ctx, hipStreamWaitEvent(r->side, e, 0));
    return RNN_OK;
}

int conv_dw_side(rnn_resnet *r, const NetConv &c, const rnn_conv_spec &sp, const float *dy,
                 const float *x, size_t &ev) {
    rnn_ctx *ctx = r->ctx;
    if (!use_side(r)) return conv_dw(r, c, sp, dy, x);
    TRY(fork_side(r, ev));
    hipStream_t main = ctx->stream;
    ctx->stream = r->side;
    int rc = conv_dw(r, c, sp, dy, x);
    // its slab sums into g right away, off the step's critical tail
    if (rc == RNN_OK && c.fseg >= 0)
        rc = rnn_grad_finalize_launch(ctx, r->fsegs + c.fseg, 1, c.fblk, r->pv, r->pg, r->pm,
                                      r->scal, 0);
    ctx->stream = main;
    return rc;
}

// The main stream waits for every dW issued on the side stream.
int join_side(rnn_resnet *r, size_t &ev) {
    rnn_ctx *ctx = r->ctx;
    if (!use_side(r) || ev == 0) return RNN_OK;
    if (ev == r->events.size()) {
        hipEvent_t e;
        RNN_HIP(ctx, hipEventCreateWithFlags(&e, hipEventDisableTiming));
        r->events.push_back(e);
    }
    hipEvent_t e = r->events[ev++];
    RNN_HIP(ctx, hipEventRecord(e, r->side));
    RNN_HIP(ctx, hipStreamWaitEvent(ctx->stream, e, 0));
    return RNN_OK;
}

int backward(rnn_resnet *r, const float *dlogits, bool sgd) {
    rnn_ctx *ctx = r->ctx;
    const size_t n = r->n, nb = r->blocks.size();
    size_t ev = 0;
    if (use_side(r)) {
        // the classifier's weight gradient on the side stream, its input
        // gradient on the main one
        TRY(fork_side(r, ev));
        hipStream_t main = ctx->stream;
        ctx->stream = r->side;
        const int rc = rnn_fc_backward_launch(ctx, n, r->fin, r->nclass, dlogits, r->pooled,
                                              pv_of(r, r->fc_w), pg_of(r, r->fc_w),
                                              pg_of(r, r->fc_b), nullptr);
        ctx->stream = main;
        TRY(rc);
        TRY(rnn_fc_backward_launch(ctx, n, r->fin, r->nclass, dlogits, r->pooled,
                                   pv_of(r, r->fc_w), nullptr, nullptr, r->dpool));
    } else {
        TRY(rnn_fc_backward_launch(ctx, n, r->fin, r->nclass, dlogits, r->pooled,
                                   pv_of(r, r->fc_w), pg_of(r, r->fc_w), pg_of(r, r->fc_b),
                                   r->dpool));
    }
    const float *feat = nb == 0 ? r->s0 : r->blocks.back().out;
    // GAP backward (nn.rs:465-473) masked by the last ReLU output
    TRY(resid(r, nb, r->fin, r->fh * r->fw, r->d0, nullptr, feat, r->dpool));
    float *d = r->d0, *other = r->d1;
    for (size_t i = nb; i-- > 0;) {
        NetBlock &b = r->blocks[i];
        const size_t hw = (size_t)b.hout * b.wout;
        // a conv's output gradient keeps a buffer of its own while a dW
        // reads it later (on the side stream, or in the grouped launch)
        float *dy2 = use_side(r) || b.c2.grouped ? b.c2.dyb : r->t1;
        TRY(rnn_bn_backward_apply_launch(ctx, n, b.b2.c, hw, d, nullptr, b.y2,
                                         bn_state(r, b.b2), b.b2.part, dy2));
        rnn_conv_spec s2 = b.c2.spec(b.hout, b.wout);
        if (!b.c2.grouped) TRY(conv_dw_side(r, b.c2, s2, dy2, b.h, ev));
        TRY(rnn_conv2d_backward_x_wp(ctx, &s2, n, dy2, pv_of(r, b.c2.w), b.c2.wp_x, r->t2));
        float *dy1 = use_side(r) || b.c1.grouped ? b.c1.dyb : r->t1;
        TRY(rnn_bn_backward_launch(ctx, n, b.b1.c, hw, r->t2, b.h, b.y1, bn_state(r, b.b1),
                                   r->part, dy1));
        rnn_conv_spec s1 = b.c1.spec(b.hin, b.win);
        if (!b.c1.grouped) TRY(conv_dw_side(r, b.c1, s1, dy1, b.in, ev));
        TRY(rnn_conv2d_backward_x_wp(ctx, &s1, n, dy1, pv_of(r, b.c1.w), b.c1.wp_x, other));
        const float *add = d;  // dx = c1 dX + d (add_, model.rs:72)
        if (b.down) {
            float *dyd = use_side(r) ? b.cd.dyb : r->t2;
            TRY(rnn_bn_backward_apply_launch(ctx, n, b.bd.c, hw, d, nullptr, b.ys,
                                             bn_state(r, b.bd), b.bd.part, dyd));
            rnn_conv_spec sd = b.cd.spec(b.hin, b.win);
            TRY(conv_dw_side(r, b.cd, sd, dyd, b.in, ev));
            TRY(rnn_conv2d_backward_x_wp(ctx, &sd, n, dyd, pv_of(r, b.cd.w), b.cd.wp_x, r->t3));
            add = r->t3;  // dx = c1 dX + shortcut dX (add_, model.rs:70-71)
        }
        TRY(resid(r, i, b.c1.cin, (size_t)b.hin * b.win, other, add, b.in, nullptr));
        std::swap(d, other);
        if (r->group_dw == 2 && use_side(r))
            for (auto &G : r->dwgs)
                if (G.first_block == i && G.L.njobs) {
                    // this stage's output gradients are all written
                    TRY(fork_side(r, ev));
                    hipStream_t main = ctx->stream;
                    ctx->stream = r->side;
                    const int rc = rnn_conv_dw_group_launch(ctx, &G.L);
                    ctx->stream = main;
                    TRY(rc);
                }
    }
    rnn_conv_spec sp = r->stem.spec((uint32_t)r->H, (uint32_t)r->W);
    // d is already relu_back_'d by the stem output (model.rs:159)
    TRY(rnn_bn_backward_apply_launch(ctx, n, r->stem_bn.c, (size_t)sp.oh * sp.ow, d, nullptr,
                                     r->y0, bn_state(r, r->stem_bn), r->stem_bn.part, r->t1));
    // The stem's dX would be the image gradient: discarded (model.rs:161).
    TRY(conv_dw(r, r->stem, sp, r->t1, r->x));
    // the last grouped weight gradients, their output gradients all written
    for (auto &G : r->dwgs)
        if (!(r->group_dw == 2 && use_side(r))) TRY(rnn_conv_dw_group_launch(ctx, &G.L));
    if (use_side(r)) {
        // the side stream summed the other convs' slabs into g
        TRY(join_side(r, ev));
        TRY(rnn_grad_finalize_launch(ctx, r->rsegs, r->nrseg, r->nrseg_blocks, r->pv, r->pg,
                                     r->pm, r->scal, 0));
        if (!sgd) return RNN_OK;
        TRY(rnn_sgd_launch(ctx, r->np, r->ndecay, r->pv, r->pg, r->pm, 0.f, 0.f, 0.f, r->scal));
        return pack_all(r);
    }
    TRY(rnn_grad_finalize_launch(ctx, r->segs, r->nseg, r->nseg_blocks, r->pv, r->pg, r->pm,
                                 r->scal, sgd ? 1 : 0));
    // the step changed the weights: their packed copies follow
    return sgd ? pack_all(r) : RNN_OK;
}

int sgd(rnn_resnet *r, const float *scal, float lr, float mom, float wd) {
    return rnn_sgd_launch(r->ctx, r->np, r->ndecay, r->pv, r->pg, r->pm, lr, mom, wd, scal);
}

// One train step on the inputs already in r->x / r->labels, scalars in
// r->scal: forward, softmax-CE, backward, SGD (train.rs:686-699).
int step_body(rnn_resnet *r) {
    TRY(forward(r, true));
    TRY(rnn_softmax_ce_launch(r->ctx, r->n, r->nclass, r->logits, r->labels, 0.0f, r->scal,
                              r->dlogits, r->loss, r->correct, r->ce_ticket, r->ce_rows));
    return backward(r, r->dlogits, true);
}

// Runs one step: eagerly, or through the recorded graph (recording it on the
// second call of a plan).  If recording fails nothing of the step has run: the
// reason is kept, the network stays eager and the step runs now.
int run_step(rnn_resnet *r) {
    rnn_ctx *ctx = r->ctx;
    if (r->packs_dirty) TRY(pack_all(r));
    if (!r->use_graph || r->step_calls == 0) return step_body(r);
    if (!r->gexec) {
        // Recording needs a stream of its own (the caller's may be the null
        // stream, which cannot record).  Recording runs nothing, so no
        // ordering with the caller's stream is needed here; the replay is
        // launched on the caller's stream below.
        if (!r->rec_stream)
            RNN_HIP(ctx, hipStreamCreateWithFlags(&r->rec_stream, hipStreamNonBlocking));
        hipStream_t caller = ctx->stream;
        ctx->stream = r->rec_stream;
        hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
        int st = RNN_E_HIP;
        hipGraph_t g = nullptr;
        if (e == hipSuccess) {
            r->capturing = true;
            st = step_body(r);
            r->capturing = false;
            e = hipStreamEndCapture(ctx->stream, &g);
        }
        ctx->stream = caller;
        if (st == RNN_OK && e == hipSuccess && g) {
            r->graph = g;
            e = hipGraphInstantiate(&r->gexec, g, nullptr, nullptr, 0);
        } else if (g) {
            (void)hipGraphDestroy(g);
        }
        if (st != RNN_OK || e != hipSuccess || !r->gexec) {
            const int calls = r->step_calls;
            drop_graph(r);
            r->step_calls = calls;
            snprintf(r->graph_err, sizeof(r->graph_err), "capture: status %d, %s", st,
                     hipGetErrorString(e));
            (void)hipGetLastError();
            r->use_graph = false;
            return step_body(r);
        }
    }
    RNN_HIP(ctx, hipGraphLaunch(r->gexec, ctx->stream));
    return RNN_OK;
}

bool shape_ok(rnn_resnet *r, size_t n, size_t h, size_t w) {
    return n > 0 && h >= 4 && w >= 4 && n <= 8192 && n * r->width * h * w < (1ull << 32);
}

}  // namespace

extern "C" {

int rnn_resnet_create(rnn_ctx *ctx, size_t depth_n, size_t width, size_t nclass, uint64_t seed,
                      rnn_resnet **out) {
    if (!ctx || !out) return RNN_E_NULL;
    *out = nullptr;
    if (depth_n == 0 || width == 0 || nclass == 0 || width > 4096 || nclass > 65536 ||
        depth_n > 1024)
        return rnn_fail(ctx, RNN_E_INVALID, "resnet_create: depth %zu width %zu nclass %zu",
                        depth_n, width, nclass);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    rnn_resnet *r = new rnn_resnet();
    r->ctx = ctx;
    r->depth = (uint32_t)depth_n;
    r->width = (uint32_t)width;
    r->nclass = (uint32_t)nclass;
    // Steps run eagerly with the weight gradients on a second stream
    // (RNN_DW_OVERLAP=0: on the main stream) unless RNN_GRAPH=1 or
    // rnn_resnet_set_graph asks for the recorded graph: in a graph the
    // cross-stream edges cost more than the overlap gains, so a recorded step
    // keeps every kernel on one stream.
    const char *ov = getenv("RNN_DW_OVERLAP");
    r->overlap = !(ov && ov[0] == '0');
    const char *g = getenv("RNN_GRAPH");
    r->use_graph = g ? g[0] != '0' : !r->overlap;
    const char *bp = getenv("RNN_BN_PASSES");
    r->fuse_bn = !(bp && strcmp(bp, "separate") == 0);
    const char *gd = getenv("RNN_DW_GROUP");
    if (gd) r->group_dw = gd[0] == '2' ? 2 : gd[0] == '0' ? 0 : 1;
    // ResNet::new (model.rs:113-135): blocks first (their convs draw from the
    // Rng in c1, c2, shortcut order), then the stem conv, then the classifier.
    const uint32_t widths[3] = {(uint32_t)width, (uint32_t)width * 2, (uint32_t)width * 4};
    uint32_t cin = (uint32_t)width;
    size_t nbuf = 0;
    auto make_bn = [&](uint32_t c) {
        NetBn bn;
        bn.c = c;
        bn.buf = nbuf;
        nbuf += 2 * c;
        return bn;
    };
    // Visit order (for_each_param, model.rs:164-175 / 79-91): stem w, stem BN
    // g, b; per block c1 w, b1 g, b, c2 w, b2 g, b, [shortcut w, g, b]; fc w, b.
    r->stem = make_conv(3, (uint32_t)width, 3, 1, 1);
    r->stem.w = add_param(r, (size_t)width * 27, true);
    r->stem_bn = make_bn((uint32_t)width);
    r->stem_bn.g = add_param(r, width, false);
    r->stem_bn.b = add_param(r, width, false);
    for (int s = 0; s < 3; s++)
        for (size_t bi = 0; bi < depth_n; bi++) {
            const uint32_t co = widths[s];
            const uint32_t stride = (s > 0 && bi == 0) ? 2 : 1;
            NetBlock b;
            b.c1 = make_conv(cin, co, 3, stride, 1);
            b.c1.w = add_param(r, (size_t)co * cin * 9, true);
            b.b1 = make_bn(co);
            b.b1.g = add_param(r, co, false);
            b.b1.b = add_param(r, co, false);
            b.c2 = make_conv(co, co, 3, 1, 1);
            b.c2.w = add_param(r, (size_t)co * co * 9, true);
            b.b2 = make_bn(co);
            b.b2.g = add_param(r, co, false);
            b.b2.b = add_param(r, co, false);
            b.down = stride != 1 || cin != co;
            if (b.down) {
                b.cd = make_conv(cin, co, 1, stride, 0);
                b.cd.w = add_param(r, (size_t)co * cin, true);
                b.bd = make_bn(co);
                b.bd.g = add_param(r, co, false);
                b.bd.b = add_param(r, co, false);
            }
            r->blocks.push_back(b);
            cin = co;
        }
    r->fin = cin;
    r->fc_w = add_param(r, (size_t)cin * nclass, true);
    r->fc_b = add_param(r, nclass, false);
    r->nbuf = nbuf;
    // Flat layout: weight-decayed parameters first, each group in visit order.
    size_t off = 0;
    for (int pass = 0; pass < 2; pass++)
        for (auto &p : r->params)
            if (p.decay == (pass == 0)) {
                p.off = off;
                off += p.len;
                if (pass == 0) r->ndecay = off;
            }
    r->np = off;
    // Host values: Kaiming draws in creation order, BN gamma 1 (0 for the
    // second BN of a block, model.rs:22-23), beta 0, classifier * 0.5.
    std::vector<float> hv(r->np, 0.0f), hb(r->nbuf, 0.0f);
    HostRng rng(seed);
    auto kaiming = [&](int p, size_t fan_in) {
        const float sc = sqrtf(2.0f / (float)fan_in);
        float *v = hv.data() + r->params[p].off;
        for (size_t i = 0; i < r->params[p].len; i++) v[i] = rng.normal() * sc;
    };
    auto bn_init = [&](const NetBn &bn, float gamma) {
        float *gv = hv.data() + r->params[bn.g].off;
        for (uint32_t i = 0; i < bn.c; i++) gv[i] = gamma;
        for (uint32_t i = 0; i < bn.c; i++) hb[bn.buf + bn.c + i] = 1.0f;  // running var
    };
    for (auto &b : r->blocks) {
        kaiming(b.c1.w, (size_t)b.c1.cin * 9);
        kaiming(b.c2.w, (size_t)b.c2.cin * 9);
        if (b.down) kaiming(b.cd.w, b.cd.cin);
        bn_init(b.b1, 1.0f);
        bn_init(b.b2, 0.0f);
        if (b.down) bn_init(b.bd, 1.0f);
    }
    kaiming(r->stem.w, 27);
    bn_init(r->stem_bn, 1.0f);
    kaiming(r->fc_w, cin);
    {
        float *v = hv.data() + r->params[r->fc_w].off;
        for (size_t i = 0; i < r->params[r->fc_w].len; i++) v[i] = v[i] * 0.5f;
    }
    // Device state: v, g, m, buffers, BN coefficients.
    size_t ncoef = 2 * (size_t)r->stem_bn.c;
    for (auto &b : r->blocks) ncoef += 2 * (size_t)(b.b1.c + b.b2.c + (b.down ? b.bd.c : 0));
    const size_t bytes = (3 * r->np + r->nbuf + ncoef) * sizeof(float);
    void *mem = nullptr;
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMalloc(&mem, bytes);
    if (e != hipSuccess) {
        delete r;
        return rnn_fail(ctx, RNN_E_NOMEM, "resnet_create hipMalloc(%zu): %s", bytes,
                        hipGetErrorString(e));
    }
    r->pv = (float *)mem;
    r->pg = r->pv + r->np;
    r->pm = r->pg + r->np;
    r->bufs = r->pm + r->np;
    r->coefs = r->bufs + r->nbuf;
    float *cp = r->coefs;
    auto give = [&](NetBn &bn) {
        bn.coef = cp;
        cp += 2 * (size_t)bn.c;
    };
    give(r->stem_bn);
    for (auto &b : r->blocks) {
        give(b.b1);
        give(b.b2);
        if (b.down) give(b.bd);
    }
    e = hipMemcpy(r->pv, hv.data(), r->np * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(r->pg, 0, 2 * r->np * sizeof(float));
    if (e == hipSuccess)
        e = hipMemcpy(r->bufs, hb.data(), r->nbuf * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(r->coefs, 0, ncoef * sizeof(float));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(mem);
        delete r;
        return rnn_fail(ctx, RNN_E_HIP, "resnet_create upload: %s", hipGetErrorString(e));
    }
    *out = r;
    return RNN_OK;
}

int rnn_resnet_destroy(rnn_resnet *r) {
    if (!r) return RNN_E_NULL;
    rnn_ctx *ctx = r->ctx;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    (void)hipStreamSynchronize(ctx->stream);
    drop_graph(r);
    if (r->rec_stream) (void)hipStreamDestroy(r->rec_stream);
    if (r->side) {
        (void)hipStreamSynchronize(r->side);
        (void)hipStreamDestroy(r->side);
    }
    for (hipEvent_t e : r->events) (void)hipEventDestroy(e);
    if (r->arena) (void)hipFree(r->arena);
    if (r->pv) (void)hipFree(r->pv);
    delete r;
    return RNN_OK;
}

size_t rnn_resnet_num_params(const rnn_resnet *r) { return r ? r->np : 0; }
size_t rnn_resnet_num_buffers(const rnn_resnet *r) { return r ? r->nbuf : 0; }
size_t rnn_resnet_num_tensors(const rnn_resnet *r) { return r ? r->params.size() : 0; }

int rnn_resnet_tensor_len(const rnn_resnet *r, size_t i, size_t *len, int *decay) {
    if (!r || !len) return RNN_E_NULL;
    if (i >= r->params.size()) return rnn_fail(r->ctx, RNN_E_INVALID, "tensor %zu out of range", i);
    *len = r->params[i].len;
    if (decay) *decay = r->params[i].decay ? 1 : 0;
    return RNN_OK;
}

int rnn_resnet_copy(rnn_resnet *r, int which, float *dst, const float *src) {
    if (!r) return RNN_E_NULL;
    rnn_ctx *ctx = r->ctx;
    if ((dst == nullptr) == (src == nullptr))
        return rnn_fail(ctx, RNN_E_INVALID, "resnet_copy: exactly one of dst / src");
    if (which < 0 || which > 3) return rnn_fail(ctx, RNN_E_INVALID, "resnet_copy: which %d", which);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (which == 3) {
        const size_t bytes = r->nbuf * sizeof(float);
        if (dst)
            RNN_HIP(ctx, hipMemcpyAsync(dst, r->bufs, bytes, hipMemcpyDeviceToDevice, ctx->stream));
        else
            RNN_HIP(ctx, hipMemcpyAsync(r->bufs, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
        return RNN_OK;
    }
    float *base = which == 0 ? r->pv : which == 1 ? r->pg : r->pm;
    if (which == 0 && src) r->packs_dirty = true;
    size_t pos = 0;  // position in for_each_param order
    for (auto &p : r->params) {
        if (dst)
            RNN_HIP(ctx, hipMemcpyAsync(dst + pos, base + p.off, p.len * sizeof(float),
                                        hipMemcpyDeviceToDevice, ctx->stream));
        else
            RNN_HIP(ctx, hipMemcpyAsync(base + p.off, src + pos, p.len * sizeof(float),
                                        hipMemcpyDeviceToDevice, ctx->stream));
        pos += p.len;
    }
    return RNN_OK;
}

int rnn_resnet_forward(rnn_resnet *r, size_t n, size_t h, size_t w, const float *x, int train,
                       float *logits) {
    if (!r) return RNN_E_NULL;
    rnn_ctx *ctx = r->ctx;
    if (!x || !logits) return rnn_fail(ctx, RNN_E_NULL, "resnet_forward: null pointer");
    if (!shape_ok(r, n, h, w))
        return rnn_fail(ctx, RNN_E_INVALID, "resnet_forward: n %zu h %zu w %zu", n, h, w);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    TRY(plan(r, n, h, w));
    RNN_HIP(ctx, hipMemcpyAsync(r->x, x, n * 3 * h * w * sizeof(float), hipMemcpyDeviceToDevice,
                                ctx->stream));
    if (r->packs_dirty) TRY(pack_all(r));
    TRY(forward(r, train != 0));
    RNN_HIP(ctx, hipMemcpyAsync(logits, r->logits, n * r->nclass * sizeof(float),
                                hipMemcpyDeviceToDevice, ctx->stream));
    return RNN_OK;
}

int rnn_resnet_backward(rnn_resnet *r, const float *dlogits) {
    if (!r) return RNN_E_NULL;
    rnn_ctx *ctx = r->ctx;
    if (!dlogits) return rnn_fail(ctx, RNN_E_NULL, "resnet_backward: null pointer");
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!r->arena || !r->fwd_train)
        return rnn_fail(ctx, RNN_E_INVALID, "resnet_backward: no train-mode forward to differentiate");
    RNN_HIP(ctx, hipMemcpyAsync(r->dlogits, dlogits, r->n * r->nclass * sizeof(float),
                                hipMemcpyDeviceToDevice, ctx->stream));
    return backward(r, r->dlogits, false);
}

int rnn_resnet_step(rnn_resnet *r, float lr, float momentum, float wd) {
    if (!r) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(r->ctx->mu);
    r->packs_dirty = true;
    return sgd(r, nullptr, lr, momentum, wd);
}

int rnn_resnet_train_step(rnn_resnet *r, size_t n, size_t h, size_t w, const float *x,
                          const uint32_t *labels, float smooth, float lr, float momentum, float wd,
                          float *loss, uint32_t *correct) {
    if (!r) return RNN_E_NULL;
    rnn_ctx *ctx = r->ctx;
    if (!x != !labels)
        return rnn_fail(ctx, RNN_E_NULL, "resnet_train_step: x and labels must both be set "
                                         "or both be NULL");
    if (!shape_ok(r, n, h, w))
        return rnn_fail(ctx, RNN_E_INVALID, "resnet_train_step: n %zu h %zu w %zu", n, h, w);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!x) {
        if (!r->arena || r->n != n || r->H != h || r->W != w)
            return rnn_fail(ctx, RNN_E_INVALID,
                            "resnet_train_step: no input slots of this shape (rnn_resnet_inputs)");
    } else {
        TRY(plan(r, n, h, w));
        RNN_HIP(ctx, hipMemcpyAsync(r->x, x, n * 3 * h * w * sizeof(float),
                                    hipMemcpyDeviceToDevice, ctx->stream));
        RNN_HIP(ctx, hipMemcpyAsync(r->labels, labels, n * sizeof(uint32_t),
                                    hipMemcpyDeviceToDevice, ctx->stream));
    }
    // the step scalars live in r->scal; rewrite them only when they change
    const float sc[4] = {lr, momentum, wd, smooth};
    if (!r->scal_valid || std::memcmp(sc, r->scal_host, sizeof(sc)) != 0) {
        TRY(rnn_set_scalars_launch(ctx, r->scal, lr, momentum, wd, smooth));
        std::memcpy(r->scal_host, sc, sizeof(sc));
        r->scal_valid = true;
    }
    // The first call of a plan runs eagerly (it also sizes the shared
    // workspace); the second records the graph; later calls replay it.
    TRY(run_step(r));
    r->step_calls++;
    r->fwd_train = true;
    if (loss)
        RNN_HIP(ctx, hipMemcpyAsync(loss, r->loss, sizeof(float), hipMemcpyDeviceToDevice,
                                    ctx->stream));
    if (correct)
        RNN_HIP(ctx, hipMemcpyAsync(correct, r->correct, sizeof(uint32_t),
                                    hipMemcpyDeviceToDevice, ctx->stream));
    return RNN_OK;
}

int rnn_resnet_inputs(rnn_resnet *r, size_t n, size_t h, size_t w, float **x,
                      uint32_t **labels) {
    if (!r) return RNN_E_NULL;
    rnn_ctx *ctx = r->ctx;
    if (!x || !labels) return rnn_fail(ctx, RNN_E_NULL, "resnet_inputs: null pointer");
    if (!shape_ok(r, n, h, w))
        return rnn_fail(ctx, RNN_E_INVALID, "resnet_inputs: n %zu h %zu w %zu", n, h, w);
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    TRY(plan(r, n, h, w));
    *x = r->x;
    *labels = r->labels;
    return RNN_OK;
}

int rnn_resnet_set_graph(rnn_resnet *r, int on) {
    if (!r) return RNN_E_NULL;
    std::lock_guard<std::recursive_mutex> lk(r->ctx->mu);
    RNN_HIP(r->ctx, hipStreamSynchronize(r->ctx->stream));
    drop_graph(r);
    r->use_graph = on != 0;
    r->graph_err[0] = 0;
    return RNN_OK;
}

int rnn_resnet_graph_state(const rnn_resnet *r, const char **why) {
    if (!r) return RNN_E_NULL;
    if (why) *why = r->graph_err;
    return r->gexec ? 1 : 0;
}

int rnn_resnet_logits(rnn_resnet *r, float *logits) {
    if (!r || !logits) return RNN_E_NULL;
    rnn_ctx *ctx = r->ctx;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    if (!r->arena) return rnn_fail(ctx, RNN_E_INVALID, "resnet_logits: no forward yet");
    RNN_HIP(ctx, hipMemcpyAsync(logits, r->logits, r->n * r->nclass * sizeof(float),
                                hipMemcpyDeviceToDevice, ctx->stream));
    return RNN_OK;
}

int rnn_dbg_resnet_buffer(rnn_resnet *r, size_t block, int which, const float **ptr,
                          size_t *len) {
    if (!r || !ptr || !len) return RNN_E_NULL;
    *ptr = nullptr;
    *len = 0;
    if (!r->arena) return rnn_fail(r->ctx, RNN_E_INVALID, "dbg_resnet_buffer: no plan yet");
    if (block >= r->blocks.size())
        return rnn_fail(r->ctx, RNN_E_INVALID, "dbg_resnet_buffer: block %zu of %zu", block,
                        r->blocks.size());
    const NetBlock &b = r->blocks[block];
    const size_t a = r->n * b.c1.cout * b.hout * b.wout;
    const float *tab[11] = {b.y1,     b.h,      b.y2,      b.ys,      b.out,   b.c1.dyb,
                            b.c2.dyb, b.cd.dyb, b.b1.coef, b.b2.coef, b.in};
    if (which < 0 || which > 10 || !tab[which])
        return rnn_fail(r->ctx, RNN_E_INVALID, "dbg_resnet_buffer: no buffer %d", which);
    *ptr = tab[which];
    *len = which == 10 ? r->n * (size_t)b.c1.cin * b.hin * b.win
                       : (which >= 8 ? 2 * (size_t)b.c1.cout : a);
    return RNN_OK;
}

int rnn_dbg_resnet_dw_group(rnn_resnet *r, int launch, double *flops) {
    if (!r || !flops) return RNN_E_NULL;
    *flops = 0;
    if (!r->arena) return rnn_fail(r->ctx, RNN_E_INVALID, "dbg_resnet_dw_group: no plan yet");
    for (auto &G : r->dwgs) {
        if (!G.L.njobs) continue;
        for (auto &m : G.m)
            *flops += 2.0 * m.sp.cout * m.sp.cin * m.sp.k * m.sp.k * m.sp.oh * m.sp.ow * (double)r->n;
    }
    if (!launch) return RNN_OK;
    rnn_ctx *ctx = r->ctx;
    std::lock_guard<std::recursive_mutex> lk(ctx->mu);
    for (auto &G : r->dwgs) TRY(rnn_conv_dw_group_launch(ctx, &G.L));
    return RNN_OK;
}

uint64_t rnn_resnet_flops(const rnn_resnet *r, size_t h, size_t w) {
    // ResNet::flops (model.rs:179-198): forward FLOP per image.
    if (!r) return 0;
    uint64_t f = 2ull * 3 * 9 * r->stem.cout * h * w;
    size_t hh = h, ww = w, c = r->stem.cout;
    for (auto &b : r->blocks) {
        const size_t oh = hh / b.c1.stride, ow = ww / b.c1.stride;
        f += 2ull * b.c1.cin * 9 * b.c1.cout * oh * ow;
        f += 2ull * b.c2.cin * 9 * b.c2.cout * oh * ow;
        if (b.down) f += 2ull * b.cd.cin * b.cd.cout * oh * ow;
        hh = oh;
        ww = ow;
        c = b.c2.cout;
    }
    return f + 2ull * c * r->nclass;
}

}  // extern "C"
