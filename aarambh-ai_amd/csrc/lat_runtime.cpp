// Host runtime of the latent-attention MoE decoder (benchmark config 5): context,
// device weights, the fp16 latent cache, the verify forward over the gfx950
// kernels of lat.hip and the aarh_lat_* C ABI of include/aarambh_hip.h.
//
// Block (nn/src/mla.rs:402-489 + nn/src/moe.rs:212-406), per layer:
//   1. fused [q_proj | kv_a_proj | k_rope_proj] GEMV on norm1(x)      -> raw rows
//   2. q prep (RoPE on q_rope, q_lat = up_k^T q_nope), kv prep (RMSNorm of the
//      latent, RoPE of k_rope, append to the cache)
//   3. latent attention (chunked, MFMA) and up_v per head               -> o_proj input
//   4. o_proj GEMV with the residual add; its epilogue writes norm2's fragments
//   5. router GEMV (also writes the normalised FFN input rows)          -> logits
//   6. top-k routing -> per-expert row lists; grouped expert gate/up (SwiGLU)
//      and down over only the routed rows; combine in expert order + shared
//      experts, residual add, fragments for the next consumer.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/aarambh_hip.h"
#include "kernels.hpp"

using namespace aarh;

namespace {

struct LTensor {  // tiled quantised (or row-major f32) weight matrix
    int fmt = WF_F32;
    int N = 0, K = 0;
    uint8_t* w = nullptr;
    uint32_t* sz = nullptr;
    float* rscale = nullptr;
};

struct LatLayer {
    float *norm1 = nullptr, *norm2 = nullptr, *kvn = nullptr;
    LTensor qkr, op, router, gu, dn;
    // stored values of up_k / up_v as fp16 hi + lo pairs: up_k^T [nh][lat][nope], up_v [nh][vd][lat]
    _Float16 *upk_hi = nullptr, *upk_lo = nullptr, *upv_hi = nullptr, *upv_lo = nullptr;
};

enum LPart { L_EMBED, L_NORM, L_QP, L_KVA, L_KRP, L_UPK, L_UPV, L_OP, L_ROUTER, L_GATE, L_UP, L_DOWN, L_LMHEAD };

struct LSlot {
    std::string name;
    int64_t rows = 0, cols = 0;
    int kind = AARH_T_NORM;
    LPart part = L_NORM;
    int layer = -1, expert = -1;
    float** norm_ptr = nullptr;
};

struct LProf {
    int cls;
    hipEvent_t a, b;
    double bytes;
    int moe_layer, moe_phase;  // expert phases: bytes from the routed counts at collection
};

constexpr int PAD_SLACK = 32;  // cache positions past max_seq_len for padding rows

}  // namespace

struct aarh_lat_ctx {
    aarh_lat_config cfg{};
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    int H = 0, V = 0, L = 0, nh = 0, nope = 0, rd = 0, lat = 0, vd = 0;
    int QW = 0, RAW = 0, OD = 0, E = 0, E16 = 0, NS = 0, D = 0, K = 0, KDc = 0;

    void* embed = nullptr;
    int embed_fmt = WF_F32;
    LTensor lm;
    std::vector<LatLayer> layers;
    float* final_norm = nullptr;
    std::vector<LSlot> slots;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    float* staging = nullptr;
    size_t staging_elems = 0;
    LTensor tmpq;          // quantisation target of up_k / up_v before their MFMA operand copies
    float* tmpf = nullptr;  // their stored values as f32 rows

    int cap = 0;
    std::vector<_Float16*> kc, vt;
    std::vector<int> kv_len;

    int Mmax = 0, A = 0;
    float *x = nullptr, *raw = nullptr, *q = nullptr, *att = nullptr, *xn = nullptr, *rl = nullptr;
    float *olat = nullptr, *hbuf = nullptr, *ybuf = nullptr, *ssq = nullptr, *hidden = nullptr, *logits = nullptr, *gap = nullptr;
    uint16_t *frag_a = nullptr, *frag_b = nullptr;
    float* apart = nullptr;
    size_t apart_elems = 0;
    float* gpart = nullptr;
    size_t gpart_elems = 0;
    unsigned* gcnt = nullptr;
    int *cnt = nullptr, *off = nullptr, *arow = nullptr, *rowmap = nullptr;  // cnt/off per layer
    int *chunk_e = nullptr, *chunk_r0 = nullptr, *nchunk = nullptr;
    unsigned long long* selm = nullptr;
    float* wsel = nullptr;
    int cus = 256;
    float* aw = nullptr;
    int32_t *d_pos0 = nullptr, *d_slot = nullptr;
    uint32_t* d_ids = nullptr;
    int32_t *h_pos0 = nullptr, *h_slot = nullptr;
    uint32_t* h_ids = nullptr;
    int last_M = 0;

    bool prof = false;
    std::vector<LProf> prof_recs;
    std::vector<hipEvent_t> ev_pool;
    double prof_ms[AARH_PROF_COUNT] = {0};
    double prof_bytes[AARH_PROF_COUNT] = {0};
    int64_t prof_n[AARH_PROF_COUNT] = {0};
};

namespace {

typedef aarh_lat_ctx Ctx;

int fail(Ctx* c, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (c) c->err = buf;
    return code;
}

#define HIPCHK(c, call)                                                                                  \
    do {                                                                                                 \
        hipError_t e_ = (call);                                                                          \
        if (e_ != hipSuccess) return fail((c), AARH_ERR_DEVICE, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

#define KCHK(c, call)                                                                                               \
    do {                                                                                                            \
        int r_ = (call);                                                                                            \
        if (r_ != 0) return fail((c), r_, "kernel launch failed: %s (code %d: %s)", #call, r_, last_launch_error()); \
    } while (0)

template <class T>
int dalloc(Ctx* c, T** p, size_t bytes) {
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc((void**)p, bytes);
    if (e != hipSuccess) return fail(c, AARH_ERR_DEVICE, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return 0;
}

size_t weight_bytes(int fmt, int64_t N, int64_t K) {
    switch (fmt) {
        case WF_INT4: return (size_t)(N * K / 2);
        case WF_INT8: return (size_t)(N * K);
        case WF_BF16: return (size_t)(N * K * 2);
        default: return (size_t)(N * K * 4);
    }
}

// Bytes a pass over rows [0, N) x K of a tensor of this format must read (weights + scales).
double alg_bytes(int fmt, double N, double K) {
    const double per = fmt == WF_INT4 ? 0.5 : fmt == WF_INT8 ? 1.0 : fmt == WF_BF16 ? 2.0 : 4.0;
    double b = N * K * per;
    if (fmt == WF_INT4) b += N * (K / 128) * 4.0;
    if (fmt == WF_INT8) b += N * 4.0;
    return b;
}

int alloc_tensor(Ctx* c, LTensor& t, int fmt, int N, int K) {
    t.fmt = fmt;
    t.N = N;
    t.K = K;
    // projection kernels address weights through one buffer resource with 32-bit byte offsets
    if (weight_bytes(fmt, N, K) >= ((size_t)1 << 31))
        return fail(c, AARH_ERR_UNSUPPORTED, "a %d x %d weight matrix of %zu bytes exceeds the 2 GiB per-tensor limit", N,
                    K, weight_bytes(fmt, N, K));
    if (dalloc(c, &t.w, weight_bytes(fmt, N, K))) return AARH_ERR_DEVICE;
    HIPCHK(c, hipMemset(t.w, 0, weight_bytes(fmt, N, K)));
    if (fmt == WF_INT4) {
        const size_t n = (size_t)N / 16 * (K / 128) * 16;
        if (dalloc(c, &t.sz, n * 4)) return AARH_ERR_DEVICE;
        std::vector<uint32_t> ones(n, 0x3C00u);  // scale 1.0, zero 0 until loaded
        HIPCHK(c, hipMemcpy(t.sz, ones.data(), n * 4, hipMemcpyHostToDevice));
    }
    if (fmt == WF_INT8) {
        if (dalloc(c, &t.rscale, (size_t)N * 4)) return AARH_ERR_DEVICE;
        std::vector<float> ones(N, 1.0f);
        HIPCHK(c, hipMemcpy(t.rscale, ones.data(), (size_t)N * 4, hipMemcpyHostToDevice));
    }
    return 0;
}

void free_tensor(LTensor& t) {
    if (t.w) (void)hipFree(t.w);
    if (t.sz) (void)hipFree(t.sz);
    if (t.rscale) (void)hipFree(t.rscale);
    t = LTensor{};
}

hipEvent_t take_event(Ctx* c) {
    if (!c->ev_pool.empty()) {
        hipEvent_t e = c->ev_pool.back();
        c->ev_pool.pop_back();
        return e;
    }
    hipEvent_t e;
    (void)hipEventCreate(&e);
    return e;
}

struct ProfScope {
    Ctx* c;
    int cls;
    double bytes;
    int moe_layer, moe_phase;
    hipEvent_t a = nullptr;
    ProfScope(Ctx* c_, int cls_, double bytes_, int ml = -1, int mph = 0)
        : c(c_), cls(cls_), bytes(bytes_), moe_layer(ml), moe_phase(mph) {
        if (c->prof) {
            a = take_event(c);
            (void)hipEventRecord(a, c->stream);
        }
    }
    ~ProfScope() {
        if (c->prof) {
            hipEvent_t b = take_event(c);
            (void)hipEventRecord(b, c->stream);
            c->prof_recs.push_back({cls, a, b, bytes, moe_layer, moe_phase});
        }
    }
};

int frag_mp(int M) { return M <= 4 ? 4 : (M <= 8 ? 8 : 16); }

RowMap rm(int S, long long seq_stride, long long row_stride) {
    RowMap r;
    r.S = S;
    r.seq_stride = seq_stride;
    r.row_stride = row_stride;
    return r;
}

XFrag xfrag(Ctx* c, uint16_t* buf, int fmt, int k, int mp, const float* norm_w, bool ssq) {
    XFrag f{};
    if (fmt == WF_F32) return f;
    f.buf = buf;
    f.fmt = fmt;
    f.mp = mp;
    f.G = k / 128;
    f.norm_w = norm_w;
    f.ssq = ssq ? c->ssq : nullptr;
    f.ssq_ld = c->H / 16;
    return f;
}

// y = x . W^T over M rows (fused RMSNorm input, epilogue), as the dense decoder's
// projections: the GEMV in 16-row launches, the many-row GEMM above 16 rows.
int gemv(Ctx* c, const LTensor& t, int M, const float* x, int ldx, const uint16_t* xf, int mp, const float* norm_w,
         float* hidden_out, int epi, float* out, int ldo, float* resid, const XFrag& fo, int cls) {
    GemvArgs a{};
    a.fmt = t.fmt;
    a.w = t.w;
    a.sz = t.sz;
    a.rscale = t.rscale;
    a.N = t.N;
    a.K = t.K;
    a.x = x;
    a.xmap = rm(M, 0, ldx);
    a.xf = xf;
    a.mp = mp;
    a.norm_w = norm_w;
    a.ssq_in = c->ssq;
    a.ssq_ld = c->H / 16;
    a.eps = c->cfg.norm_eps;
    a.hidden_out = hidden_out;
    a.epi = epi;
    a.out = out;
    a.omap = rm(M, 0, ldo);
    a.resid = resid;
    a.ldr = t.N;
    a.fo = fo;
    a.gpart = c->gpart;
    a.gcnt = c->gcnt;
    a.gpart_elems = (long long)c->gpart_elems;
    const double wb = alg_bytes(t.fmt, t.N, t.K);
    if (t.fmt != WF_F32 && M > 16) {
        ProfScope ps(c, cls, wb);
        a.m_base = 0;
        a.M = M;
        int r = launch_gemm(a, c->stream);
        if (r)
            return fail(c, r, "gemm launch failed (fmt %d N %d K %d M %d): code %d %s", t.fmt, t.N, t.K, M, r,
                        last_launch_error());
        return 0;
    }
    ProfScope ps(c, cls, wb * ((M + 15) / 16));
    for (int m0 = 0; m0 < M; m0 += 16) {
        a.m_base = m0;
        a.M = std::min(16, M - m0);
        int r = launch_gemv(a, c->stream);
        if (r)
            return fail(c, r, "gemv launch failed (fmt %d N %d K %d M %d): code %d %s", t.fmt, t.N, t.K, a.M, r,
                        last_launch_error());
    }
    return 0;
}

int ensure_apart(Ctx* c, size_t elems) {
    if (elems <= c->apart_elems) return 0;
    if (c->apart) {
        HIPCHK(c, hipStreamSynchronize(c->stream));
        (void)hipFree(c->apart);
        c->apart = nullptr;
        c->apart_elems = 0;
    }
    if (dalloc(c, &c->apart, elems * 4)) return AARH_ERR_DEVICE;
    c->apart_elems = elems;
    return 0;
}

// One latent block over M = nseq * S rows; x arrives with norm1 fragments in frag_a
// (and its sums of squares); `after` is the consumer of the block's output.
int run_block(Ctx* c, int l, int nseq, int S, int max_kv, const XFrag& after) {
    const LatLayer& w = c->layers[l];
    const int M = nseq * S, H = c->H, mp = frag_mp(M);
    int r;
    if ((r = gemv(c, w.qkr, M, c->x, H, c->frag_a, mp, w.norm1, nullptr, EPI_STORE, c->raw, c->RAW, nullptr,
                  XFrag{}, AARH_PROF_GEMV_QKV)))
        return r;
    MlaArgs m{};
    m.nseq = nseq;
    m.S = S;
    m.nh = c->nh;
    m.nope = c->nope;
    m.rd = c->rd;
    m.lat = c->lat;
    m.vd = c->vd;
    m.pos0 = c->d_pos0;
    m.slot = c->d_slot;
    m.raw = c->raw;
    m.raw_ld = c->RAW;
    m.rope_cos = c->rope_cos;
    m.rope_sin = c->rope_sin;
    m.upk_hi = w.upk_hi;
    m.upk_lo = w.upk_lo;
    m.upv_hi = w.upv_hi;
    m.upv_lo = w.upv_lo;
    m.kvn_w = w.kvn;
    m.eps = c->cfg.norm_eps;
    m.q = c->q;
    m.kc = c->kc[l];
    m.vt = c->vt[l];
    m.cap = c->cap;
    m.scale = (float)(1.0 / std::sqrt((double)(c->nope + c->rd)));
    const int rows = S * c->nh;
    m.ntiles = (rows + 15) / 16;
    m.tiles_per_wg = std::min(m.ntiles, mla_tiles_per_wg_max());
    const int ntg = (m.ntiles + m.tiles_per_wg - 1) / m.tiles_per_wg;
    const int base = nseq * ntg;
    const int max_chunks = std::max(1, (max_kv + 31) / 32);
    // about one workgroup per CU (each holds a CU's LDS), at most 64 chunks for the merge
    int nch = std::max(1, std::min(std::min(max_chunks, 64), (c->cus + base - 1) / base));
    const int chunk = ((max_kv + nch - 1) / nch + 31) / 32 * 32;
    nch = (max_kv + chunk - 1) / chunk;
    m.chunk = chunk;
    m.nchunks = nch;
    if ((r = ensure_apart(c, (size_t)nseq * m.ntiles * nch * 16 * (c->lat + 4)))) return r;
    m.part = c->apart;
    m.olat = c->olat;
    m.fo = xfrag(c, c->frag_b, w.op.fmt, c->OD, mp, nullptr, false);
    m.out = w.op.fmt == WF_F32 ? c->att : nullptr;
    {
        // cache bytes read (c_kv + k_rope rows, transposed c_kv) and up_k / up_v reads
        const double kvb = (double)max_kv * nseq * (2.0 * (c->lat + c->rd) + 2.0 * c->lat);
        const double ub = 4.0 * (double)c->nh * c->lat * (c->nope + c->vd);  // fp16 hi + lo pairs
        ProfScope ps(c, AARH_PROF_ATTENTION, kvb + ub);
        KCHK(c, launch_mla_qprep(m, c->stream));
        KCHK(c, launch_mla_kvprep(m, c->stream));
        KCHK(c, launch_mla_attn(m, c->stream));
        KCHK(c, launch_mla_out(m, c->stream));
    }
    if ((r = gemv(c, w.op, M, c->att, c->OD, c->frag_b, mp, nullptr, nullptr, EPI_RESID, nullptr, 0, c->x,
                  xfrag(c, c->frag_a, w.router.fmt, H, mp, w.norm2, true), AARH_PROF_GEMV_WO)))
        return r;
    if ((r = gemv(c, w.router, M, c->x, H, c->frag_a, mp, w.norm2, c->xn, EPI_STORE, c->rl, c->E16, nullptr, XFrag{},
                  AARH_PROF_GEMV_GATEUP)))
        return r;
    MoeArgs e{};
    e.M = M;
    e.E = c->E;
    e.K = c->K;
    e.NS = c->NS;
    e.H = H;
    e.D = c->D;
    e.logits = c->rl;
    e.lld = c->E16;
    e.cnt = c->cnt + (size_t)l * (c->E + c->NS);
    e.off = c->off + (size_t)l * (c->E + c->NS + 1);
    e.arow = c->arow;
    e.aw = c->aw;
    e.rowmap = c->rowmap;
    e.fmt = w.gu.fmt;
    e.gu = w.gu.w;
    e.gu_sz = w.gu.sz;
    e.gu_rs = w.gu.rscale;
    e.dn = w.dn.w;
    e.dn_sz = w.dn.sz;
    e.dn_rs = w.dn.rscale;
    e.xn = c->xn;
    e.h = c->hbuf;
    e.y = c->ybuf;
    e.x = c->x;
    e.fo = after;
    e.gap = c->gap;
    e.selm = c->selm;
    e.wsel = c->wsel;
    e.chunk_e = c->chunk_e;
    e.chunk_r0 = c->chunk_r0;
    e.nchunk = c->nchunk;
    // chunk capacity and an estimate of the chunks present (experts hit + shared + overflow)
    const int mc = (M + 15) / 16;
    e.cmax = M * c->K / 16 + c->E + c->NS * mc;
    const int cexp = std::min(c->E, M * c->K) + c->NS * mc + M * c->K / 16;
    // slices per chunk: about one workgroup per CU over the chunks present.  Each
    // workgroup gathers its chunk's rows before it streams, so longer streams per
    // workgroup beat more workgroups (measured: 2 and 3 workgroups per CU were 6-15 %
    // slower at 5 and 160 rows)
    auto slices = [&](int ntiles) {
        const int nsteps = (ntiles + moe_tiles_per_step(w.gu.fmt) - 1) / moe_tiles_per_step(w.gu.fmt);
        return std::max(1, std::min(nsteps, (c->cus + cexp - 1) / cexp));
    };
    {
        ProfScope ps(c, AARH_PROF_GEMV_GATEUP, 0, l, 1);
        KCHK(c, launch_moe_route(e, c->stream));
        e.bpe = slices(2 * c->D / 16);
        KCHK(c, launch_moe_ffn(e, 1, c->stream));
    }
    {
        ProfScope ps(c, AARH_PROF_GEMV_DOWN, 0, l, 2);
        e.bpe = slices(H / 16);
        KCHK(c, launch_moe_ffn(e, 2, c->stream));
        KCHK(c, launch_moe_combine(e, c->stream));
    }
    return 0;
}

int forward_dev(Ctx* c, int nseq, int S, int max_kv) {
    const int M = nseq * S, H = c->H, mp = frag_mp(M);
    {
        ProfScope ps(c, AARH_PROF_OTHER, 0);
        KCHK(c, launch_fill_f32(c->gap, M, INFINITY, c->stream));
        const LatLayer& l0 = c->layers[0];
        KCHK(c, launch_embed(c->embed, c->embed_fmt, H, c->d_ids, M, c->x,
                             xfrag(c, c->frag_a, l0.qkr.fmt, H, mp, l0.norm1, true), c->stream));
    }
    for (int l = 0; l < c->L; l++) {
        const XFrag after = l + 1 < c->L ? xfrag(c, c->frag_a, c->layers[l + 1].qkr.fmt, H, mp, c->layers[l + 1].norm1, true)
                                         : xfrag(c, c->frag_a, c->lm.fmt, H, mp, c->final_norm, true);
        int r = run_block(c, l, nseq, S, max_kv, after);
        if (r) return r;
    }
    return gemv(c, c->lm, M, c->x, H, c->frag_a, mp, c->final_norm, c->hidden, EPI_STORE, c->logits, c->V, nullptr,
                XFrag{}, AARH_PROF_GEMV_LMHEAD);
}

int sync_stream(Ctx* c) {
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return 0;
}

void build_slots(Ctx* c) {
    const int64_t H = c->H;
    auto add = [&](const std::string& n, int64_t r, int64_t cc, int kind, LPart p, int layer, int expert,
                   float** np) {
        LSlot s;
        s.name = n;
        s.rows = r;
        s.cols = cc;
        s.kind = kind;
        s.part = p;
        s.layer = layer;
        s.expert = expert;
        s.norm_ptr = np;
        c->slots.push_back(s);
    };
    add("embedding.weight", c->V, H, AARH_T_EMBED, L_EMBED, -1, -1, nullptr);
    for (int l = 0; l < c->L; l++) {
        LatLayer* b = &c->layers[l];
        const std::string p = "blocks." + std::to_string(l) + ".";
        add(p + "norm1.weight", 1, H, AARH_T_NORM, L_NORM, l, -1, &b->norm1);
        add(p + "mla.q_proj.weight", c->QW, H, AARH_T_LINEAR, L_QP, l, -1, nullptr);
        add(p + "mla.kv_a_proj.weight", c->lat, H, AARH_T_LINEAR, L_KVA, l, -1, nullptr);
        add(p + "mla.kv_a_norm.weight", 1, c->lat, AARH_T_NORM, L_NORM, l, -1, &b->kvn);
        add(p + "mla.up_k.weight", (int64_t)c->nh * c->nope, c->lat, AARH_T_LINEAR, L_UPK, l, -1, nullptr);
        add(p + "mla.up_v.weight", (int64_t)c->nh * c->vd, c->lat, AARH_T_LINEAR, L_UPV, l, -1, nullptr);
        add(p + "mla.k_rope_proj.weight", c->rd, H, AARH_T_LINEAR, L_KRP, l, -1, nullptr);
        add(p + "mla.o_proj.weight", H, c->OD, AARH_T_LINEAR, L_OP, l, -1, nullptr);
        add(p + "norm2.weight", 1, H, AARH_T_NORM, L_NORM, l, -1, &b->norm2);
        add(p + "ffn.router.weight", c->E, H, AARH_T_LINEAR, L_ROUTER, l, -1, nullptr);
        for (int e = 0; e < c->E + c->NS; e++) {
            const std::string g = e < c->E ? p + "ffn.experts." + std::to_string(e) + "."
                                           : p + "ffn.shared_experts." + std::to_string(e - c->E) + ".";
            add(g + "w_gate.weight", c->D, H, AARH_T_LINEAR, L_GATE, l, e, nullptr);
            add(g + "w_up.weight", c->D, H, AARH_T_LINEAR, L_UP, l, e, nullptr);
            add(g + "w_down.weight", H, c->D, AARH_T_LINEAR, L_DOWN, l, e, nullptr);
        }
    }
    add("final_norm.weight", 1, H, AARH_T_NORM, L_NORM, -1, -1, &c->final_norm);
    // LmHead::untied_with_qat (model.rs:239-248): its own [vocab, hidden] weight after final_norm
    if (c->cfg.untied_lm_head) add("lm_head.weight", c->V, H, AARH_T_EMBED, L_LMHEAD, -1, -1, nullptr);
}

int ensure_staging(Ctx* c, size_t elems) {
    if (elems <= c->staging_elems) return 0;
    if (c->staging) {
        HIPCHK(c, hipStreamSynchronize(c->stream));
        (void)hipFree(c->staging);
        c->staging = nullptr;
        c->staging_elems = 0;
    }
    if (dalloc(c, &c->staging, elems * 4)) return AARH_ERR_DEVICE;
    c->staging_elems = elems;
    return 0;
}

// The tiled matrix (and its row offset and gate/up interleave) holding a linear tensor.
void linear_target(Ctx* c, const LSlot& s, LTensor** t, int* ro, int* inter) {
    LatLayer& b = c->layers[s.layer];
    *ro = 0;
    *inter = 0;
    switch (s.part) {
        case L_QP: *t = &b.qkr; break;
        case L_KVA: *t = &b.qkr; *ro = c->QW; break;
        case L_KRP: *t = &b.qkr; *ro = c->QW + c->lat; break;
        case L_OP: *t = &b.op; break;
        case L_ROUTER: *t = &b.router; break;
        case L_GATE: *t = &b.gu; *ro = s.expert * 2 * c->D; *inter = 1; break;
        case L_UP: *t = &b.gu; *ro = s.expert * 2 * c->D; *inter = 2; break;
        default: *t = &b.dn; *ro = s.expert * c->H; break;
    }
}

// up_k / up_v held in tmpq (the attention format's stored values) -> fp16 hi + lo operands.
int split_upkv(Ctx* c, const LSlot& s) {
    LatLayer& b = c->layers[s.layer];
    LTensor& t = c->tmpq;
    KCHK(c, launch_dequant_tiled(t.w, t.sz, t.rscale, t.fmt, (int)s.rows, (int)s.cols, c->tmpf, 0, c->stream));
    if (s.part == L_UPK)
        KCHK(c, launch_split_hilo(c->tmpf, b.upk_hi, b.upk_lo, (int)s.rows, (int)s.cols, c->nope, c->stream));
    else
        KCHK(c, launch_split_hilo(c->tmpf, b.upv_hi, b.upv_lo, (int)s.rows, (int)s.cols, 0, c->stream));
    return 0;
}

// Place the tensor held in c->staging (f32, reference shape) into its device form.
int place_staging(Ctx* c, int id) {
    const LSlot& s = c->slots[id];
    const int64_t n = s.rows * s.cols;
    if (s.part == L_EMBED) {
        if (c->embed_fmt == WF_F32) {
            HIPCHK(c, hipMemcpyAsync(c->embed, c->staging, n * 4, hipMemcpyDeviceToDevice, c->stream));
        } else {
            KCHK(c, launch_to_bf16(c->staging, (uint16_t*)c->embed, n, c->stream));
            if (!c->cfg.untied_lm_head)
                KCHK(c, launch_quantise_tiled(c->staging, c->V, c->H, WF_BF16, c->lm.w, nullptr, nullptr, 0, c->V, 0,
                                              c->stream));
        }
        return 0;
    }
    if (s.part == L_LMHEAD) {
        if (c->embed_fmt == WF_F32) {
            HIPCHK(c, hipMemcpyAsync(c->lm.w, c->staging, n * 4, hipMemcpyDeviceToDevice, c->stream));
        } else {
            KCHK(c, launch_quantise_tiled(c->staging, c->V, c->H, WF_BF16, c->lm.w, nullptr, nullptr, 0, c->V, 0,
                                          c->stream));
        }
        return 0;
    }
    if (s.part == L_NORM) {
        HIPCHK(c, hipMemcpyAsync(*s.norm_ptr, c->staging, n * 4, hipMemcpyDeviceToDevice, c->stream));
        return 0;
    }
    if (s.part == L_UPK || s.part == L_UPV) {
        // exactly the values the attention format stores, split into fp16 hi + lo MFMA operands
        LTensor& t = c->tmpq;
        KCHK(c, launch_quantise_tiled(c->staging, (int)s.rows, (int)s.cols, t.fmt, t.w, t.sz, t.rscale, 0, (int)s.rows,
                                      0, c->stream));
        return split_upkv(c, s);
    }
    LTensor* t = nullptr;
    int ro = 0, inter = 0;
    linear_target(c, s, &t, &ro, &inter);
    KCHK(c, launch_quantise_tiled(c->staging, (int)s.rows, (int)s.cols, t->fmt, t->w, t->sz, t->rscale, ro, t->N,
                                  inter, c->stream));
    return 0;
}

int stage_rows(Ctx* c, const uint32_t* ids, const int32_t* slots, const int32_t* offsets, int nseq, int S,
               int* max_kv) {
    if (nseq <= 0 || S <= 0) return fail(c, AARH_ERR_SHAPE, "batch and sequence length must be non-zero");
    if (nseq * S > c->Mmax) return fail(c, AARH_ERR_SHAPE, "nseq*S=%d exceeds max_rows %d", nseq * S, c->Mmax);
    int mk = 0;
    for (int b = 0; b < nseq; b++) {
        const int sl = slots[b], off = offsets[b];
        if (sl < 0 || sl >= c->cfg.max_batch) return fail(c, AARH_ERR_SHAPE, "bad slot %d", sl);
        for (int b2 = 0; b2 < b; b2++)
            if (slots[b2] == sl) return fail(c, AARH_ERR_SHAPE, "slot %d used twice", sl);
        if (off < 0 || off > c->kv_len[sl])
            return fail(c, AARH_ERR_SHAPE, "offset %d beyond cached length %d of slot %d", off, c->kv_len[sl], sl);
        if (off + S > c->cfg.max_seq_len)
            return fail(c, AARH_ERR_SHAPE, "sequence length %d with offset %d exceeds max_seq_len %d", S, off,
                        c->cfg.max_seq_len);
        mk = std::max(mk, off + S);
    }
    for (int i = 0; i < nseq * S; i++)
        if ((int64_t)ids[i] >= c->V) return fail(c, AARH_ERR_SHAPE, "token id %u exceeds vocabulary", ids[i]);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    memcpy(c->h_pos0, offsets, nseq * 4);
    memcpy(c->h_slot, slots, nseq * 4);
    memcpy(c->h_ids, ids, (size_t)nseq * S * 4);
    HIPCHK(c, hipMemcpyAsync(c->d_pos0, c->h_pos0, nseq * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_slot, c->h_slot, nseq * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_ids, c->h_ids, (size_t)nseq * S * 4, hipMemcpyHostToDevice, c->stream));
    *max_kv = mk;
    return 0;
}

int prof_collect(Ctx* c) {
    if (c->prof_recs.empty()) return 0;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    std::vector<int32_t> counts;
    const int EN = c->E + c->NS;
    for (auto& r : c->prof_recs) {
        float ms = 0;
        (void)hipEventElapsedTime(&ms, r.a, r.b);
        double bytes = r.bytes;
        if (r.moe_layer >= 0) {
            // weights of the experts the layer routed rows to (each read once)
            if (counts.empty()) {
                counts.resize((size_t)c->L * EN);
                HIPCHK(c, hipMemcpy(counts.data(), c->cnt, counts.size() * 4, hipMemcpyDeviceToHost));
            }
            int used = 0;
            for (int e = 0; e < EN; e++) used += counts[(size_t)r.moe_layer * EN + e] > 0;
            const int fmt = c->layers[r.moe_layer].gu.fmt;
            bytes = r.moe_phase == 1 ? used * alg_bytes(fmt, 2.0 * c->D, c->H) : used * alg_bytes(fmt, c->H, c->D);
        }
        c->prof_ms[r.cls] += ms;
        c->prof_bytes[r.cls] += bytes;
        c->prof_n[r.cls] += 1;
        c->ev_pool.push_back(r.a);
        c->ev_pool.push_back(r.b);
    }
    c->prof_recs.clear();
    return 0;
}

}  // namespace

namespace aarh {
// Records a failure on a latent context for the checkpoint readers (weights.cpp).
int lat_ctx_fail(aarh_lat_ctx* c, int code, const char* msg) { return fail(c, code, "%s", msg); }
}  // namespace aarh

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* aarh_lat_last_error(const aarh_lat_ctx* c) { return c ? c->err.c_str() : "null context"; }

void aarh_lat_destroy(aarh_lat_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    auto F = [](void* p) {
        if (p) (void)hipFree(p);
    };
    F(c->embed);
    if (c->lm.w != c->embed) free_tensor(c->lm);
    for (auto& b : c->layers) {
        F(b.norm1);
        F(b.norm2);
        F(b.kvn);
        F(b.upk_hi);
        F(b.upk_lo);
        F(b.upv_hi);
        F(b.upv_lo);
        free_tensor(b.qkr);
        free_tensor(b.op);
        free_tensor(b.router);
        free_tensor(b.gu);
        free_tensor(b.dn);
    }
    free_tensor(c->tmpq);
    F(c->tmpf);
    F(c->final_norm);
    F(c->rope_cos);
    F(c->rope_sin);
    F(c->staging);
    for (size_t i = 0; i < c->kc.size(); i++) {
        F(c->kc[i]);
        F(c->vt[i]);
    }
    for (void* p : {(void*)c->x, (void*)c->raw, (void*)c->q, (void*)c->att, (void*)c->xn, (void*)c->rl,
                    (void*)c->olat, (void*)c->hbuf, (void*)c->ybuf, (void*)c->ssq, (void*)c->hidden, (void*)c->logits, (void*)c->gap,
                    (void*)c->frag_a, (void*)c->frag_b, (void*)c->apart, (void*)c->gpart, (void*)c->gcnt,
                    (void*)c->cnt, (void*)c->off, (void*)c->arow, (void*)c->rowmap, (void*)c->aw, (void*)c->chunk_e,
                    (void*)c->chunk_r0, (void*)c->nchunk, (void*)c->selm, (void*)c->wsel, (void*)c->d_pos0,
                    (void*)c->d_slot, (void*)c->d_ids})
        F(p);
    if (c->h_pos0) (void)hipHostFree(c->h_pos0);
    if (c->h_slot) (void)hipHostFree(c->h_slot);
    if (c->h_ids) (void)hipHostFree(c->h_ids);
    for (auto& r : c->prof_recs) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    for (auto e : c->ev_pool) (void)hipEventDestroy(e);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

int aarh_lat_create(int device, const aarh_lat_config* cfg, aarh_lat_ctx** out) {
    if (!cfg || !out) return AARH_ERR_CONFIG;
    *out = nullptr;
    Ctx* c = new Ctx();
    c->cfg = *cfg;
    c->device = device;
    const auto& g = *cfg;
    *out = c;
    if (g.vocab_size <= 0 || g.hidden_dim <= 0 || g.n_layers <= 0 || g.n_heads <= 0 || g.max_seq_len <= 0 ||
        g.latent_dim <= 0 || g.rope_dim <= 0 || g.nope_dim <= 0 || g.v_dim <= 0 || g.n_experts < 2 || g.top_k < 1 ||
        g.top_k > g.n_experts || g.expert_dim <= 0 || g.n_shared < 0 || g.max_batch <= 0 || g.max_rows <= 0)
        return fail(c, AARH_ERR_CONFIG, "model dimensions must be positive (n_experts >= 2, 1 <= top_k <= n_experts)");
    c->H = g.hidden_dim;
    c->V = g.vocab_size;
    c->L = g.n_layers;
    c->nh = g.n_heads;
    c->nope = g.nope_dim;
    c->rd = g.rope_dim;
    c->lat = g.latent_dim;
    c->vd = g.v_dim;
    c->QW = c->nh * (c->nope + c->rd);
    c->RAW = c->QW + c->lat + c->rd;
    c->OD = c->nh * c->vd;
    c->E = g.n_experts;
    c->E16 = (c->E + 15) / 16 * 16;  // router rows padded to whole 16-row tiles (zero weights)
    c->NS = g.n_shared;
    c->D = g.expert_dim;
    c->K = g.top_k;
    c->KDc = c->lat + c->rd;
    c->Mmax = g.max_rows;
    c->A = c->Mmax * (c->K + c->NS);
    if (!mla_supported(c->lat, c->rd, c->vd, c->nope))
        return fail(c, AARH_ERR_UNSUPPORTED, "latent/rope widths (%d, %d) unsupported: (512, 64) or (128, 32), nope %% 32 == 0, v_dim %% 16 == 0",
                    c->lat, c->rd);
    if (c->H % 128 || c->V % 128 || c->D % 128 || c->OD % 128 || c->RAW % 16 || (c->nh * c->nope) % 16 || c->OD % 16)
        return fail(c, AARH_ERR_UNSUPPORTED,
                    "hidden, vocab, expert and n_heads*v_dim widths must be multiples of 128 (q/kv rows of 16)");
    if (c->E > 64 || c->E + c->NS > 72)
        return fail(c, AARH_ERR_UNSUPPORTED, "at most 64 routed and 72 total experts");
    if (c->H / 128 > 16 || c->D / 128 > 16) return fail(c, AARH_ERR_UNSUPPORTED, "hidden / expert width above 2048");
    if (g.expert_format < AARH_W_BF16 || g.expert_format > AARH_W_INT4_G128 || g.attn_format < 0 ||
        g.attn_format > AARH_W_INT4_G128 || (g.lm_head_format != 0 && g.lm_head_format != 1) ||
        (g.untied_lm_head != 0 && g.untied_lm_head != 1))
        return fail(c, AARH_ERR_CONFIG, "unknown or unsupported weight format (experts: bf16, int8, int4)");
    if (g.kv_format != AARH_KV_F16) return fail(c, AARH_ERR_UNSUPPORTED, "the latent cache is fp16 (AARH_KV_F16)");
    if (g.max_rows > 256) return fail(c, AARH_ERR_UNSUPPORTED, "max_rows must be <= 256");
    c->cap = (g.max_seq_len + PAD_SLACK + 31) / 32 * 32;
    if (hipSetDevice(device) != hipSuccess) return fail(c, AARH_ERR_DEVICE, "hipSetDevice(%d) failed", device);
    HIPCHK(c, hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    if (hipDeviceGetAttribute(&c->cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || c->cus <= 0)
        c->cus = 256;
    c->layers.resize(c->L);
    build_slots(c);
    int r;
    c->embed_fmt = g.lm_head_format == 1 ? WF_BF16 : WF_F32;
    if (dalloc(c, (uint8_t**)&c->embed, weight_bytes(c->embed_fmt, c->V, c->H))) return AARH_ERR_DEVICE;
    HIPCHK(c, hipMemset(c->embed, 0, weight_bytes(c->embed_fmt, c->V, c->H)));
    if (c->embed_fmt == WF_F32) {
        c->lm.fmt = WF_F32;
        c->lm.N = c->V;
        c->lm.K = c->H;
        if (!g.untied_lm_head) {
            c->lm.w = (uint8_t*)c->embed;  // row-major f32 weights are shared
        } else {
            if (dalloc(c, &c->lm.w, weight_bytes(WF_F32, c->V, c->H))) return AARH_ERR_DEVICE;
            HIPCHK(c, hipMemset(c->lm.w, 0, weight_bytes(WF_F32, c->V, c->H)));
        }
    } else if ((r = alloc_tensor(c, c->lm, WF_BF16, c->V, c->H))) {
        return r;
    }
    const int af = g.attn_format, ef = g.expert_format;
    for (auto& b : c->layers) {
        if (dalloc(c, &b.norm1, c->H * 4) || dalloc(c, &b.norm2, c->H * 4) || dalloc(c, &b.kvn, c->lat * 4))
            return AARH_ERR_DEVICE;
        KCHK(c, launch_fill_f32(b.norm1, c->H, 1.0f, c->stream));
        KCHK(c, launch_fill_f32(b.norm2, c->H, 1.0f, c->stream));
        KCHK(c, launch_fill_f32(b.kvn, c->lat, 1.0f, c->stream));
        if ((r = alloc_tensor(c, b.qkr, af, c->RAW, c->H)) || (r = alloc_tensor(c, b.op, af, c->H, c->OD)) ||
            (r = alloc_tensor(c, b.router, af, c->E16, c->H)) ||
            (r = alloc_tensor(c, b.gu, ef, (c->E + c->NS) * 2 * c->D, c->H)) ||
            (r = alloc_tensor(c, b.dn, ef, (c->E + c->NS) * c->H, c->D)))
            return r;
        const size_t ub = (size_t)c->nh * c->nope * c->lat * 2, vb = (size_t)c->nh * c->vd * c->lat * 2;
        if (dalloc(c, &b.upk_hi, ub) || dalloc(c, &b.upk_lo, ub) || dalloc(c, &b.upv_hi, vb) ||
            dalloc(c, &b.upv_lo, vb))
            return AARH_ERR_DEVICE;
        HIPCHK(c, hipMemset(b.upk_hi, 0, ub));
        HIPCHK(c, hipMemset(b.upk_lo, 0, ub));
        HIPCHK(c, hipMemset(b.upv_hi, 0, vb));
        HIPCHK(c, hipMemset(b.upv_lo, 0, vb));
    }
    if ((r = alloc_tensor(c, c->tmpq, af, c->nh * std::max(c->nope, c->vd), c->lat))) return r;
    if (dalloc(c, &c->tmpf, (size_t)c->nh * std::max(c->nope, c->vd) * c->lat * 4)) return AARH_ERR_DEVICE;
    if (dalloc(c, &c->final_norm, c->H * 4)) return AARH_ERR_DEVICE;
    KCHK(c, launch_fill_f32(c->final_norm, c->H, 1.0f, c->stream));
    // MLA's own rope_dim-wide RoPE table (model.rs:1112-1118, rope_scaling.rs:6-11), host f32
    {
        const int half = c->rd / 2, npos = g.max_seq_len + PAD_SLACK;
        std::vector<float> cs((size_t)npos * half), sn((size_t)npos * half), inv(half);
        for (int i = 0; i < half; i++)
            inv[i] = (float)(1.0 / std::pow((double)g.rope_theta, 2.0 * (double)i / (double)c->rd));
        for (int p = 0; p < npos; p++)
            for (int i = 0; i < half; i++) {
                const float a = (float)p * inv[i];
                cs[(size_t)p * half + i] = cosf(a);
                sn[(size_t)p * half + i] = sinf(a);
            }
        if (dalloc(c, &c->rope_cos, cs.size() * 4) || dalloc(c, &c->rope_sin, sn.size() * 4)) return AARH_ERR_DEVICE;
        HIPCHK(c, hipMemcpy(c->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
        HIPCHK(c, hipMemcpy(c->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    }
    // latent cache: [slots][cap][lat + rd] rows and the transposed [slots][lat][cap] latent;
    // zero-filled so positions past a sequence's length hold finite values
    {
        const size_t kb = (size_t)g.max_batch * c->cap * c->KDc * 2, vb = (size_t)g.max_batch * c->lat * c->cap * 2;
        c->kc.assign(c->L, nullptr);
        c->vt.assign(c->L, nullptr);
        for (int l = 0; l < c->L; l++) {
            if (dalloc(c, &c->kc[l], kb) || dalloc(c, &c->vt[l], vb)) return AARH_ERR_DEVICE;
            HIPCHK(c, hipMemset(c->kc[l], 0, kb));
            HIPCHK(c, hipMemset(c->vt[l], 0, vb));
        }
        c->kv_len.assign(g.max_batch, 0);
    }
    {
        const size_t M = c->Mmax, H = c->H, A = c->A, EN = c->E + c->NS;
        if (dalloc(c, &c->x, M * H * 4) || dalloc(c, &c->raw, M * c->RAW * 4) ||
            dalloc(c, &c->q, M * c->nh * c->KDc * 4) || dalloc(c, &c->olat, M * c->nh * c->lat * 4) || dalloc(c, &c->att, M * c->OD * 4) ||
            dalloc(c, &c->xn, M * H * 4) || dalloc(c, &c->rl, M * c->E16 * 4) || dalloc(c, &c->hbuf, A * c->D * 4) ||
            dalloc(c, &c->ybuf, A * H * 4) || dalloc(c, &c->ssq, M * (H / 16) * 4) || dalloc(c, &c->hidden, M * H * 4) ||
            dalloc(c, &c->logits, M * c->V * 4) || dalloc(c, &c->gap, M * 4) ||
            dalloc(c, &c->cnt, c->L * EN * 4) || dalloc(c, &c->off, c->L * (EN + 1) * 4) ||
            dalloc(c, &c->arow, A * 4) || dalloc(c, &c->aw, A * 4) || dalloc(c, &c->rowmap, M * (c->K + c->NS) * 4))
            return AARH_ERR_DEVICE;
        const size_t cmax = M * c->K / 16 + c->E + c->NS * ((M + 15) / 16);
        if (dalloc(c, &c->chunk_e, cmax * 4) || dalloc(c, &c->chunk_r0, cmax * 4) || dalloc(c, &c->nchunk, 16) ||
            dalloc(c, &c->selm, M * 8) || dalloc(c, &c->wsel, M * 64 * 4))
            return AARH_ERR_DEVICE;
        HIPCHK(c, hipMemset(c->nchunk, 0, 16));
        HIPCHK(c, hipMemset(c->cnt, 0, c->L * EN * 4));
        const size_t gmax = (size_t)std::max(c->H, c->OD) / 128;
        const size_t halves = ((M + 15) / 16) * gmax * 16 * 32 * 8;
        if (dalloc(c, &c->frag_a, halves * 2) || dalloc(c, &c->frag_b, halves * 2)) return AARH_ERR_DEVICE;
        HIPCHK(c, hipMemset(c->frag_a, 0, halves * 2));
        HIPCHK(c, hipMemset(c->frag_b, 0, halves * 2));
        if (M > 16) {
            c->gpart_elems = (size_t)16 << 20;
            if (dalloc(c, &c->gpart, c->gpart_elems * 4) || dalloc(c, &c->gcnt, 8192 * 4)) return AARH_ERR_DEVICE;
            HIPCHK(c, hipMemset(c->gcnt, 0, 8192 * 4));
        }
        if (dalloc(c, &c->d_pos0, M * 4) || dalloc(c, &c->d_slot, M * 4) || dalloc(c, &c->d_ids, M * 4))
            return AARH_ERR_DEVICE;
        HIPCHK(c, hipHostMalloc((void**)&c->h_pos0, M * 4, 0));
        HIPCHK(c, hipHostMalloc((void**)&c->h_slot, M * 4, 0));
        HIPCHK(c, hipHostMalloc((void**)&c->h_ids, M * 4, 0));
    }
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return AARH_OK;
}

int aarh_lat_get_config(const aarh_lat_ctx* c, aarh_lat_config* out) {
    if (!c || !out) return AARH_ERR_CONFIG;
    *out = c->cfg;
    return AARH_OK;
}

int aarh_lat_num_tensors(const aarh_lat_ctx* c) { return c ? (int)c->slots.size() : 0; }

int aarh_lat_tensor_info(const aarh_lat_ctx* c, int id, char* name, int name_cap, int64_t* rows, int64_t* cols,
                         int32_t* kind) {
    if (!c || id < 0 || id >= (int)c->slots.size()) return AARH_ERR_SHAPE;
    const LSlot& s = c->slots[id];
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", s.name.c_str());
    if (rows) *rows = s.rows;
    if (cols) *cols = s.cols;
    if (kind) *kind = s.kind;
    return AARH_OK;
}

int aarh_lat_load_tensor_f32(aarh_lat_ctx* c, int id, const float* host, int64_t numel) {
    if (!c || id < 0 || id >= (int)c->slots.size()) return fail(c, AARH_ERR_SHAPE, "bad tensor id %d", id);
    const LSlot& s = c->slots[id];
    if (numel != s.rows * s.cols)
        return fail(c, AARH_ERR_SHAPE, "tensor %s expects %lld values, got %lld", s.name.c_str(),
                    (long long)(s.rows * s.cols), (long long)numel);
    if (ensure_staging(c, (size_t)numel)) return AARH_ERR_DEVICE;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(c->staging, host, numel * 4, hipMemcpyHostToDevice));
    int r = place_staging(c, id);
    if (r) return r;
    return sync_stream(c);
}

int aarh_lat_load_tensor_packed_i4(aarh_lat_ctx* c, int id, const int64_t* shape, int32_t ndims, int64_t group_size,
                                   const uint8_t* data, int64_t data_len, const float* scales, const float* zeros,
                                   int64_t n_groups) {
    if (!c || id < 0 || id >= (int)c->slots.size()) return fail(c, AARH_ERR_SHAPE, "bad tensor id %d", id);
    const LSlot& s = c->slots[id];
    if (s.kind != AARH_T_LINEAR)
        return fail(c, AARH_ERR_UNSUPPORTED, "tensor %s is not a linear weight", s.name.c_str());
    const bool expert = s.part == L_GATE || s.part == L_UP || s.part == L_DOWN;
    const int fmt = expert ? c->cfg.expert_format : c->cfg.attn_format;
    if (fmt != AARH_W_INT4_G128)
        return fail(c, AARH_ERR_UNSUPPORTED, "tensor %s is not stored as INT4 g128 in this model", s.name.c_str());
    if (!shape || !data || ndims != 2 || shape[0] != s.rows || shape[1] != s.cols)
        return fail(c, AARH_ERR_SHAPE, "PackedInt4Tensor shape does not match %s [%lld, %lld]", s.name.c_str(),
                    (long long)s.rows, (long long)s.cols);
    const size_t ng = (size_t)s.rows * (s.cols / 128), nb = (size_t)s.rows * s.cols / 2;
    std::vector<uint16_t> sh(ng), zh(ng);
    int r = aarh_packed_i4_params(shape, ndims, group_size, data_len, scales, zeros, n_groups, sh.data(), zh.data());
    if (r) return fail(c, r, "%s: %s", s.name.c_str(), aarh_host_last_error());
    if (ensure_staging(c, (nb + 4 * ng + 3) / 4 + 1)) return AARH_ERR_DEVICE;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    uint8_t* st = (uint8_t*)c->staging;
    HIPCHK(c, hipMemcpy(st, data, nb, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(st + nb, sh.data(), ng * 2, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(st + nb + ng * 2, zh.data(), ng * 2, hipMemcpyHostToDevice));
    const uint16_t* dsh = (const uint16_t*)(st + nb);
    const uint16_t* dzh = (const uint16_t*)(st + nb + ng * 2);
    if (s.part == L_UPK || s.part == L_UPV) {
        LTensor& t = c->tmpq;
        KCHK(c, launch_repack_int4(st, dsh, dzh, (int)s.rows, (int)s.cols, t.w, t.sz, 0, (int)s.rows, 0, c->stream));
        if ((r = split_upkv(c, s))) return r;
        return sync_stream(c);
    }
    LTensor* t = nullptr;
    int ro = 0, inter = 0;
    linear_target(c, s, &t, &ro, &inter);
    KCHK(c, launch_repack_int4(st, dsh, dzh, (int)s.rows, (int)s.cols, t->w, t->sz, ro, t->N, inter, c->stream));
    return sync_stream(c);
}

int aarh_lat_init_synthetic(aarh_lat_ctx* c, uint64_t seed, float std) {
    if (!c) return AARH_ERR_CONFIG;
    size_t maxn = 0;
    for (auto& s : c->slots) maxn = std::max(maxn, (size_t)(s.rows * s.cols));
    if (ensure_staging(c, maxn)) return AARH_ERR_DEVICE;
    const float router_std = 1.0f / sqrtf((float)c->H);
    for (int id = 0; id < (int)c->slots.size(); id++) {
        const LSlot& s = c->slots[id];
        const int64_t n = s.rows * s.cols;
        if (s.kind == AARH_T_NORM) {
            KCHK(c, launch_fill_f32(c->staging, n, 1.0f, c->stream));
        } else {
            KCHK(c, launch_synth_fill(c->staging, n, seed, (unsigned)id, s.part == L_ROUTER ? router_std : std,
                                      c->stream));
        }
        int r = place_staging(c, id);
        if (r) return r;
    }
    return sync_stream(c);
}

int aarh_lat_kv_len(const aarh_lat_ctx* c, int slot, int32_t* out) {
    if (!c || !out || slot < 0 || slot >= c->cfg.max_batch) return AARH_ERR_SHAPE;
    *out = c->kv_len[slot];
    return 0;
}

int aarh_lat_kv_rollback(aarh_lat_ctx* c, int slot, int32_t new_len) {
    if (!c || slot < 0 || slot >= c->cfg.max_batch) return fail(c, AARH_ERR_SHAPE, "bad slot %d", slot);
    if (new_len < 0 || new_len > c->kv_len[slot])
        return fail(c, AARH_ERR_SHAPE, "cannot grow the latent cache from %d to %d with rollback", c->kv_len[slot],
                    new_len);
    c->kv_len[slot] = new_len;
    return 0;
}

int aarh_lat_kv_fill_synthetic(aarh_lat_ctx* c, int slot, int32_t len, uint64_t seed) {
    if (!c || slot < 0 || slot >= c->cfg.max_batch) return fail(c, AARH_ERR_SHAPE, "bad slot %d", slot);
    if (len < 0 || len > c->cfg.max_seq_len)
        return fail(c, AARH_ERR_SHAPE, "length %d exceeds max_seq_len %d", len, c->cfg.max_seq_len);
    for (int l = 0; l < c->L; l++)
        KCHK(c, launch_lat_kv_fill_synthetic(c->kc[l], c->vt[l], slot, c->lat, c->rd, c->cap, len, seed, l, c->stream));
    c->kv_len[slot] = len;
    return sync_stream(c);
}

int aarh_lat_forward(aarh_lat_ctx* c, const uint32_t* ids, const int32_t* slots, const int32_t* offsets, int nseq,
                     int S, float* logits_out, float* hidden_out) {
    if (!c) return AARH_ERR_CONFIG;
    if (!ids || !slots || !offsets) return fail(c, AARH_ERR_SHAPE, "null ids / slots / offsets");
    int mk = 0;
    int r = stage_rows(c, ids, slots, offsets, nseq, S, &mk);
    if (r) return r;
    const int M = nseq * S;
    r = forward_dev(c, nseq, S, mk);
    if (r) return r;
    c->last_M = M;
    for (int b = 0; b < nseq; b++) c->kv_len[slots[b]] = offsets[b] + S;
    if (logits_out)
        HIPCHK(c, hipMemcpyAsync(logits_out, c->logits, (size_t)M * c->V * 4, hipMemcpyDeviceToHost, c->stream));
    if (hidden_out)
        HIPCHK(c, hipMemcpyAsync(hidden_out, c->hidden, (size_t)M * c->H * 4, hipMemcpyDeviceToHost, c->stream));
    return sync_stream(c);
}

int aarh_lat_router_gaps(aarh_lat_ctx* c, float* out) {
    if (!c || !out) return AARH_ERR_CONFIG;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(out, c->gap, (size_t)c->last_M * 4, hipMemcpyDeviceToHost));
    return 0;
}

int aarh_lat_expert_counts(aarh_lat_ctx* c, int32_t* out) {
    if (!c || !out) return AARH_ERR_CONFIG;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(out, c->cnt, (size_t)c->L * (c->E + c->NS) * 4, hipMemcpyDeviceToHost));
    return 0;
}

int aarh_lat_prof_enable(aarh_lat_ctx* c, int enable) {
    if (!c) return AARH_ERR_CONFIG;
    int r = prof_collect(c);
    if (r) return r;
    c->prof = enable != 0;
    for (int i = 0; i < AARH_PROF_COUNT; i++) {
        c->prof_ms[i] = 0;
        c->prof_bytes[i] = 0;
        c->prof_n[i] = 0;
    }
    return 0;
}

int aarh_lat_prof_get(aarh_lat_ctx* c, int cls, double* total_ms, double* alg_bytes_out, int64_t* launches) {
    if (!c || cls < 0 || cls >= AARH_PROF_COUNT) return AARH_ERR_CONFIG;
    int r = prof_collect(c);
    if (r) return r;
    if (total_ms) *total_ms = c->prof_ms[cls];
    if (alg_bytes_out) *alg_bytes_out = c->prof_bytes[cls];
    if (launches) *launches = c->prof_n[cls];
    return 0;
}

}  // extern "C"
