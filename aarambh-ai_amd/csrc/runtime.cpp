// Host runtime of libaarambh_hip: context, device weights, KV cache, the
// verify forward (layer loop over the gfx950 kernels), MTP heads, the MTP
// speculative engine loop, and the C ABI declared in include/aarambh_hip.h.
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

struct DevTensor {
    int fmt = WF_F32;
    int N = 0, K = 0;
    uint8_t* w = nullptr;
    uint32_t* sz = nullptr;
    float* rscale = nullptr;
};

struct BlockW {
    float* norm1 = nullptr;
    float* norm2 = nullptr;
    DevTensor qkv, wo, gu, down;
};

struct HeadW {
    float* trunk = nullptr;
    float* token = nullptr;
    float* out_norm = nullptr;
    BlockW blk;
};

// Tensor ids follow the reference checkpoint order (model.rs:82-279): embedding,
// per layer [norm1, wq, wk, wv, wo, norm2, w_gate, w_up, w_down], final_norm,
// per MTP head [trunk_norm, token_norm, refine.norm1, wq, wk, wv, wo,
// refine.norm2, w_gate, w_up, w_down, output_norm].
enum Part { P_EMBED, P_NORM, P_WQ, P_WK, P_WV, P_WO, P_GATE, P_UP, P_DOWN, P_LMHEAD };
struct TensorSlot {
    std::string name;
    int64_t rows = 0, cols = 0;
    int kind = AARH_T_NORM;
    Part part = P_NORM;
    float** norm_ptr = nullptr;
    BlockW* blk = nullptr;
};

struct ProfRec {
    int cls;
    hipEvent_t a, b;
    double bytes;
};

// A captured verify forward and the arguments its launches bake in.
struct FwdGraph {
    int nseq = 0, S = 0, kv_span = 0;
    float* lout = nullptr;
    RowMap lmap{};
    float* hout = nullptr;
    const uint32_t* ids = nullptr;
    const int32_t *pos0 = nullptr, *slot = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t last_use = 0;
};

}  // namespace

struct aarh_ctx {
    aarh_model_config cfg{};
    int device = 0;
    hipStream_t stream = nullptr;
    // second stream (default priority) for output metadata that no later kernel of the
    // round reads: the top candidates run there beside the acceptance kernel
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    int hd = 0, QD = 0, KD = 0, F = 0, Fp = 0, H = 0, V = 0, nheads_mtp = 0;
    std::string err;

    // weights
    void* embed = nullptr;  // gather table, row-major [V][H] (f32 or bf16)
    int embed_fmt = WF_F32;
    DevTensor lm;           // tied LM head
    std::vector<BlockW> layers;
    float* final_norm = nullptr;
    std::vector<HeadW> heads;
    std::vector<TensorSlot> slots;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    float* staging = nullptr;
    size_t staging_elems = 0;

    // KV cache
    int cap = 0;
    std::vector<void*> kc, vc;
    std::vector<uint16_t*> ksc, vsc;
    std::vector<int> kv_len;
    void *mkc = nullptr, *mvc = nullptr;  // MTP local caches (f32)
    int mcap = 0;

    // scratch
    int Mmax = 0;
    float *x = nullptr, *q = nullptr, *att = nullptr, *h = nullptr, *ssq_a = nullptr, *kvnew = nullptr;
    uint16_t *frag_a = nullptr, *frag_b = nullptr;  // activation fragments (x-like / att-h-like inputs)
    float *hidden = nullptr, *logits = nullptr, *part = nullptr, *apart = nullptr, *hn = nullptr;
    size_t apart_elems = 0;
    unsigned* acnt = nullptr;
    float* gpart = nullptr;     // many-row GEMM split-K partials
    size_t gpart_elems = 0;
    unsigned* gcnt = nullptr;  // its arrival counters
    int32_t *d_pos0 = nullptr, *d_slot = nullptr, *d_zero = nullptr, *d_seqidx = nullptr;
    uint32_t* d_ids = nullptr;
    int32_t *h_pos0 = nullptr, *h_slot = nullptr;
    uint32_t* h_ids = nullptr;
    // pinned staging slots for the small per-call host -> device arrays (row ids,
    // positions, pointer lists): a slot is written again once the event recorded
    // after its copies has completed, so staging needs no stream synchronisation
    static constexpr int STAGE_SLOTS = 8;
    static constexpr size_t STAGE_BYTES = (size_t)64 << 10;
    char* h_stage = nullptr;
    hipEvent_t stage_ev[STAGE_SLOTS] = {};
    bool stage_busy[STAGE_SLOTS] = {};
    int stage_next = 0;
    // acceptance scratch: row distribution parameters and per-sequence arrival counters
    uint32_t* acc_rstat = nullptr;
    unsigned* acc_cnt = nullptr;
    int acc_rows_cap = 0, acc_seq_cap = 0;

    // captured verify forwards
    bool graphs = true;
    std::vector<FwdGraph> gcache;
    uint64_t gclock = 0;

    // profiling
    int replay_schedule = AARH_REPLAY_REPLACEMENT;
    bool prof = false;
    std::vector<ProfRec> prof_recs;
    std::vector<hipEvent_t> ev_pool;
    double prof_ms[AARH_PROF_COUNT] = {0};
    double prof_bytes[AARH_PROF_COUNT] = {0};
    int64_t prof_n[AARH_PROF_COUNT] = {0};
};

namespace {

int fail(aarh_ctx* c, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (c) c->err = buf;
    return code;
}

#define HIPCHK(c, call)                                                                        \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess) return fail((c), AARH_ERR_DEVICE, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

#define KCHK(c, call)                                                                          \
    do {                                                                                       \
        int r_ = (call);                                                                       \
        if (r_ != 0) return fail((c), r_, "kernel launch failed: %s (code %d: %s)", #call, r_, last_launch_error()); \
    } while (0)

template <class T>
int dalloc(aarh_ctx* c, T** p, size_t bytes) {
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

// Algorithmic bytes a launch must move: quantised weights and their scales.
double alg_weight_bytes(const DevTensor& t) {
    double b = (double)weight_bytes(t.fmt, t.N, t.K);
    if (t.fmt == WF_INT4) b += (double)t.N * (t.K / 128) * 4.0;
    if (t.fmt == WF_INT8) b += (double)t.N * 4.0;
    return b;
}

int alloc_tensor(aarh_ctx* c, DevTensor& t, int fmt, int N, int K) {
    t.fmt = fmt;
    t.N = N;
    t.K = K;
    // GEMV / GEMM address weights through one buffer resource with 32-bit byte offsets
    if (weight_bytes(fmt, N, K) >= ((size_t)1 << 31))
        return fail(c, AARH_ERR_UNSUPPORTED, "a %d x %d weight matrix of %zu bytes exceeds the 2 GiB per-tensor limit", N,
                    K, weight_bytes(fmt, N, K));
    if (dalloc(c, &t.w, weight_bytes(fmt, N, K))) return AARH_ERR_DEVICE;
    HIPCHK(c, hipMemset(t.w, 0, weight_bytes(fmt, N, K)));
    if (fmt == WF_INT4) {
        size_t n = (size_t)N / 16 * (K / 128) * 16;
        if (dalloc(c, &t.sz, n * 4)) return AARH_ERR_DEVICE;
        // scale 1.0, zero 0 for never-loaded rows (fp16 0x3C00)
        std::vector<uint32_t> ones(n, 0x3C00u);
        HIPCHK(c, hipMemcpy(t.sz, ones.data(), n * 4, hipMemcpyHostToDevice));
    }
    if (fmt == WF_INT8) {
        if (dalloc(c, &t.rscale, (size_t)N * 4)) return AARH_ERR_DEVICE;
        std::vector<float> ones(N, 1.0f);
        HIPCHK(c, hipMemcpy(t.rscale, ones.data(), (size_t)N * 4, hipMemcpyHostToDevice));
    }
    return 0;
}

void free_tensor(DevTensor& t) {
    if (t.w) (void)hipFree(t.w);
    if (t.sz) (void)hipFree(t.sz);
    if (t.rscale) (void)hipFree(t.rscale);
    t = DevTensor{};
}

hipEvent_t take_event(aarh_ctx* c) {
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
    aarh_ctx* c;
    int cls;
    double bytes;
    hipEvent_t a = nullptr;
    hipEvent_t b = nullptr;
    // Instrumented launches inside the scope re-record a / b at their own dispatch
    // start / end; a scope without one keeps the stream-order records taken here.
    ProfScope(aarh_ctx* c_, int cls_, double bytes_) : c(c_), cls(cls_), bytes(bytes_) {
        if (c->prof) {
            a = take_event(c);
            b = take_event(c);
            (void)hipEventRecord(a, c->stream);
            g_launch_timing = {a, b, 0};
        }
    }
    ~ProfScope() {
        if (c->prof) {
            if (g_launch_timing.launches == 0) (void)hipEventRecord(b, c->stream);
            g_launch_timing = {nullptr, nullptr, 0};
            c->prof_recs.push_back({cls, a, b, bytes});
        }
    }
};

// Fragment row tile of an M-row activation (hi + lo halves; 16-row chunks for
// the many-row GEMM).  Plain fp16 activations would halve the GEMM's MFMA work
// but measured up to 2.8e-3 relative logit error on random-init models (the
// INT8 KV cache turns k errors of 2^-12 into flipped codes), above the 2e-3
// bar, so every projection keeps the lo halves.
int frag_mp(int M) { return M <= 4 ? 4 : (M <= 8 ? 8 : 16); }

// Cache positions past max_seq_len reserved for padding rows of ragged batches.
constexpr int PAD_SLACK = 32;

// Fragments of an activation matrix for a consumer of format `fmt` with K = k
// (null buffer: the consumer reads f32 rows).
XFrag xfrag(aarh_ctx* c, uint16_t* buf, int fmt, int k, int mp, const float* norm_w, bool ssq) {
    XFrag f{};
    if (fmt == WF_F32) return f;
    f.buf = buf;
    f.fmt = fmt;
    f.mp = mp;
    f.G = k / 128;
    f.norm_w = norm_w;
    f.ssq = ssq ? c->ssq_a : nullptr;
    f.ssq_ld = c->H / 16;
    return f;
}

// y = x . W^T over M activation rows with a fused RMSNorm input (norm_w) and
// epilogue; launched in chunks of at most 16 rows.  Quantised weights read the
// input as fragments `xf` (row tile mp) with the RMSNorm statistic from the
// producer's partial sums; f32 weights read the rows x.  `fo` receives the
// RESID / SWIGLU result as fragments for the next consumer.
int gemv(aarh_ctx* c, const DevTensor& t, int M, const float* x, RowMap xmap, const uint16_t* xf, int mp,
         const float* norm_w, float* hidden_out, int epi, float* out, RowMap omap, float* resid, int ldr,
         const XFrag& fo, const QkvEpi* qkv, int cls) {
    GemvArgs a{};
    a.fmt = t.fmt;
    a.w = t.w;
    a.sz = t.sz;
    a.rscale = t.rscale;
    a.N = t.N;
    a.K = t.K;
    a.x = x;
    a.xmap = xmap;
    a.xf = xf;
    a.mp = mp;
    a.norm_w = norm_w;
    a.ssq_in = c->ssq_a;
    a.ssq_ld = c->H / 16;
    a.eps = c->cfg.norm_eps;
    a.hidden_out = hidden_out;
    a.epi = epi;
    a.out = out;
    a.omap = omap;
    a.resid = resid;
    a.ldr = ldr;
    a.fo = fo;
    a.gpart = c->gpart;
    a.gcnt = c->gcnt;
    a.gpart_elems = (long long)c->gpart_elems;
    if (qkv) a.qkv = *qkv;
    if (t.fmt != WF_F32 && M > 16) {
        ProfScope ps(c, cls, alg_weight_bytes(t));
        a.m_base = 0;
        a.M = M;
        int r = launch_gemm(a, c->stream);
        if (r)
            return fail(c, r, "gemm launch failed (fmt %d N %d K %d M %d): code %d %s", t.fmt, t.N, t.K, M, r,
                        last_launch_error());
        return 0;
    }
    ProfScope ps(c, cls, alg_weight_bytes(t) * ((M + 15) / 16));
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

RowMap rm(int S, long long seq_stride, long long row_stride) {
    RowMap r;
    r.S = S;
    r.seq_stride = seq_stride;
    r.row_stride = row_stride;
    return r;
}

// One transformer block (block.rs:331-350) over M = nseq * S rows whose
// residual stream is c->x and whose ssq partials for norm1 are in c->ssq_a.
// The input x arrives with fragments in frag_a for w.qkv (norm1); `after`
// describes the consumer of the block's output x (next block or LM head).
int run_block(aarh_ctx* c, const BlockW& w, int nseq, int S, const int32_t* d_pos0, const int32_t* d_slot,
              int kv_fmt, int cap, void* kc, void* vc, uint16_t* ks, uint16_t* vs, int max_kv_len,
              const XFrag& after) {
    const int M = nseq * S, H = c->H;
    const int mp = frag_mp(M);
    QkvEpi e{};
    e.n_heads = c->cfg.n_heads;
    e.n_kv = c->cfg.n_kv_heads;
    e.hd = c->hd;
    e.S = S;
    e.pos0 = d_pos0;
    e.rope_cos = c->rope_cos;
    e.rope_sin = c->rope_sin;
    e.q_out = c->q;
    e.kv_out = c->kvnew;
    int r;
    if ((r = gemv(c, w.qkv, M, c->x, rm(M, 0, H), c->frag_a, mp, w.norm1, nullptr, EPI_QKV, nullptr, rm(S, 0, 0),
                  nullptr, 0, XFrag{}, &e, AARH_PROF_GEMV_QKV)))
        return r;
    // attention
    AttnArgs at{};
    at.nseq = nseq;
    at.S = S;
    at.n_heads = c->cfg.n_heads;
    at.n_kv = c->cfg.n_kv_heads;
    at.hd = c->hd;
    at.pos0 = d_pos0;
    at.slot = d_slot;
    at.q = c->q;
    at.knew = c->kvnew;
    at.kv_fmt = kv_fmt;
    at.cap = cap;
    at.kc = kc;
    at.vc = vc;
    at.ks = ks;
    at.vs = vs;
    at.scale = (float)(1.0 / std::sqrt((double)c->hd));
    const int G = c->cfg.n_heads / c->cfg.n_kv_heads;
    const int Rt = S * G;
    const bool mf = attention_uses_mfma(kv_fmt, c->hd);
    // tokens per chunk granule (MFMA: 8 waves x 32-token blocks) and target workgroup count
    // (MFMA: one 8-wave workgroup per CU)
    const int gran = mf ? 256 : 64;
    const int target = mf ? 256 : 512;
    at.rows_per_tile = std::min(mf ? 16 : 32, Rt);
    at.ntiles = (Rt + at.rows_per_tile - 1) / at.rows_per_tile;
    const int base = nseq * c->cfg.n_kv_heads * at.ntiles;
    const int max_chunks = std::max(1, (max_kv_len + gran - 1) / gran);
    int nch = std::max(1, std::min(std::min(max_chunks, mf ? 32 : 64), (target + base - 1) / base));
    int chunk = ((max_kv_len + nch - 1) / nch + gran - 1) / gran * gran;
    nch = (max_kv_len + chunk - 1) / chunk;
    at.chunk = chunk;
    at.nchunks = nch;
    size_t need = (size_t)base * nch * 32 * (c->hd + 4);
    if (need > c->apart_elems) return fail(c, AARH_ERR_SHAPE, "attention scratch too small");
    at.part = c->apart;
    at.counters = c->acnt;
    at.out = c->att;
    at.fo = xfrag(c, c->frag_b, w.wo.fmt, c->QD, mp, nullptr, false);
    {
        double kvb = 0;
        if (kv_fmt == KV_INT8) kvb = (double)max_kv_len * nseq * c->cfg.n_kv_heads * (2.0 * c->hd + 4.0);
        else kvb = (double)max_kv_len * nseq * c->cfg.n_kv_heads * 2.0 * c->hd * (kv_fmt == KV_F16 ? 2 : 4);
        ProfScope ps(c, AARH_PROF_ATTENTION, kvb);
        KCHK(c, launch_attention(at, c->stream));
    }
    if ((r = gemv(c, w.wo, M, c->att, rm(M, 0, c->QD), c->frag_b, mp, nullptr, nullptr, EPI_RESID, nullptr,
                  rm(1, 0, 0), c->x, H, xfrag(c, c->frag_a, w.gu.fmt, H, mp, w.norm2, true), nullptr,
                  AARH_PROF_GEMV_WO)))
        return r;
    // h as f32 rows only when the down projection reads rows (f32 weights); quantised
    // weights read the fragments written beside it
    if ((r = gemv(c, w.gu, M, c->x, rm(M, 0, H), c->frag_a, mp, w.norm2, nullptr, EPI_SWIGLU,
                  w.down.fmt == WF_F32 ? c->h : nullptr, rm(M, 0, c->Fp),
                  nullptr, 0, xfrag(c, c->frag_b, w.down.fmt, c->Fp, mp, nullptr, false), nullptr,
                  AARH_PROF_GEMV_GATEUP)))
        return r;
    if ((r = gemv(c, w.down, M, c->h, rm(M, 0, c->Fp), c->frag_b, mp, nullptr, nullptr, EPI_RESID, nullptr,
                  rm(1, 0, 0), c->x, H, after, nullptr, AARH_PROF_GEMV_DOWN)))
        return r;
    return 0;
}

// forward_with_cache_output on device: ids/pos0/slot are device arrays for
// nseq sequences x S tokens; logits go to `lout` via `lmap`, normed hidden to
// `hout` ([M][H]) when non-null.  kv_span bounds max(pos0) + S (it sets the
// attention's chunking; chunks past a sequence's own length are empty).
int forward_launches(aarh_ctx* c, const uint32_t* d_ids, const int32_t* d_pos0, const int32_t* d_slot, int nseq,
                     int S, int kv_span, float* lout, RowMap lmap, float* hout) {
    const int M = nseq * S, H = c->H;
    const int mp = frag_mp(M);
    {
        ProfScope ps(c, AARH_PROF_OTHER, 0);
        const BlockW& b0 = c->layers[0];
        KCHK(c, launch_embed(c->embed, c->embed_fmt, H, d_ids, M, c->x,
                             xfrag(c, c->frag_a, b0.qkv.fmt, H, mp, b0.norm1, true), c->stream));
    }
    for (int l = 0; l < c->cfg.n_layers; l++) {
        const XFrag after = l + 1 < c->cfg.n_layers
                                ? xfrag(c, c->frag_a, c->layers[l + 1].qkv.fmt, H, mp, c->layers[l + 1].norm1, true)
                                : xfrag(c, c->frag_a, c->lm.fmt, H, mp, c->final_norm, true);
        int r = run_block(c, c->layers[l], nseq, S, d_pos0, d_slot, c->cfg.kv_format, c->cap, c->kc[l], c->vc[l],
                          c->ksc[l], c->vsc[l], kv_span, after);
        if (r) return r;
    }
    return gemv(c, c->lm, M, c->x, rm(M, 0, H), c->frag_a, mp, c->final_norm, hout, EPI_STORE, lout, lmap, nullptr,
                0, XFrag{}, nullptr, AARH_PROF_GEMV_LMHEAD);
}

// The verify forward is about 5 launches per layer of 5-80 us kernels; host
// launch cost is of the same order, so repeated shapes replay a captured HIP
// graph (one host call).  Key: everything the launches bake in.  A shape is
// captured the second time it is seen (the first run also initialises the
// launchers' one-time attributes outside any capture).  Prompt prefill chunks
// (more rows per sequence than any round forward has) run without a graph: their
// kernels are long enough to hide the launches, and their shapes (the last chunk of
// each prompt length) rarely repeat, so capturing them would only churn the cache.
constexpr int GRAPH_KV_GRANULE = 256;  // kv_span rounding: one graph serves 256 cache positions
constexpr size_t GRAPH_CACHE_MAX = 160;
constexpr int GRAPH_MAX_S = PAD_SLACK;  // verify and replay forwards have at most num_draft_tokens + 1 rows

bool same_key(const FwdGraph& g, const FwdGraph& k) {
    return g.nseq == k.nseq && g.S == k.S && g.kv_span == k.kv_span && g.lout == k.lout && g.hout == k.hout &&
           g.lmap.S == k.lmap.S && g.lmap.seq_stride == k.lmap.seq_stride && g.lmap.row_stride == k.lmap.row_stride &&
           g.ids == k.ids && g.pos0 == k.pos0 && g.slot == k.slot;
}

int forward_dev(aarh_ctx* c, const uint32_t* d_ids, const int32_t* d_pos0, const int32_t* d_slot, int nseq, int S,
                int max_kv_len, float* lout, RowMap lmap, float* hout) {
    const int M = nseq * S;
    if (M > c->Mmax) return fail(c, AARH_ERR_SHAPE, "rows %d exceed max_rows %d", M, c->Mmax);
    const int kv_span = std::min(c->cap, (max_kv_len + GRAPH_KV_GRANULE - 1) / GRAPH_KV_GRANULE * GRAPH_KV_GRANULE);
    if (!c->graphs || c->prof || S > GRAPH_MAX_S)
        return forward_launches(c, d_ids, d_pos0, d_slot, nseq, S, kv_span, lout, lmap, hout);
    FwdGraph key{};
    key.nseq = nseq;
    key.S = S;
    key.kv_span = kv_span;
    key.lout = lout;
    key.lmap = lmap;
    key.hout = hout;
    key.ids = d_ids;
    key.pos0 = d_pos0;
    key.slot = d_slot;
    for (auto& g : c->gcache) {
        if (!same_key(g, key)) continue;
        g.last_use = ++c->gclock;
        if (g.exec) {
            HIPCHK(c, hipGraphLaunch(g.exec, c->stream));
            return 0;
        }
        // second sighting: capture this shape's launches once, then replay
        hipGraph_t graph = nullptr;
        HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        int r = forward_launches(c, d_ids, d_pos0, d_slot, nseq, S, kv_span, lout, lmap, hout);
        hipError_t e = hipStreamEndCapture(c->stream, &graph);
        if (r) {
            if (graph) (void)hipGraphDestroy(graph);
            return r;
        }
        if (e != hipSuccess) return fail(c, AARH_ERR_DEVICE, "graph capture failed: %s", hipGetErrorString(e));
        e = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (e != hipSuccess) {
            g.exec = nullptr;
            return fail(c, AARH_ERR_DEVICE, "graph instantiation failed: %s", hipGetErrorString(e));
        }
        HIPCHK(c, hipGraphLaunch(g.exec, c->stream));
        return 0;
    }
    // first sighting: run directly and remember the shape (evicting the least recently used)
    if (c->gcache.size() >= GRAPH_CACHE_MAX) {
        auto lru = std::min_element(c->gcache.begin(), c->gcache.end(),
                                    [](const FwdGraph& a, const FwdGraph& b) { return a.last_use < b.last_use; });
        if (lru->exec) (void)hipGraphExecDestroy(lru->exec);
        c->gcache.erase(lru);
    }
    key.last_use = ++c->gclock;
    c->gcache.push_back(key);
    return forward_launches(c, d_ids, d_pos0, d_slot, nseq, S, kv_span, lout, lmap, hout);
}

// forward_mtp_head on device for nseq sequences: anchor rows (stride), ids
// [nseq][ids_stride] (first head+1 used); logits row of seq j -> lout + j*lstride.
int mtp_head_dev(aarh_ctx* c, int head, const float* d_anchor, long long anchor_stride, const uint32_t* d_ids,
                 int ids_stride, int nseq, float* lout, long long lstride) {
    if (head < 0 || head >= c->nheads_mtp) return fail(c, AARH_ERR_CONFIG, "MTP head index %d is not configured", head);
    const int L = head + 2, H = c->H;
    if (nseq * L > c->Mmax) return fail(c, AARH_ERR_SHAPE, "MTP rows exceed max_rows");
    const HeadW& hw = c->heads[head];
    {
        ProfScope ps(c, AARH_PROF_OTHER, 0);
        KCHK(c, launch_mtp_prep(d_anchor, anchor_stride, c->embed, c->embed_fmt, d_ids, ids_stride, nseq, L, H, hw.trunk,
                                hw.token, c->cfg.norm_eps, c->x,
                                xfrag(c, c->frag_a, hw.blk.qkv.fmt, H, frag_mp(nseq * L), hw.blk.norm1, true),
                                c->stream));
    }
    // local cache slots 0..nseq-1 at positions 0..L-1 (no KV cache: mtp.rs:104-114)
    int r = run_block(c, hw.blk, nseq, L, c->d_zero, c->d_seqidx, KV_F32, c->mcap, c->mkc, c->mvc, nullptr, nullptr, L,
                      XFrag{});
    if (r) return r;
    const int mp = frag_mp(nseq);
    {
        ProfScope ps(c, AARH_PROF_OTHER, 0);
        KCHK(c, launch_norm_rows(c->x + (size_t)(L - 1) * H, rm(1, (long long)L * H, 0), nseq, H, hw.out_norm,
                                 c->cfg.norm_eps, c->hn, xfrag(c, c->frag_a, c->lm.fmt, H, mp, nullptr, false),
                                 c->stream));
    }
    // LM head without a norm prologue on the normalised last rows
    DevTensor lm = c->lm;
    return gemv(c, lm, nseq, c->hn, rm(nseq, 0, H), c->frag_a, mp, nullptr, nullptr, EPI_STORE, lout,
                rm(1, lstride, 0), nullptr, 0, XFrag{}, nullptr, AARH_PROF_GEMV_LMHEAD);
}

int sync_stream(aarh_ctx* c) {
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return 0;
}

// The next pinned staging slot (STAGE_BYTES), once the copies that last read it
// have run; nullptr when the context has no staging slots or the wait fails.
char* stage_acquire(aarh_ctx* c, int* slot) {
    if (!c->h_stage) return nullptr;
    const int i = c->stage_next;
    c->stage_next = (i + 1) % aarh_ctx::STAGE_SLOTS;
    if (c->stage_busy[i]) {
        if (hipEventSynchronize(c->stage_ev[i]) != hipSuccess) return nullptr;
        c->stage_busy[i] = false;
    }
    *slot = i;
    return c->h_stage + (size_t)i * aarh_ctx::STAGE_BYTES;
}

// Marks a slot in use until the copies enqueued from it so far have run.
int stage_release(aarh_ctx* c, int slot) {
    HIPCHK(c, hipEventRecord(c->stage_ev[slot], c->stream));
    c->stage_busy[slot] = true;
    return 0;
}

}  // namespace

namespace aarh {
// Records a failure on a context for the library's other translation units (weights.cpp).
int ctx_fail(aarh_ctx* c, int code, const char* msg) { return fail(c, code, "%s", msg); }
// RopeScalingConfig::validate (config.rs:52-96) of a checkpoint config, for weights.cpp.
int rope_scaling_check(int head_dim, int max_seq_len, const aarh_rope_scaling* s, std::string& err);
}  // namespace aarh

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* aarh_last_error(const aarh_ctx* c) { return c ? c->err.c_str() : "null context"; }
void* aarh_stream(aarh_ctx* c) { return c ? (void*)c->stream : nullptr; }
int aarh_sync(aarh_ctx* c) { return sync_stream(c); }

void aarh_destroy(aarh_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (auto& g : c->gcache)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
    auto F = [](void* p) {
        if (p) (void)hipFree(p);
    };
    F(c->embed);
    if (c->lm.w != c->embed) free_tensor(c->lm);
    for (auto& b : c->layers) {
        F(b.norm1);
        F(b.norm2);
        free_tensor(b.qkv);
        free_tensor(b.wo);
        free_tensor(b.gu);
        free_tensor(b.down);
    }
    F(c->final_norm);
    for (auto& h : c->heads) {
        F(h.trunk);
        F(h.token);
        F(h.out_norm);
        F(h.blk.norm1);
        F(h.blk.norm2);
        free_tensor(h.blk.qkv);
        free_tensor(h.blk.wo);
        free_tensor(h.blk.gu);
        free_tensor(h.blk.down);
    }
    F(c->rope_cos);
    F(c->rope_sin);
    F(c->staging);
    for (size_t i = 0; i < c->kc.size(); i++) {
        F(c->kc[i]);
        F(c->vc[i]);
        F(c->ksc[i]);
        F(c->vsc[i]);
    }
    F(c->mkc);
    F(c->mvc);
    for (void* p : {(void*)c->x, (void*)c->q, (void*)c->att, (void*)c->h, (void*)c->ssq_a, (void*)c->kvnew,
                    (void*)c->frag_a, (void*)c->frag_b,
                    (void*)c->hidden, (void*)c->logits, (void*)c->apart, (void*)c->hn,
                    (void*)c->acnt, (void*)c->gpart, (void*)c->gcnt, (void*)c->d_pos0, (void*)c->d_slot, (void*)c->d_zero, (void*)c->d_seqidx,
                    (void*)c->d_ids, (void*)c->acc_rstat, (void*)c->acc_cnt})
        F(p);
    if (c->h_pos0) (void)hipHostFree(c->h_pos0);
    if (c->h_slot) (void)hipHostFree(c->h_slot);
    if (c->h_ids) (void)hipHostFree(c->h_ids);
    if (c->h_stage) (void)hipHostFree(c->h_stage);
    for (auto ev : c->stage_ev)
        if (ev) (void)hipEventDestroy(ev);
    for (auto& r : c->prof_recs) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    for (auto e : c->ev_pool) (void)hipEventDestroy(e);
    if (c->side) {
        (void)hipStreamSynchronize(c->side);
        (void)hipStreamDestroy(c->side);
    }
    if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
    if (c->ev_join) (void)hipEventDestroy(c->ev_join);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

static int build_slots(aarh_ctx* c) {
    const auto& g = c->cfg;
    const int64_t H = g.hidden_dim, F = g.ffn_dim, QD = c->QD, KD = c->KD;
    auto add = [&](const std::string& n, int64_t r, int64_t cc, int kind, Part p, float** np, BlockW* b) {
        TensorSlot s;
        s.name = n;
        s.rows = r;
        s.cols = cc;
        s.kind = kind;
        s.part = p;
        s.norm_ptr = np;
        s.blk = b;
        c->slots.push_back(s);
    };
    add("embedding.weight", g.vocab_size, H, AARH_T_EMBED, P_EMBED, nullptr, nullptr);
    for (int l = 0; l < g.n_layers; l++) {
        BlockW* b = &c->layers[l];
        std::string p = "blocks." + std::to_string(l) + ".";
        add(p + "norm1.weight", 1, H, AARH_T_NORM, P_NORM, &b->norm1, b);
        add(p + "attn.wq.weight", QD, H, AARH_T_LINEAR, P_WQ, nullptr, b);
        add(p + "attn.wk.weight", KD, H, AARH_T_LINEAR, P_WK, nullptr, b);
        add(p + "attn.wv.weight", KD, H, AARH_T_LINEAR, P_WV, nullptr, b);
        add(p + "attn.wo.weight", H, QD, AARH_T_LINEAR, P_WO, nullptr, b);
        add(p + "norm2.weight", 1, H, AARH_T_NORM, P_NORM, &b->norm2, b);
        add(p + "ffn.w_gate.weight", F, H, AARH_T_LINEAR, P_GATE, nullptr, b);
        add(p + "ffn.w_up.weight", F, H, AARH_T_LINEAR, P_UP, nullptr, b);
        add(p + "ffn.w_down.weight", H, F, AARH_T_LINEAR, P_DOWN, nullptr, b);
    }
    add("final_norm.weight", 1, H, AARH_T_NORM, P_NORM, &c->final_norm, nullptr);
    for (int h = 0; h < c->nheads_mtp; h++) {
        HeadW* hw = &c->heads[h];
        BlockW* b = &hw->blk;
        std::string p = "mtp.heads." + std::to_string(h) + ".";
        add(p + "trunk_norm.weight", 1, H, AARH_T_NORM, P_NORM, &hw->trunk, nullptr);
        add(p + "token_norm.weight", 1, H, AARH_T_NORM, P_NORM, &hw->token, nullptr);
        add(p + "refine.norm1.weight", 1, H, AARH_T_NORM, P_NORM, &b->norm1, b);
        add(p + "refine.attn.wq.weight", QD, H, AARH_T_LINEAR, P_WQ, nullptr, b);
        add(p + "refine.attn.wk.weight", KD, H, AARH_T_LINEAR, P_WK, nullptr, b);
        add(p + "refine.attn.wv.weight", KD, H, AARH_T_LINEAR, P_WV, nullptr, b);
        add(p + "refine.attn.wo.weight", H, QD, AARH_T_LINEAR, P_WO, nullptr, b);
        add(p + "refine.norm2.weight", 1, H, AARH_T_NORM, P_NORM, &b->norm2, b);
        add(p + "refine.ffn.w_gate.weight", F, H, AARH_T_LINEAR, P_GATE, nullptr, b);
        add(p + "refine.ffn.w_up.weight", F, H, AARH_T_LINEAR, P_UP, nullptr, b);
        add(p + "refine.ffn.w_down.weight", H, F, AARH_T_LINEAR, P_DOWN, nullptr, b);
        add(p + "output_norm.weight", 1, H, AARH_T_NORM, P_NORM, &hw->out_norm, nullptr);
    }
    // LmHead::untied_with_qat (model.rs:239-248): its own [vocab, hidden] weight, which the
    // MTP heads' output projection shares (model.rs:250-262)
    if (g.untied_lm_head) add("lm_head.weight", g.vocab_size, H, AARH_T_EMBED, P_LMHEAD, nullptr, nullptr);
    return 0;
}

static int alloc_block(aarh_ctx* c, BlockW& b) {
    const int fmt = c->cfg.weight_format, H = c->H;
    if (dalloc(c, &b.norm1, H * 4) || dalloc(c, &b.norm2, H * 4)) return AARH_ERR_DEVICE;
    KCHK(c, launch_fill_f32(b.norm1, H, 1.0f, c->stream));
    KCHK(c, launch_fill_f32(b.norm2, H, 1.0f, c->stream));
    int r;
    if ((r = alloc_tensor(c, b.qkv, fmt, c->QD + 2 * c->KD, H))) return r;
    if ((r = alloc_tensor(c, b.wo, fmt, H, c->QD))) return r;
    if ((r = alloc_tensor(c, b.gu, fmt, 2 * c->Fp, H))) return r;
    if ((r = alloc_tensor(c, b.down, fmt, H, c->Fp))) return r;
    return 0;
}

}  // extern "C"

namespace {

// Inverse frequencies and cos / sin factor of the model's RoPE (inverse_frequencies_for_config,
// rope_scaling.rs:24-33): base frequencies (:6-11), linear (:46-52), NTK-aware theta (:14-22,
// 53-56) or YaRN (:62-92, correction range :107-136), all in f64 and cast to f32.
// Returns 0, or AARH_ERR_CONFIG with RopeScalingConfig::validate's message (config.rs:52-98).
int rope_frequencies(int hd, double theta, int max_seq_len, const aarh_rope_scaling* s, std::vector<float>& inv,
                     float* attn, std::string& err) {
    const int half = hd / 2;
    inv.assign(half, 0.0f);
    *attn = 1.0f;
    auto base = [&](double th, std::vector<float>& out) {
        for (int i = 0; i < half; i++) out[i] = (float)(1.0 / std::pow(th, 2.0 * (double)i / (double)hd));
    };
    if (!s || s->method == AARH_ROPE_NONE) {
        base(theta, inv);
        return 0;
    }
    if (!(s->factor > 1.0) || !std::isfinite(s->factor)) {
        err = "rope_scaling.factor must be finite and greater than 1.0";
        return AARH_ERR_CONFIG;
    }
    if (s->original_max_seq_len <= 0) {
        err = "rope_scaling.original_max_seq_len must be non-zero";
        return AARH_ERR_CONFIG;
    }
    if (max_seq_len < s->original_max_seq_len) {
        err = "max_seq_len " + std::to_string(max_seq_len) + " must be >= rope_scaling.original_max_seq_len " +
              std::to_string(s->original_max_seq_len);
        return AARH_ERR_CONFIG;
    }
    if (hd <= 2) {
        err = "head_dim must be greater than 2 for RoPE scaling";
        return AARH_ERR_CONFIG;
    }
    if (!(s->attn_factor > 0.0) || !std::isfinite(s->attn_factor)) {
        err = "rope_scaling.attn_factor must be finite and positive";
        return AARH_ERR_CONFIG;
    }
    if (s->method == AARH_ROPE_YARN) {
        if (!(s->beta_fast > 0.0) || !(s->beta_slow > 0.0) || !std::isfinite(s->beta_fast) ||
            !std::isfinite(s->beta_slow)) {
            err = "rope_scaling beta values must be finite and positive";
            return AARH_ERR_CONFIG;
        }
        if (s->beta_fast <= s->beta_slow) {
            err = "rope_scaling.beta_fast must be greater than beta_slow";
            return AARH_ERR_CONFIG;
        }
    }
    *attn = (float)s->attn_factor;
    if (s->method == AARH_ROPE_LINEAR) {
        base(theta, inv);
        const float f = (float)s->factor;
        for (int i = 0; i < half; i++) inv[i] = inv[i] / f;
        return 0;
    }
    if (s->method == AARH_ROPE_NTK) {
        base(theta * std::pow(s->factor, (double)hd / ((double)hd - 2.0)), inv);
        return 0;
    }
    if (s->method != AARH_ROPE_YARN) {
        err = "unknown rope_scaling method";
        return AARH_ERR_CONFIG;
    }
    // YaRN: blend of the extrapolated and interpolated frequency by a linear ramp over the
    // correction range [low, high] of dimension indices
    const double pi = 3.14159265358979323846;
    auto corr_dim = [&](double rot) {
        return (double)hd * std::log((double)s->original_max_seq_len / (rot * 2.0 * pi)) / (2.0 * std::log(theta));
    };
    const double max_dim = (double)std::max(0, half - 1);
    double low = std::min(std::max(std::floor(corr_dim(s->beta_fast)), 0.0), max_dim);
    double high = std::min(std::max(std::ceil(corr_dim(s->beta_slow)), 0.0), max_dim);
    if (std::fabs(high - low) < 2.220446049250313e-16) high += 0.001;
    for (int i = 0; i < half; i++) {
        const double extrapolated = 1.0 / std::pow(theta, 2.0 * (double)i / (double)hd);
        const double interpolated = extrapolated / s->factor;
        const double ramp = std::min(std::max(((double)i - low) / (high - low), 0.0), 1.0);
        inv[i] = (float)(interpolated * ramp + extrapolated * (1.0 - ramp));
    }
    return 0;
}

}  // namespace

int aarh::rope_scaling_check(int head_dim, int max_seq_len, const aarh_rope_scaling* s, std::string& err) {
    std::vector<float> inv;
    float attn = 1.0f;
    if (head_dim <= 0 || head_dim % 2) {
        err = "RoPE head_dim must be non-zero and even";
        return AARH_ERR_CONFIG;
    }
    return rope_frequencies(head_dim, 10000.0, max_seq_len, s, inv, &attn, err);
}

namespace {

// cos / sin tables [positions][hd / 2] (rope.rs:43-72: angle pos * freq in f32, times the
// attention factor) uploaded into the context's table buffers.
int upload_rope(aarh_ctx* c, const aarh_rope_scaling* s) {
    const int half = c->hd / 2, npos = c->cfg.max_seq_len + PAD_SLACK;
    std::vector<float> inv;
    float attn = 1.0f;
    std::string err;
    int r = rope_frequencies(c->hd, (double)c->cfg.rope_theta, c->cfg.max_seq_len, s, inv, &attn, err);
    if (r) return fail(c, r, "%s", err.c_str());
    std::vector<float> cs((size_t)npos * half), sn((size_t)npos * half);
    for (int p = 0; p < npos; p++)
        for (int i = 0; i < half; i++) {
            const float a = (float)p * inv[i];
            cs[(size_t)p * half + i] = cosf(a) * attn;
            sn[(size_t)p * half + i] = sinf(a) * attn;
        }
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(c->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(c->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    return 0;
}

}  // namespace

extern "C" {

int aarh_create(int device, const aarh_model_config* cfg, aarh_ctx** out) {
    if (!cfg || !out) return AARH_ERR_CONFIG;
    *out = nullptr;
    aarh_ctx* c = new aarh_ctx();
    c->cfg = *cfg;
    c->device = device;
    const auto& g = *cfg;
    auto bad = [&](int code, const char* msg) {
        c->err = msg;
        *out = c;
        return code;
    };
    if (g.vocab_size <= 0 || g.hidden_dim <= 0 || g.ffn_dim <= 0 || g.n_layers <= 0 || g.n_heads <= 0 ||
        g.n_kv_heads <= 0 || g.max_seq_len <= 0 || g.max_batch <= 0 || g.max_rows <= 0)
        return bad(AARH_ERR_CONFIG, "model dimensions must be non-zero");
    if (g.hidden_dim % g.n_heads || g.n_heads % g.n_kv_heads)
        return bad(AARH_ERR_CONFIG, "hidden_dim must divide by n_heads and n_heads by n_kv_heads");
    c->H = g.hidden_dim;
    c->V = g.vocab_size;
    c->hd = g.hidden_dim / g.n_heads;
    c->QD = g.n_heads * c->hd;
    c->KD = g.n_kv_heads * c->hd;
    c->F = g.ffn_dim;
    c->nheads_mtp = g.num_future_tokens > 1 ? g.num_future_tokens - 1 : 0;
    if (c->hd > 128 || 128 % c->hd || c->hd % 16)
        return bad(AARH_ERR_UNSUPPORTED, "head_dim must be 16, 32, 64 or 128");
    if (c->H % 128 || c->V % 128 || (c->QD + 2 * c->KD) % 128)
        return bad(AARH_ERR_UNSUPPORTED, "hidden, vocab and q+k+v widths must be multiples of 128");
    if (g.weight_format != AARH_W_F32 && g.ffn_dim % 128)
        return bad(AARH_ERR_UNSUPPORTED, "quantised ffn_dim must be a multiple of 128");
    if (g.weight_format < 0 || g.weight_format > 3 || (g.lm_head_format != 0 && g.lm_head_format != 1) ||
        g.kv_format < 0 || g.kv_format > 2 || (g.untied_lm_head != 0 && g.untied_lm_head != 1))
        return bad(AARH_ERR_CONFIG, "unknown weight / lm head / kv format");
    if (g.max_rows > 512) return bad(AARH_ERR_UNSUPPORTED, "max_rows must be <= 512");
    c->Fp = (c->F + 127) / 128 * 128;
    c->Mmax = g.max_rows;
    // V^T rows padded so 32-token blocks stay in bounds; PAD_SLACK positions past the
    // context limit take the padding rows of ragged lock-step engine batches
    c->cap = (g.max_seq_len + PAD_SLACK + 31) / 32 * 32;
    *out = c;
    if (hipSetDevice(device) != hipSuccess) return fail(c, AARH_ERR_DEVICE, "hipSetDevice(%d) failed", device);
    HIPCHK(c, hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    HIPCHK(c, hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking));
    HIPCHK(c, hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming));
    HIPCHK(c, hipEventCreateWithFlags(&c->ev_join, hipEventDisableTiming));
    // the statically allocated acceptance scratch of this device (once per device)
    if (accept_static_init(device, c->stream))
        return fail(c, AARH_ERR_DEVICE, "static acceptance scratch set-up failed: %s", last_launch_error());
    c->layers.resize(g.n_layers);
    c->heads.resize(c->nheads_mtp);
    build_slots(c);
    int r;
    // embedding / LM head
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
    for (auto& b : c->layers)
        if ((r = alloc_block(c, b))) return r;
    if (dalloc(c, &c->final_norm, c->H * 4)) return AARH_ERR_DEVICE;
    KCHK(c, launch_fill_f32(c->final_norm, c->H, 1.0f, c->stream));
    for (auto& h : c->heads) {
        if ((r = alloc_block(c, h.blk))) return r;
        if (dalloc(c, &h.trunk, c->H * 4) || dalloc(c, &h.token, c->H * 4) || dalloc(c, &h.out_norm, c->H * 4))
            return AARH_ERR_DEVICE;
        KCHK(c, launch_fill_f32(h.trunk, c->H, 1.0f, c->stream));
        KCHK(c, launch_fill_f32(h.token, c->H, 1.0f, c->stream));
        KCHK(c, launch_fill_f32(h.out_norm, c->H, 1.0f, c->stream));
    }
    // RoPE tables (rope_scaling.rs:6-11, rope.rs:43-72), computed on the host in f32 like the reference.
    {
        const size_t n = (size_t)(g.max_seq_len + PAD_SLACK) * (c->hd / 2);
        if (dalloc(c, &c->rope_cos, n * 4) || dalloc(c, &c->rope_sin, n * 4)) return AARH_ERR_DEVICE;
        if ((r = upload_rope(c, nullptr))) return r;
    }
    // KV cache
    {
        const size_t esz = g.kv_format == AARH_KV_INT8 ? 1 : (g.kv_format == AARH_KV_F16 ? 2 : 4);
        const size_t per = (size_t)g.max_batch * g.n_kv_heads * c->cap * c->hd * esz;
        const size_t sper = (size_t)g.max_batch * g.n_kv_heads * c->cap * 2;
        c->kc.resize(g.n_layers);
        c->vc.resize(g.n_layers);
        c->ksc.assign(g.n_layers, nullptr);
        c->vsc.assign(g.n_layers, nullptr);
        for (int l = 0; l < g.n_layers; l++) {
            if (dalloc(c, (uint8_t**)&c->kc[l], per) || dalloc(c, (uint8_t**)&c->vc[l], per)) return AARH_ERR_DEVICE;
            HIPCHK(c, hipMemset(c->kc[l], 0, per));
            HIPCHK(c, hipMemset(c->vc[l], 0, per));
            if (g.kv_format == AARH_KV_INT8) {
                if (dalloc(c, &c->ksc[l], sper) || dalloc(c, &c->vsc[l], sper)) return AARH_ERR_DEVICE;
                HIPCHK(c, hipMemset(c->ksc[l], 0, sper));
                HIPCHK(c, hipMemset(c->vsc[l], 0, sper));
            }
        }
        c->kv_len.assign(g.max_batch, 0);
        c->mcap = std::max(2, g.num_future_tokens + 1);
        const size_t mper = (size_t)c->Mmax * g.n_kv_heads * c->mcap * c->hd * 4;
        if (dalloc(c, (uint8_t**)&c->mkc, mper) || dalloc(c, (uint8_t**)&c->mvc, mper)) return AARH_ERR_DEVICE;
    }
    // scratch
    {
        const int M = c->Mmax;
        const size_t H = c->H;
        if (dalloc(c, &c->x, M * H * 4) || dalloc(c, &c->q, (size_t)M * c->QD * 4) ||
            dalloc(c, &c->att, (size_t)M * c->QD * 4) || dalloc(c, &c->h, (size_t)M * c->Fp * 4) ||
            dalloc(c, &c->ssq_a, (H / 16) * M * 4) ||
            dalloc(c, &c->hidden, M * H * 4) || dalloc(c, &c->hn, M * H * 4) ||
            dalloc(c, &c->logits, (size_t)M * c->V * 4))
            return AARH_ERR_DEVICE;
        HIPCHK(c, hipMemset(c->h, 0, (size_t)M * c->Fp * 4));
        // new K / V rows of a forward, appended to the cache by the attention kernel
        if (dalloc(c, &c->kvnew, (size_t)M * 2 * c->KD * 4)) return AARH_ERR_DEVICE;
        // activation fragments: row chunks x groups x 16 (t, lg) x 32 entries x 8 halves
        {
            const size_t gmax = (size_t)std::max({c->H, c->QD, c->Fp}) / 128;
            const size_t halves = (size_t)((M + 15) / 16) * gmax * 16 * 32 * 8;
            if (dalloc(c, &c->frag_a, halves * 2) || dalloc(c, &c->frag_b, halves * 2)) return AARH_ERR_DEVICE;
            HIPCHK(c, hipMemset(c->frag_a, 0, halves * 2));
            HIPCHK(c, hipMemset(c->frag_b, 0, halves * 2));
        }
        // attention scratch: groups = nseq*n_kv*ntiles <= n_kv*(M + M*G/16); the chunk count
        // is at most ceil(512/groups) so groups*chunks <= groups + 512.
        const int G = g.n_heads / g.n_kv_heads;
        const size_t groups = (size_t)g.n_kv_heads * ((size_t)M + ((size_t)M * G + 15) / 16);
        c->apart_elems = (groups + 512) * 32 * (c->hd + 4);
        if (dalloc(c, &c->apart, c->apart_elems * 4)) return AARH_ERR_DEVICE;
        if (dalloc(c, &c->acnt, groups * 4)) return AARH_ERR_DEVICE;
        HIPCHK(c, hipMemset(c->acnt, 0, groups * 4));
        if (M > 16) {
            // GEMM split-K partial tiles (64 KiB per block): up to 1024 blocks
            c->gpart_elems = (size_t)16 << 20;
            if (dalloc(c, &c->gpart, c->gpart_elems * 4) || dalloc(c, &c->gcnt, 8192 * 4)) return AARH_ERR_DEVICE;
            HIPCHK(c, hipMemset(c->gcnt, 0, 8192 * 4));
        }
        if (dalloc(c, &c->d_pos0, M * 4) || dalloc(c, &c->d_slot, M * 4) || dalloc(c, &c->d_zero, M * 4) ||
            dalloc(c, &c->d_seqidx, M * 4) || dalloc(c, &c->d_ids, M * 4))
            return AARH_ERR_DEVICE;
        std::vector<int32_t> zero(M, 0), idx(M);
        for (int i = 0; i < M; i++) idx[i] = i;
        HIPCHK(c, hipMemcpy(c->d_zero, zero.data(), M * 4, hipMemcpyHostToDevice));
        HIPCHK(c, hipMemcpy(c->d_seqidx, idx.data(), M * 4, hipMemcpyHostToDevice));
        HIPCHK(c, hipHostMalloc((void**)&c->h_pos0, M * 4, 0));
        HIPCHK(c, hipHostMalloc((void**)&c->h_slot, M * 4, 0));
        HIPCHK(c, hipHostMalloc((void**)&c->h_ids, (size_t)M * 4, 0));
        HIPCHK(c, hipHostMalloc((void**)&c->h_stage, aarh_ctx::STAGE_SLOTS * aarh_ctx::STAGE_BYTES, 0));
        for (auto& ev : c->stage_ev) HIPCHK(c, hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    }
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return AARH_OK;
}

int aarh_num_tensors(const aarh_ctx* c) { return (int)c->slots.size(); }

int aarh_get_config(const aarh_ctx* c, aarh_model_config* out) {
    if (!c || !out) return AARH_ERR_CONFIG;
    *out = c->cfg;
    return AARH_OK;
}

int aarh_tensor_info(const aarh_ctx* c, int id, char* name, int name_cap, int64_t* rows, int64_t* cols,
                     int32_t* kind) {
    if (!c || id < 0 || id >= (int)c->slots.size()) return AARH_ERR_SHAPE;
    const TensorSlot& s = c->slots[id];
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", s.name.c_str());
    if (rows) *rows = s.rows;
    if (cols) *cols = s.cols;
    if (kind) *kind = s.kind;
    return AARH_OK;
}

static int ensure_staging(aarh_ctx* c, size_t elems) {
    if (elems <= c->staging_elems) return 0;
    if (c->staging) {
        HIPCHK(c, hipStreamSynchronize(c->stream));
        (void)hipFree(c->staging);
        c->staging = nullptr;
    }
    if (dalloc(c, &c->staging, elems * 4)) return AARH_ERR_DEVICE;
    c->staging_elems = elems;
    return 0;
}

// Destination tensor, row offset and interleave mode of a linear part.
static void part_target(aarh_ctx* c, const TensorSlot& s, DevTensor** t, int* row_off, int* inter) {
    BlockW* b = s.blk;
    *row_off = 0;
    *inter = 0;
    switch (s.part) {
        case P_WQ: *t = &b->qkv; *inter = c->hd; break;
        case P_WK: *t = &b->qkv; *row_off = c->QD; *inter = c->hd; break;
        case P_WV: *t = &b->qkv; *row_off = c->QD + c->KD; *inter = c->hd; break;
        case P_WO: *t = &b->wo; break;
        case P_GATE: *t = &b->gu; *inter = 1; break;
        case P_UP: *t = &b->gu; *inter = 2; break;
        default: *t = &b->down; break;
    }
}

// Upload one tensor already resident in c->staging (f32, reference shape).
static int place_f32_staging(aarh_ctx* c, int id) {
    const TensorSlot& s = c->slots[id];
    const int64_t n = s.rows * s.cols;
    if (s.part == P_EMBED) {
        // the tied LM head reads the embedding: row-major f32 in place, or its own bf16 tiles
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
    if (s.part == P_LMHEAD) {
        if (c->embed_fmt == WF_F32) {
            HIPCHK(c, hipMemcpyAsync(c->lm.w, c->staging, n * 4, hipMemcpyDeviceToDevice, c->stream));
        } else {
            KCHK(c, launch_quantise_tiled(c->staging, c->V, c->H, WF_BF16, c->lm.w, nullptr, nullptr, 0, c->V, 0,
                                          c->stream));
        }
        return 0;
    }
    if (s.part == P_NORM) {
        HIPCHK(c, hipMemcpyAsync(*s.norm_ptr, c->staging, n * 4, hipMemcpyDeviceToDevice, c->stream));
        return 0;
    }
    DevTensor* t;
    int ro, inter;
    part_target(c, s, &t, &ro, &inter);
    if (s.part == P_DOWN && c->Fp != c->F) {
        // pad K (ffn) to a multiple of 128 with zero columns (f32 weights only);
        // callers reserve n + rows*Fp staging elements
        if ((size_t)n + (size_t)s.rows * c->Fp > c->staging_elems) return fail(c, AARH_ERR_SHAPE, "staging too small");
        float* padded = c->staging + n;
        HIPCHK(c, hipMemsetAsync(padded, 0, (size_t)s.rows * c->Fp * 4, c->stream));
        HIPCHK(c, hipMemcpy2DAsync(padded, (size_t)c->Fp * 4, c->staging, (size_t)c->F * 4, (size_t)c->F * 4,
                                   (size_t)s.rows, hipMemcpyDeviceToDevice, c->stream));
        KCHK(c, launch_quantise_tiled(padded, (int)s.rows, c->Fp, t->fmt, t->w, t->sz, t->rscale, ro, t->N, inter,
                                      c->stream));
        return 0;
    }
    KCHK(c, launch_quantise_tiled(c->staging, (int)s.rows, (int)s.cols, t->fmt, t->w, t->sz, t->rscale, ro, t->N,
                                  inter, c->stream));
    return 0;
}

int aarh_load_tensor_f32(aarh_ctx* c, int id, const float* host, int64_t numel) {
    if (!c || id < 0 || id >= (int)c->slots.size()) return fail(c, AARH_ERR_SHAPE, "bad tensor id %d", id);
    const TensorSlot& s = c->slots[id];
    if (numel != s.rows * s.cols)
        return fail(c, AARH_ERR_SHAPE, "tensor %s expects %lld values, got %lld", s.name.c_str(),
                    (long long)(s.rows * s.cols), (long long)numel);
    // room for the zero-padded copy of a down projection whose ffn width is not a multiple of 128
    const size_t extra = s.part == P_DOWN ? (size_t)s.rows * c->Fp : 0;
    if (ensure_staging(c, (size_t)numel + extra)) return AARH_ERR_DEVICE;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(c->staging, host, numel * 4, hipMemcpyHostToDevice));
    int r = place_f32_staging(c, id);
    if (r) return r;
    return sync_stream(c);
}

int aarh_load_tensor_int4(aarh_ctx* c, int id, const uint8_t* packed, const uint16_t* scales, const uint16_t* zeros,
                          int64_t rows, int64_t cols, int32_t group) {
    if (!c || id < 0 || id >= (int)c->slots.size()) return fail(c, AARH_ERR_SHAPE, "bad tensor id %d", id);
    const TensorSlot& s = c->slots[id];
    if (s.kind != AARH_T_LINEAR || c->cfg.weight_format != AARH_W_INT4_G128)
        return fail(c, AARH_ERR_UNSUPPORTED, "tensor %s is not an INT4 g128 linear in this model", s.name.c_str());
    if (rows != s.rows || cols != s.cols || group != 128 || cols % 128)
        return fail(c, AARH_ERR_SHAPE, "INT4 tensor %s shape/group mismatch", s.name.c_str());
    const size_t ng = (size_t)rows * (cols / 128);
    for (size_t i = 0; i < ng; i++) {
        // zero points must keep (q - z) exact in fp16 on the device path
        uint16_t h = zeros[i];
        int e = (h >> 10) & 31;
        if (e >= 25) return fail(c, AARH_ERR_UNSUPPORTED, "INT4 zero point out of range in %s", s.name.c_str());
    }
    const size_t nb = (size_t)rows * cols / 2;
    if (ensure_staging(c, (nb + 2 * ng * 2 + 3) / 4 + 1)) return AARH_ERR_DEVICE;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    uint8_t* st = (uint8_t*)c->staging;
    HIPCHK(c, hipMemcpy(st, packed, nb, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(st + nb, scales, ng * 2, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(st + nb + ng * 2, zeros, ng * 2, hipMemcpyHostToDevice));
    DevTensor* t;
    int ro, inter;
    part_target(c, s, &t, &ro, &inter);
    KCHK(c, launch_repack_int4(st, (const uint16_t*)(st + nb), (const uint16_t*)(st + nb + ng * 2), (int)rows, (int)cols,
                               t->w, t->sz, ro, t->N, inter, c->stream));
    return sync_stream(c);
}

int aarh_load_tensor_packed_i4(aarh_ctx* c, int id, const int64_t* shape, int32_t ndims, int64_t group_size,
                               const uint8_t* data, int64_t data_len, const float* scales, const float* zeros,
                               int64_t n_groups) {
    if (!c || id < 0 || id >= (int)c->slots.size()) return fail(c, AARH_ERR_SHAPE, "bad tensor id %d", id);
    const TensorSlot& s = c->slots[id];
    if (s.kind != AARH_T_LINEAR || c->cfg.weight_format != AARH_W_INT4_G128)
        return fail(c, AARH_ERR_UNSUPPORTED, "tensor %s is not an INT4 g128 linear in this model", s.name.c_str());
    if (!shape || !data || ndims != 2 || shape[0] != s.rows || shape[1] != s.cols)
        return fail(c, AARH_ERR_SHAPE, "PackedInt4Tensor shape does not match %s [%lld, %lld]", s.name.c_str(),
                    (long long)s.rows, (long long)s.cols);
    const size_t ng = (size_t)s.rows * (s.cols / 128);
    std::vector<uint16_t> sh(ng), zh(ng);
    int r = aarh_packed_i4_params(shape, ndims, group_size, data_len, scales, zeros, n_groups, sh.data(), zh.data());
    if (r) return fail(c, r, "%s: %s", s.name.c_str(), aarh_host_last_error());
    return aarh_load_tensor_int4(c, id, data, sh.data(), zh.data(), s.rows, s.cols, 128);
}

int aarh_load_tensor_int8(aarh_ctx* c, int id, const int8_t* codes, const float* scales, int64_t rows, int64_t cols) {
    if (!c || id < 0 || id >= (int)c->slots.size()) return fail(c, AARH_ERR_SHAPE, "bad tensor id %d", id);
    const TensorSlot& s = c->slots[id];
    if (s.kind != AARH_T_LINEAR || c->cfg.weight_format != AARH_W_INT8_ROW)
        return fail(c, AARH_ERR_UNSUPPORTED, "tensor %s is not an INT8 linear in this model", s.name.c_str());
    if (rows != s.rows || cols != s.cols || cols % 128)
        return fail(c, AARH_ERR_SHAPE, "INT8 tensor %s shape mismatch", s.name.c_str());
    const size_t nb = (size_t)rows * cols;
    if (ensure_staging(c, (nb + rows * 4 + 3) / 4 + 1)) return AARH_ERR_DEVICE;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    uint8_t* st = (uint8_t*)c->staging;
    HIPCHK(c, hipMemcpy(st, codes, nb, hipMemcpyHostToDevice));
    size_t so = (nb + 3) / 4 * 4;
    HIPCHK(c, hipMemcpy(st + so, scales, rows * 4, hipMemcpyHostToDevice));
    DevTensor* t;
    int ro, inter;
    part_target(c, s, &t, &ro, &inter);
    KCHK(c, launch_repack_int8((const int8_t*)st, (const float*)(st + so), (int)rows, (int)cols, t->w, t->rscale, ro,
                               t->N, inter, c->stream));
    return sync_stream(c);
}

int aarh_init_synthetic(aarh_ctx* c, uint64_t seed, float std) {
    if (!c) return AARH_ERR_CONFIG;
    size_t maxn = 0;
    for (auto& s : c->slots) maxn = std::max(maxn, (size_t)(s.rows * s.cols));
    if (ensure_staging(c, maxn + (size_t)c->H * c->Fp + 16)) return AARH_ERR_DEVICE;
    for (int id = 0; id < (int)c->slots.size(); id++) {
        const TensorSlot& s = c->slots[id];
        const int64_t n = s.rows * s.cols;
        if (s.kind == AARH_T_NORM) {
            KCHK(c, launch_fill_f32(c->staging, n, 1.0f, c->stream));
        } else {
            KCHK(c, launch_synth_fill(c->staging, n, seed, (unsigned)id, std, c->stream));
        }
        int r = place_f32_staging(c, id);
        if (r) return r;
    }
    return sync_stream(c);
}

int aarh_kv_reset(aarh_ctx* c, int slot) {
    if (!c || slot < 0 || slot >= c->cfg.max_batch) return fail(c, AARH_ERR_SHAPE, "bad slot %d", slot);
    c->kv_len[slot] = 0;
    return 0;
}

int aarh_kv_len(const aarh_ctx* c, int slot, int32_t* out) {
    if (!c || slot < 0 || slot >= c->cfg.max_batch) return AARH_ERR_SHAPE;
    *out = c->kv_len[slot];
    return 0;
}

int aarh_kv_rollback(aarh_ctx* c, int slot, int32_t new_len) {
    if (!c || slot < 0 || slot >= c->cfg.max_batch) return fail(c, AARH_ERR_SHAPE, "bad slot %d", slot);
    if (new_len < 0 || new_len > c->kv_len[slot])
        return fail(c, AARH_ERR_SHAPE, "cannot grow KV cache from %d to %d with rollback", c->kv_len[slot], new_len);
    c->kv_len[slot] = new_len;
    return 0;
}

int aarh_kv_fill_synthetic(aarh_ctx* c, int slot, int32_t len, uint64_t seed) {
    if (!c || slot < 0 || slot >= c->cfg.max_batch) return fail(c, AARH_ERR_SHAPE, "bad slot %d", slot);
    if (len < 0 || len > c->cfg.max_seq_len)
        return fail(c, AARH_ERR_SHAPE, "length %d exceeds max_seq_len %d", len, c->cfg.max_seq_len);
    for (int l = 0; l < c->cfg.n_layers; l++)
        KCHK(c, launch_kv_fill_synthetic(c->kc[l], c->vc[l], c->ksc[l], c->vsc[l], c->cfg.kv_format, slot,
                                         c->cfg.n_kv_heads, c->hd, c->cap, len, seed, l, c->stream));
    c->kv_len[slot] = len;
    return sync_stream(c);
}

// Validate and stage (slots, offsets, ids) from host arrays; returns max kv length.
// pad: positions allowed past max_seq_len (engine padding rows only, <= PAD_SLACK).
static int stage_rows(aarh_ctx* c, const uint32_t* ids, const int32_t* slots, const int32_t* offsets, int nseq, int S,
                      int* max_kv, int pad = 0) {
    if (nseq <= 0 || S <= 0) return fail(c, AARH_ERR_SHAPE, "batch and sequence length must be non-zero");
    if (nseq * S > c->Mmax) return fail(c, AARH_ERR_SHAPE, "nseq*S=%d exceeds max_rows %d", nseq * S, c->Mmax);
    int mk = 0;
    for (int b = 0; b < nseq; b++) {
        int sl = slots[b], off = offsets[b];
        if (sl < 0 || sl >= c->cfg.max_batch) return fail(c, AARH_ERR_SHAPE, "bad slot %d", sl);
        for (int b2 = 0; b2 < b; b2++)
            if (slots[b2] == sl) return fail(c, AARH_ERR_SHAPE, "slot %d used twice", sl);
        if (off < 0 || off > c->kv_len[sl])
            return fail(c, AARH_ERR_SHAPE, "offset %d beyond cached length %d of slot %d", off, c->kv_len[sl], sl);
        if (off + S > c->cfg.max_seq_len + pad)
            return fail(c, AARH_ERR_SHAPE, "sequence length %d with offset %d exceeds max_seq_len %d", S, off,
                        c->cfg.max_seq_len);
        mk = std::max(mk, off + S);
    }
    for (int i = 0; i < nseq * S; i++)
        if ((int64_t)ids[i] >= c->V) return fail(c, AARH_ERR_SHAPE, "token id %u exceeds vocabulary", ids[i]);
    *max_kv = mk;
    if (((size_t)nseq * S + 2 * (size_t)nseq) * 4 <= aarh_ctx::STAGE_BYTES) {
        int sl = 0;
        char* p = stage_acquire(c, &sl);
        if (!p) return fail(c, AARH_ERR_DEVICE, "staging slot wait failed");
        int32_t* hp = (int32_t*)p;
        int32_t* hs = hp + nseq;
        uint32_t* hi = (uint32_t*)(hs + nseq);
        memcpy(hp, offsets, nseq * 4);
        memcpy(hs, slots, nseq * 4);
        memcpy(hi, ids, (size_t)nseq * S * 4);
        HIPCHK(c, hipMemcpyAsync(c->d_pos0, hp, nseq * 4, hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, hipMemcpyAsync(c->d_slot, hs, nseq * 4, hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, hipMemcpyAsync(c->d_ids, hi, (size_t)nseq * S * 4, hipMemcpyHostToDevice, c->stream));
        return stage_release(c, sl);
    }
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

// stage_rows for rows whose ids a device kernel writes into d_ids: validates the slots
// and offsets and stages positions, slots and nseq extra words (`meta`, to `d_meta`).
static int stage_rows_meta(aarh_ctx* c, const int32_t* slots, const int32_t* offsets, int nseq, int S, int* max_kv,
                           int pad, const int32_t* meta, int32_t* d_meta) {
    if (nseq <= 0 || S <= 0) return fail(c, AARH_ERR_SHAPE, "batch and sequence length must be non-zero");
    if (nseq * S > c->Mmax) return fail(c, AARH_ERR_SHAPE, "nseq*S=%d exceeds max_rows %d", nseq * S, c->Mmax);
    int mk = 0;
    for (int b = 0; b < nseq; b++) {
        int sl = slots[b], off = offsets[b];
        if (sl < 0 || sl >= c->cfg.max_batch) return fail(c, AARH_ERR_SHAPE, "bad slot %d", sl);
        for (int b2 = 0; b2 < b; b2++)
            if (slots[b2] == sl) return fail(c, AARH_ERR_SHAPE, "slot %d used twice", sl);
        if (off < 0 || off > c->kv_len[sl])
            return fail(c, AARH_ERR_SHAPE, "offset %d beyond cached length %d of slot %d", off, c->kv_len[sl], sl);
        if (off + S > c->cfg.max_seq_len + pad)
            return fail(c, AARH_ERR_SHAPE, "sequence length %d with offset %d exceeds max_seq_len %d", S, off,
                        c->cfg.max_seq_len);
        mk = std::max(mk, off + S);
    }
    *max_kv = mk;
    if ((size_t)3 * nseq * 4 > aarh_ctx::STAGE_BYTES) return fail(c, AARH_ERR_SHAPE, "batch %d too large to stage", nseq);
    int sl = 0;
    char* p = stage_acquire(c, &sl);
    if (!p) return fail(c, AARH_ERR_DEVICE, "staging slot wait failed");
    int32_t* hp = (int32_t*)p;
    memcpy(hp, offsets, nseq * 4);
    memcpy(hp + nseq, slots, nseq * 4);
    memcpy(hp + 2 * nseq, meta, nseq * 4);
    HIPCHK(c, hipMemcpyAsync(c->d_pos0, hp, nseq * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_slot, hp + nseq, nseq * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(d_meta, hp + 2 * nseq, nseq * 4, hipMemcpyHostToDevice, c->stream));
    return stage_release(c, sl);
}

// Host array -> device through a staging slot (no wait for the device).
static int stage_copy(aarh_ctx* c, void* dst, const void* src, size_t bytes) {
    int sl = 0;
    char* p = bytes <= aarh_ctx::STAGE_BYTES ? stage_acquire(c, &sl) : nullptr;
    if (!p) {  // too large for a slot: an ordered copy the host waits for
        HIPCHK(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
        return sync_stream(c);
    }
    memcpy(p, src, bytes);
    HIPCHK(c, hipMemcpyAsync(dst, p, bytes, hipMemcpyHostToDevice, c->stream));
    return stage_release(c, sl);
}

int aarh_forward(aarh_ctx* c, const uint32_t* ids, const int32_t* slots, const int32_t* offsets, int nseq, int S,
                 float* logits_out, float* hidden_out) {
    if (!c) return AARH_ERR_CONFIG;
    int mk = 0;
    int r = stage_rows(c, ids, slots, offsets, nseq, S, &mk);
    if (r) return r;
    const int M = nseq * S;
    r = forward_dev(c, c->d_ids, c->d_pos0, c->d_slot, nseq, S, mk, c->logits, rm(M, 0, c->V), c->hidden);
    if (r) return r;
    for (int b = 0; b < nseq; b++) c->kv_len[slots[b]] = offsets[b] + S;
    if (logits_out) HIPCHK(c, hipMemcpyAsync(logits_out, c->logits, (size_t)M * c->V * 4, hipMemcpyDeviceToHost, c->stream));
    if (hidden_out) HIPCHK(c, hipMemcpyAsync(hidden_out, c->hidden, (size_t)M * c->H * 4, hipMemcpyDeviceToHost, c->stream));
    return sync_stream(c);
}

const float* aarh_last_logits_device(const aarh_ctx* c) { return c ? c->logits : nullptr; }
const float* aarh_last_hidden_device(const aarh_ctx* c) { return c ? c->hidden : nullptr; }

int aarh_mtp_head(aarh_ctx* c, int head, const float* anchor, const uint32_t* ids, int nseq, float* logits_out) {
    if (!c) return AARH_ERR_CONFIG;
    if (head < 0 || head >= c->nheads_mtp) return fail(c, AARH_ERR_CONFIG, "MTP head index %d is not configured", head);
    if (nseq <= 0 || nseq * (head + 2) > c->Mmax) return fail(c, AARH_ERR_SHAPE, "bad MTP batch %d", nseq);
    for (int i = 0; i < nseq * (head + 1); i++)
        if ((int64_t)ids[i] >= c->V) return fail(c, AARH_ERR_SHAPE, "token id %u exceeds vocabulary", ids[i]);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(c->hidden, anchor, (size_t)nseq * c->H * 4, hipMemcpyHostToDevice));
    memcpy(c->h_ids, ids, (size_t)nseq * (head + 1) * 4);
    HIPCHK(c, hipMemcpy(c->d_ids, c->h_ids, (size_t)nseq * (head + 1) * 4, hipMemcpyHostToDevice));
    int r = mtp_head_dev(c, head, c->hidden, c->H, c->d_ids, head + 1, nseq, c->logits, c->V);
    if (r) return r;
    if (logits_out) HIPCHK(c, hipMemcpyAsync(logits_out, c->logits, (size_t)nseq * c->V * 4, hipMemcpyDeviceToHost, c->stream));
    return sync_stream(c);
}

static int ensure_accept_scratch(aarh_ctx* c, int B, int rows_per_seq) {
    const int rows = B * rows_per_seq;
    if (rows > c->acc_rows_cap) {
        if (c->acc_rstat) {
            HIPCHK(c, hipStreamSynchronize(c->stream));
            (void)hipFree(c->acc_rstat);
        }
        if (dalloc(c, &c->acc_rstat, (size_t)rows * ACC_RS_WORDS * 4)) return AARH_ERR_DEVICE;
        c->acc_rows_cap = rows;
    }
    if (B > c->acc_seq_cap) {
        if (c->acc_cnt) {
            HIPCHK(c, hipStreamSynchronize(c->stream));
            (void)hipFree(c->acc_cnt);
        }
        if (dalloc(c, &c->acc_cnt, B * 4)) return AARH_ERR_DEVICE;
        HIPCHK(c, hipMemset(c->acc_cnt, 0, B * 4));
        c->acc_seq_cap = B;
    }
    return 0;
}

// Validated argument block of an acceptance launch (scratch pointers left empty).
static int accept_args(aarh_ctx* c, const float* target, int target_rows, const float* draft,
                       const uint32_t* draft_tokens, const int32_t* n_proposals, int B, int K, int V, int bonus,
                       const aarh_sampler* s, const uint64_t* seeds, const uint64_t* word_offsets,
                       const float* uniforms, int32_t* accept_len, int32_t* token, uint32_t* flags, int32_t* draws,
                       int32_t* status, AcceptArgs* a) {
    if (B <= 0 || K < 0 || V <= 0 || target_rows < K + (bonus ? 1 : 0))
        return fail(c, AARH_ERR_SHAPE, "bad acceptance shape B=%d K=%d V=%d rows=%d", B, K, V, target_rows);
    const bool greedy = s->greedy || !(s->temperature > 1.1920929e-07f);
    if (!greedy && !(s->top_p >= 0.0f && s->top_p <= 1.0f))
        return fail(c, AARH_ERR_CONFIG, "top_p must be in [0, 1]");
    *a = AcceptArgs{};
    a->target = target;
    a->target_rows = target_rows;
    a->draft = draft;
    a->draft_tokens = draft_tokens;
    a->n_proposals = n_proposals;
    a->B = B;
    a->K = K;
    a->V = V;
    a->bonus = bonus ? 1 : 0;
    a->greedy = greedy ? 1 : 0;
    a->temperature = s->temperature;
    a->top_k = s->top_k;
    a->top_p = s->top_p;
    a->seeds = seeds;
    a->word_offsets = word_offsets;
    a->uniforms = uniforms;
    a->out_accept_len = accept_len;
    a->out_token = token;
    a->out_flags = flags;
    a->out_draws = draws;
    a->out_status = status;
    return 0;
}

int aarh_accept_sample(aarh_ctx* c, const float* target, int target_rows, const float* draft,
                       const uint32_t* draft_tokens, const int32_t* n_proposals, int B, int K, int V, int bonus,
                       const aarh_sampler* s, const uint64_t* seeds, const uint64_t* word_offsets,
                       const float* uniforms, int32_t* accept_len, int32_t* token, uint32_t* flags, int32_t* draws,
                       int32_t* status, void* stream) {
    if (!c || !s) return AARH_ERR_CONFIG;
    AcceptArgs a;
    int r = accept_args(c, target, target_rows, draft, draft_tokens, n_proposals, B, K, V, bonus, s, seeds,
                        word_offsets, uniforms, accept_len, token, flags, draws, status, &a);
    if (r) return r;
    if (ensure_accept_scratch(c, B, target_rows + K)) return AARH_ERR_DEVICE;
    a.rstat = c->acc_rstat;
    a.counters = c->acc_cnt;
    hipStream_t st = stream ? (hipStream_t)stream : c->stream;
    hipStream_t saved = c->stream;
    c->stream = st;
    {
        ProfScope ps(c, AARH_PROF_ACCEPT, (double)B * (target_rows + K) * V * 4.0);
        r = launch_accept(a, st);
    }
    c->stream = saved;
    if (r) return fail(c, r, "acceptance launch failed: %d %s", r, last_launch_error());
    return 0;
}

// The same acceptance without any allocation: row statistics and arrival counters
// live in the library's statically allocated per-GPU scratch (accept.hip), whose
// device address aarh_create resolved.  Calls that overlap on one GPU share it and race.
int aarh_accept_sample_static(aarh_ctx* c, const float* target, int target_rows, const float* draft,
                              const uint32_t* draft_tokens, const int32_t* n_proposals, int B, int K, int V,
                              int bonus, const aarh_sampler* s, const uint64_t* seeds, const uint64_t* word_offsets,
                              const float* uniforms, int32_t* accept_len, int32_t* token, uint32_t* flags,
                              int32_t* draws, int32_t* status, void* stream) {
    if (!c || !s) return AARH_ERR_CONFIG;
    AcceptArgs a;
    int r = accept_args(c, target, target_rows, draft, draft_tokens, n_proposals, B, K, V, bonus, s, seeds,
                        word_offsets, uniforms, accept_len, token, flags, draws, status, &a);
    if (r) return r;
    if (B > ACC_STATIC_SEQS || (long long)B * (target_rows + K) > ACC_STATIC_ROWS)
        return fail(c, AARH_ERR_SHAPE,
                    "acceptance of %d sequences x %d logits rows exceeds the static scratch (%d sequences, %d rows)",
                    B, target_rows + K, ACC_STATIC_SEQS, ACC_STATIC_ROWS);
    uint32_t* rstat = nullptr;
    unsigned* cnt = nullptr;
    if (accept_static_scratch(c->device, &rstat, &cnt))
        return fail(c, AARH_ERR_DEVICE, "static acceptance scratch is not set up on device %d", c->device);
    a.rstat = rstat;
    a.counters = cnt;
    hipStream_t st = stream ? (hipStream_t)stream : c->stream;
    // this call's arrival counters start at zero whatever the last call left
    r = launch_zero_u32(cnt, B, st);
    if (!r) r = launch_accept(a, st);
    if (r) return fail(c, r, "acceptance launch failed: %d %s", r, last_launch_error());
    return 0;
}

int aarh_top_candidates(aarh_ctx* c, const float* logits, int rows, int V, const aarh_sampler* s, int n,
                        uint32_t* ids, float* probs, void* stream) {
    if (!c || !s || !logits || !ids || !probs) return AARH_ERR_CONFIG;
    if (rows <= 0 || V <= 0 || n < 1 || n > CAND_MAX)
        return fail(c, AARH_ERR_SHAPE, "bad candidate shape rows=%d V=%d n=%d (n <= %d)", rows, V, n, CAND_MAX);
    const bool greedy = s->greedy || !(s->temperature > 1.1920929e-07f);
    CandArgs a{};
    a.logits = logits;
    a.ld = V;
    a.rows = rows;
    a.V = V;
    a.n = n;
    a.greedy = greedy ? 1 : 0;
    a.temperature = s->temperature;
    a.top_k = s->top_k;
    a.top_p = s->top_p;
    a.ids = ids;
    a.probs = probs;
    int r;
    {
        ProfScope ps(c, AARH_PROF_ACCEPT, (double)rows * V * 4.0);
        r = launch_candidates(a, stream ? (hipStream_t)stream : c->stream);
    }
    if (r) return fail(c, r, "candidate launch failed: %d %s", r, last_launch_error());
    return 0;
}

int aarh_set_replay_schedule(aarh_ctx* c, int schedule) {
    if (!c) return AARH_ERR_CONFIG;
    if (schedule != AARH_REPLAY_REPLACEMENT && schedule != AARH_REPLAY_REFERENCE)
        return fail(c, AARH_ERR_CONFIG, "unknown replay schedule %d", schedule);
    c->replay_schedule = schedule;
    return 0;
}

int aarh_set_graphs(aarh_ctx* c, int enable) {
    if (!c) return AARH_ERR_CONFIG;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    c->graphs = enable != 0;
    for (auto& g : c->gcache)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
    c->gcache.clear();
    return 0;
}

int aarh_set_rope_scaling(aarh_ctx* c, const aarh_rope_scaling* s) {
    if (!c) return AARH_ERR_CONFIG;
    return upload_rope(c, s);
}

int aarh_prof_enable(aarh_ctx* c, int enable) {
    if (!c) return AARH_ERR_CONFIG;
    c->prof = enable != 0;
    for (int i = 0; i < AARH_PROF_COUNT; i++) {
        c->prof_ms[i] = 0;
        c->prof_bytes[i] = 0;
        c->prof_n[i] = 0;
    }
    return 0;
}

static int prof_collect(aarh_ctx* c) {
    if (c->prof_recs.empty()) return 0;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    for (auto& r : c->prof_recs) {
        float ms = 0;
        (void)hipEventElapsedTime(&ms, r.a, r.b);
        c->prof_ms[r.cls] += ms;
        c->prof_bytes[r.cls] += r.bytes;
        c->prof_n[r.cls] += 1;
        c->ev_pool.push_back(r.a);
        c->ev_pool.push_back(r.b);
    }
    c->prof_recs.clear();
    return 0;
}

int aarh_prof_get(aarh_ctx* c, int cls, double* total_ms, double* alg_bytes, int64_t* launches) {
    if (!c || cls < 0 || cls >= AARH_PROF_COUNT) return AARH_ERR_CONFIG;
    int r = prof_collect(c);
    if (r) return r;
    if (total_ms) *total_ms = c->prof_ms[cls];
    if (alg_bytes) *alg_bytes = c->prof_bytes[cls];
    if (launches) *launches = c->prof_n[cls];
    return 0;
}

}  // extern "C"

// ===========================================================================
// Engine: MtpSpeculativeEngine::generate_with_callback (mtp_speculative.rs:86-336)
// for nseq independent requests in lock-step rounds.
// ===========================================================================
// ===========================================================================
// Engine: MtpSpeculativeEngine::generate_with_callback (mtp_speculative.rs:86-336)
// for nseq independent requests in lock-step rounds, as a session so callers
// (benchmarks, servers) can run it round by round.
// ===========================================================================
namespace {

constexpr uint32_t EOS_ID = 0;  // tokenizer/src/special.rs:33

}  // namespace

namespace {

// Top candidates of every committed token: Sampler::top_candidates_from_probabilities
// (sampler.rs:188-208) over the target distribution of the token's position
// (mtp_speculative.rs:247-250), engine.rs:70 top_candidates = 5.  Output metadata.
struct CandBuf {
    uint32_t* ids = nullptr;  // device [rows][CAND_MAX] of the current round
    float* probs = nullptr;
    std::vector<uint32_t> hids;
    std::vector<float> hprobs;
    std::vector<std::vector<uint32_t>> out_ids;  // per sequence, CAND_MAX per committed token
    std::vector<std::vector<float>> out_probs;

    int alloc(aarh_ctx* c, int rows, int nseq) {
        if (dalloc(c, &ids, (size_t)rows * CAND_MAX * 4) || dalloc(c, &probs, (size_t)rows * CAND_MAX * 4))
            return AARH_ERR_DEVICE;
        hids.assign((size_t)rows * CAND_MAX, 0);
        hprobs.assign((size_t)rows * CAND_MAX, 0.f);
        out_ids.assign(nseq, {});
        out_probs.assign(nseq, {});
        return 0;
    }
    void release() {
        if (ids) (void)hipFree(ids);
        if (probs) (void)hipFree(probs);
        ids = nullptr;
        probs = nullptr;
    }
    bool pending = false;  // launched on the side stream, not yet joined
    // Sampled rows: on the side stream (after everything queued on the main stream so
    // far), so the kernels the caller queues next on the main stream run beside it;
    // join() makes the main stream wait for it.  Greedy rows (a one-pass argmax, about
    // 10 us) and profiling runs stay on the main stream: the cross-stream waits cost
    // more than the greedy kernel.
    int launch(aarh_ctx* c, const float* rows_base, int rows, int V, const aarh_sampler& s) {
        const bool greedy = s.greedy || !(s.temperature > 1.1920929e-07f);
        if (greedy || c->prof || !c->side)
            return aarh_top_candidates(c, rows_base, rows, V, &s, CAND_MAX, ids, probs, nullptr);
        HIPCHK(c, hipEventRecord(c->ev_fork, c->stream));
        HIPCHK(c, hipStreamWaitEvent(c->side, c->ev_fork, 0));
        int r = aarh_top_candidates(c, rows_base, rows, V, &s, CAND_MAX, ids, probs, c->side);
        if (r) return r;
        HIPCHK(c, hipEventRecord(c->ev_join, c->side));
        pending = true;
        return 0;
    }
    int join(aarh_ctx* c) {
        if (!pending) return 0;
        pending = false;
        HIPCHK(c, hipStreamWaitEvent(c->stream, c->ev_join, 0));
        return 0;
    }
    // after the stream has synchronised
    int fetch(aarh_ctx* c, int rows) {
        HIPCHK(c, hipMemcpy(hids.data(), ids, (size_t)rows * CAND_MAX * 4, hipMemcpyDeviceToHost));
        HIPCHK(c, hipMemcpy(hprobs.data(), probs, (size_t)rows * CAND_MAX * 4, hipMemcpyDeviceToHost));
        return 0;
    }
    void commit(int b, int row) {
        out_ids[b].insert(out_ids[b].end(), hids.begin() + (size_t)row * CAND_MAX,
                          hids.begin() + (size_t)(row + 1) * CAND_MAX);
        out_probs[b].insert(out_probs[b].end(), hprobs.begin() + (size_t)row * CAND_MAX,
                            hprobs.begin() + (size_t)(row + 1) * CAND_MAX);
    }
    void copy_out(int nseq, int cap, uint32_t* oi, float* op) const {
        for (int b = 0; b < nseq; b++) {
            const size_t n = std::min(out_ids[b].size(), (size_t)cap * CAND_MAX);
            for (size_t i = 0; i < n; i++) {
                if (oi) oi[(size_t)b * cap * CAND_MAX + i] = out_ids[b][i];
                if (op) op[(size_t)b * cap * CAND_MAX + i] = out_probs[b][i];
            }
        }
    }
};

}  // namespace

struct aarh_session {
    aarh_ctx* c = nullptr;
    int nseq = 0, K = 0;  // nseq: rows (request capacity)
    bool greedy = true;
    aarh_sampler samp{};
    // device
    float *tgt = nullptr, *drf = nullptr, *anchor = nullptr, *vhid = nullptr;
    // acceptance results, proposals, the proposal limits and the sampled-proposal flags
    // share one allocation (`pack`, int32 words: len, tok, draws, status [nseq each],
    // props [nseq * K], limit [nseq], pstat [nseq]) so that one read-back returns
    // everything a round's host step needs
    int32_t* pack = nullptr;
    uint32_t* props = nullptr;
    int32_t *acc_len = nullptr, *acc_tok = nullptr, *acc_draws = nullptr, *acc_status = nullptr, *nprop = nullptr;
    int32_t* limit = nullptr;
    int32_t* pstat = nullptr;  // sampled proposals: invalid-distribution flags (in pack)
    uint32_t* acc_flags = nullptr;
    uint64_t *seeds = nullptr, *offs = nullptr;
    uint64_t* offs_k = nullptr;  // sampled proposals: keystream word of head p for row b at [p][nseq]
    const float** src = nullptr;
    float** dst = nullptr;
    // host state, per row: `live` = the row holds a request (admitted and not retired);
    // `finished` = it takes no further rounds (done, or a free row)
    std::vector<uint64_t> hoffs;
    std::vector<char> live, finished;
    std::vector<int> max_new, available;
    std::vector<std::vector<uint32_t>> out;
    std::vector<int32_t> finish;
    std::vector<aarh_spec_stats> stats;
    std::vector<uint32_t> hprops;
    std::vector<int32_t> slots, base, count, hnp, hlen, htok, hdraws, hstatus;
    CandBuf cand;

    ~aarh_session() {
        cand.release();
        for (void* p : {(void*)tgt, (void*)drf, (void*)anchor, (void*)vhid, (void*)pack, (void*)nprop,
                        (void*)acc_flags, (void*)seeds, (void*)offs, (void*)offs_k, (void*)src, (void*)dst})
            if (p) (void)hipFree(p);
    }
};

namespace {

// Copies row s[i] (n floats) to d[i] on the stream; the pointer lists travel through a
// pinned staging slot, so nothing waits for the device.
int copy_rows_staged(aarh_ctx* c, const float** dsrc, float** ddst, const std::vector<const float*>& s,
                     const std::vector<float*>& d, int n) {
    if (s.empty()) return 0;
    const int rows = (int)s.size();
    const size_t bytes = (size_t)rows * sizeof(void*);
    int sl = 0;
    char* p = 2 * bytes <= aarh_ctx::STAGE_BYTES ? stage_acquire(c, &sl) : nullptr;
    if (!p) {
        HIPCHK(c, hipMemcpyAsync(dsrc, s.data(), bytes, hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, hipMemcpyAsync(ddst, d.data(), bytes, hipMemcpyHostToDevice, c->stream));
        KCHK(c, launch_copy_rows(dsrc, ddst, rows, n, c->stream));
        // the host vectors must outlive the async copies
        return sync_stream(c);
    }
    memcpy(p, s.data(), bytes);
    memcpy(p + bytes, d.data(), bytes);
    HIPCHK(c, hipMemcpyAsync(dsrc, p, bytes, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(ddst, p + bytes, bytes, hipMemcpyHostToDevice, c->stream));
    int r = stage_release(c, sl);
    if (r) return r;
    KCHK(c, launch_copy_rows(dsrc, ddst, rows, n, c->stream));
    return 0;
}

int copy_rows_host_lists(aarh_session* e, const std::vector<const float*>& s, const std::vector<float*>& d, int n) {
    return copy_rows_staged(e->c, e->src, e->dst, s, d, n);
}

// Rows a round runs over: 0 .. the last unfinished row.  Finished and free rows below
// it ride along as padding; rows above it take no work.
int session_rows(const aarh_session* e) {
    int n = 0;
    for (int b = 0; b < e->nseq; b++)
        if (!e->finished[b]) n = b + 1;
    return n;
}

// One round of mtp_speculative.rs:161-322 for every unfinished sequence.
int session_round(aarh_session* e) {
    aarh_ctx* c = e->c;
    const int nseq = session_rows(e), K = e->K, V = c->V, H = c->H;
    const int cap = e->nseq;  // row stride of the packed acceptance results
    int r;
    int Kr = 1;
    for (int b = 0; b < nseq; b++) {
        e->base[b] = c->kv_len[b];
        e->count[b] = e->finished[b] ? 1 : std::min(K, e->max_new[b] - (int)e->out[b].size());
        Kr = std::max(Kr, e->count[b]);
    }
    // ---- proposals: index 0 from target_next, index p from MTP head p-1 ----
    {
        std::vector<const float*> s(nseq);
        std::vector<float*> d(nseq);
        for (int b = 0; b < nseq; b++) {
            s[b] = e->tgt + (size_t)b * (K + 1) * V;
            d[b] = e->drf + (size_t)b * K * V;
        }
        if ((r = copy_rows_host_lists(e, s, d, V))) return r;
    }
    // proposals counted this round (0 for finished rows); sampled rounds draw proposal p
    // of row b at keystream word hoffs[b] + p
    std::vector<int32_t> lim(nseq);
    for (int b = 0; b < nseq; b++) lim[b] = e->finished[b] ? 0 : e->count[b];
    if (!e->greedy) {
        std::vector<uint64_t> o((size_t)Kr * nseq);
        for (int p = 0; p < Kr; p++)
            for (int b = 0; b < nseq; b++) o[(size_t)p * nseq + b] = e->hoffs[b] + p;
        if ((r = stage_copy(c, e->offs_k, o.data(), o.size() * 8)) || (r = stage_copy(c, e->limit, lim.data(), nseq * 4)))
            return r;
    }
    for (int p = 0; p < Kr; p++) {
        if (p > 0) {
            if ((r = mtp_head_dev(c, p - 1, e->anchor, H, e->props, K, nseq, e->drf + (size_t)p * V, (long long)K * V)))
                return r;
        }
        if (e->greedy) {
            KCHK(c, launch_argmax_rows(e->drf + (size_t)p * V, (long long)K * V, nseq, V, (int32_t*)e->props + p, K,
                                       nullptr, c->stream));
        } else {
            // sample_probabilities on the proposal distribution (sampler.rs:142-152), on the
            // device; its validation (:314-335) is read back with the acceptance results
            if ((r = aarh_accept_sample(c, e->drf + (size_t)p * V, K, nullptr, nullptr, nullptr, nseq, 0, V, 1, &e->samp,
                                        e->seeds, e->offs_k + (size_t)p * nseq, nullptr, e->acc_len, e->acc_tok,
                                        e->acc_flags, e->acc_draws, e->acc_status, nullptr)))
                return r;
            KCHK(c, launch_sampled_props(e->acc_tok, e->acc_status, e->props, K, p, nseq, e->limit, EOS_ID, e->pstat,
                                         c->stream));
        }
    }
    // Proposal counts (the EOS cut) and their statistics, from the host copy of the proposals.
    auto count_proposals = [&]() {
        for (int b = 0; b < nseq; b++) {
            int np = 0;
            if (!e->finished[b]) {
                for (int p = 0; p < e->count[b]; p++) {
                    np++;
                    e->stats[b].draft_tokens_proposed++;
                    if (e->hprops[(size_t)b * K + p] == EOS_ID) break;
                }
            }
            e->hnp[b] = np;
            // heads ran in lock-step for every row; the reference stops proposing after an EOS
            // proposal (mtp_speculative.rs:196-198), so only heads 0 .. np-2 count
            if (np > 1) e->stats[b].mtp_head_forwards += np - 1;
            if (!e->greedy) e->hoffs[b] += np;
        }
    };
    // Proposals stay on the device: a kernel writes the verify rows, the counts and (sampled)
    // the acceptance's keystream offsets, and the host reads the proposals back with the
    // acceptance results (one wait per round).
    // ---- verify forward ----
    // Finished sequences ride along with padding rows written just past their committed
    // length (inside the PAD_SLACK positions every slot has beyond max_seq_len); their
    // kv_len stays, so the slot's cache remains valid for a cached_len follow-up.
    {
        // (a free row's padding goes to position 0 of its slot, so its attention is short)
        std::vector<int32_t> off(nseq);
        for (int b = 0; b < nseq; b++) off[b] = e->live[b] ? e->base[b] : 0;
        int mk = 0;
        if ((r = stage_rows_meta(c, e->slots.data(), off.data(), nseq, Kr, &mk, PAD_SLACK, lim.data(), e->limit)))
            return r;
        KCHK(c, launch_mtp_verify_rows(e->props, K, Kr, nseq, e->limit, EOS_ID, c->d_ids, e->nprop,
                                       e->greedy ? nullptr : e->offs_k, e->greedy ? nullptr : e->offs, c->stream));
        if ((r = forward_dev(c, c->d_ids, c->d_pos0, c->d_slot, nseq, Kr, mk, e->tgt + V, rm(Kr, (long long)(K + 1) * V, V),
                             e->vhid)))
            return r;
        for (int b = 0; b < nseq; b++) {
            if (e->finished[b]) continue;
            e->stats[b].rounds++;
            e->stats[b].target_decode_forwards++;
        }
    }
    // ---- acceptance (MTP round: no bonus) ----
    {
        // the top candidates (output metadata) run beside the acceptance kernel
        if ((r = e->cand.launch(c, e->tgt, nseq * (K + 1), V, e->samp))) return r;
        r = aarh_accept_sample(c, e->tgt, K + 1, e->drf, e->props, e->nprop, nseq, K, V, 0, &e->samp, e->seeds,
                               e->offs, nullptr, e->acc_len, e->acc_tok, e->acc_flags, e->acc_draws, e->acc_status,
                               nullptr);
        // join the side stream on every path: its kernel reads tgt, which later work rewrites
        const int rj = e->cand.join(c);
        if (r || (r = rj) || (r = sync_stream(c))) return r;
        if ((r = e->cand.fetch(c, nseq * (K + 1)))) return r;
        // one read-back: lengths, tokens, draws, status, the proposals, the limits and the
        // sampled-proposal flags (sections `cap` rows apart)
        std::vector<int32_t> hp((size_t)cap * (6 + K));
        HIPCHK(c, hipMemcpy(hp.data(), e->pack, hp.size() * 4, hipMemcpyDeviceToHost));
        for (int b = 0; b < nseq; b++) {
            e->hlen[b] = hp[b];
            e->htok[b] = hp[cap + b];
            e->hdraws[b] = hp[2 * cap + b];
            e->hstatus[b] = hp[3 * cap + b];
        }
        // sample_probabilities validates the proposal distribution (sampler.rs:142-152, 314-335):
        // the reference fails at the proposal, before this round's verify.  The flags arrive with
        // the acceptance read-back, so the round's verify is undone first: every sequence is
        // left as the proposal step found it (cache length, statistics, keystream position).
        bool invalid = false;
        for (int b = 0; b < nseq; b++)
            invalid = invalid || (!e->greedy && !e->finished[b] && hp[(size_t)(5 + K) * cap + b] != 0);
        if (invalid) {
            for (int b = 0; b < nseq; b++) {
                if (e->finished[b]) continue;
                c->kv_len[b] = e->base[b];
                e->stats[b].rounds--;
                e->stats[b].target_decode_forwards--;
            }
            return fail(c, AARH_ERR_CONFIG, "proposal distribution is invalid (zero mass or does not sum to one)");
        }
        memcpy(e->hprops.data(), hp.data() + 4 * cap, (size_t)nseq * K * 4);
        count_proposals();
    }
    // ---- commit, rollback, replay ----
    std::vector<int> replay_seq, replay_len;
    std::vector<const float*> ls, hs;
    std::vector<float*> ld, hdv;
    for (int b = 0; b < nseq; b++) {
        if (e->finished[b]) continue;
        if (e->hstatus[b] != 0)
            return fail(c, AARH_ERR_CONFIG, "speculative residual distribution has zero probability mass");
        if (!e->greedy) e->hoffs[b] += e->hdraws[b];
        const int np = e->hnp[b], acc = e->hlen[b];
        bool done = false;
        for (int i = 0; i < acc && !done; i++) {
            e->stats[b].draft_tokens_accepted++;
            const uint32_t t = e->hprops[(size_t)b * K + i];
            if (t == EOS_ID) {
                e->finish[b] = AARH_FINISH_EOS;
                done = true;
                break;
            }
            e->out[b].push_back(t);
            e->cand.commit(b, b * (K + 1) + i);
            if ((int)e->out[b].size() == e->max_new[b]) done = true;
        }
        if (done) {
            e->finished[b] = 1;
            c->kv_len[b] = e->base[b] + np;
            continue;
        }
        if (acc < np) {
            // target_cache.restore(snapshot) + forward(proposals[..acc] + replacement): the verify
            // forward already holds the accepted prefix's K / V (same tokens, same positions, same
            // prefix), so the cache keeps them and only the replacement is forwarded
            const uint32_t repl = (uint32_t)e->htok[b];
            c->kv_len[b] = e->base[b] + acc;
            if (repl == EOS_ID) {
                e->finish[b] = AARH_FINISH_EOS;
                e->finished[b] = 1;
                c->kv_len[b] = e->base[b];
                continue;
            }
            e->out[b].push_back(repl);
            e->cand.commit(b, b * (K + 1) + acc);
            replay_seq.push_back(b);
            replay_len.push_back(acc);  // position of the replacement relative to base
            e->hprops[(size_t)b * K + acc] = repl;
        } else {
            // everything accepted: target_next / anchor from the last verify row
            c->kv_len[b] = e->base[b] + np;
            ls.push_back(e->tgt + ((size_t)b * (K + 1) + np) * V);
            ld.push_back(e->tgt + (size_t)b * (K + 1) * V);
            hs.push_back(e->vhid + ((size_t)b * Kr + np - 1) * H);
            hdv.push_back(e->anchor + (size_t)b * H);
        }
    }
    // rows that come from the verify buffers must be copied before the replay reuses scratch
    if ((r = copy_rows_host_lists(e, ls, ld, V)) || (r = copy_rows_host_lists(e, hs, hdv, H))) return r;
    if (!replay_seq.empty()) {
        // replacement schedule: one row per rejected sequence, the replacement at base + acc;
        // reference schedule: proposals[..acc] + replacement from base (rows padded to the
        // longest by repeating the replacement past it; kv_len excludes the padding)
        const int nr = (int)replay_seq.size();
        const bool full = c->replay_schedule == AARH_REPLAY_REFERENCE;
        int S = 1;
        if (full)
            for (int j = 0; j < nr; j++) S = std::max(S, replay_len[j] + 1);
        std::vector<uint32_t> ids((size_t)nr * S);
        std::vector<int32_t> sl(nr), off(nr), last(nr);
        for (int j = 0; j < nr; j++) {
            const int b = replay_seq[j], acc = replay_len[j];
            sl[j] = b;
            if (full) {
                off[j] = e->base[b];
                last[j] = j * S + acc;
                for (int s2 = 0; s2 < S; s2++) ids[(size_t)j * S + s2] = e->hprops[(size_t)b * K + std::min(s2, acc)];
            } else {
                off[j] = e->base[b] + acc;
                last[j] = j;
                ids[j] = e->hprops[(size_t)b * K + acc];
            }
        }
        int mk = 0;
        if ((r = stage_rows(c, ids.data(), sl.data(), off.data(), nr, S, &mk, PAD_SLACK))) return r;
        if ((r = forward_dev(c, c->d_ids, c->d_pos0, c->d_slot, nr, S, mk, c->logits, rm(S, (long long)S * V, V),
                             c->hidden)))
            return r;
        std::vector<const float*> rs, rhs;
        std::vector<float*> rd, rhd;
        for (int j = 0; j < nr; j++) {
            const int b = replay_seq[j];
            e->stats[b].target_decode_forwards++;
            c->kv_len[b] = e->base[b] + replay_len[j] + 1;
            rs.push_back(c->logits + (size_t)last[j] * V);
            rd.push_back(e->tgt + (size_t)b * (K + 1) * V);
            rhs.push_back(c->hidden + (size_t)last[j] * H);
            rhd.push_back(e->anchor + (size_t)b * H);
        }
        if ((r = copy_rows_host_lists(e, rs, rd, V)) || (r = copy_rows_host_lists(e, rhs, rhd, H))) return r;
    }
    for (int b = 0; b < nseq; b++)
        if (!e->finished[b] && (int)e->out[b].size() >= e->max_new[b]) e->finished[b] = 1;
    return 0;
}

// A session of nseq rows, every row free (finished, holding no request): the checks of
// MtpSpeculativeEngine::new (mtp_speculative.rs:40-71) and the device buffers.
int session_create(aarh_ctx* c, int nseq, int num_draft_tokens, const aarh_sampler* s, aarh_session** out) {
    const auto& g = c->cfg;
    if (c->nheads_mtp == 0) return fail(c, AARH_ERR_CONFIG, "internal speculative decoding requires model.mtp configuration");
    if (num_draft_tokens < 2) return fail(c, AARH_ERR_CONFIG, "MTP speculative decoding requires at least two proposal tokens");
    if (num_draft_tokens > g.num_future_tokens)
        return fail(c, AARH_ERR_CONFIG, "requested %d MTP proposal tokens but checkpoint horizon is %d", num_draft_tokens,
                    g.num_future_tokens);
    if (num_draft_tokens >= PAD_SLACK)
        return fail(c, AARH_ERR_UNSUPPORTED, "num_draft_tokens must be below %d on the device path", PAD_SLACK);
    if (nseq <= 0 || nseq > g.max_batch) return fail(c, AARH_ERR_SHAPE, "nseq %d exceeds max_batch", nseq);
    const int K = num_draft_tokens, V = c->V, H = c->H;
    if (nseq * K > c->Mmax) return fail(c, AARH_ERR_SHAPE, "nseq x draft tokens exceeds max_rows");
    aarh_session* e = new aarh_session();
    e->c = c;
    e->nseq = nseq;
    e->K = K;
    e->greedy = s->greedy || !(s->temperature > 1.1920929e-07f);
    e->samp = *s;
    e->hoffs.assign(nseq, 0);
    e->live.assign(nseq, 0);
    e->finished.assign(nseq, 1);
    e->max_new.assign(nseq, 0);
    e->available.assign(nseq, 0);
    e->out.assign(nseq, {});
    e->finish.assign(nseq, AARH_FINISH_MAX_TOKENS);
    e->stats.assign(nseq, aarh_spec_stats{});
    e->hprops.assign((size_t)nseq * K, 0);
    for (auto* v : {&e->slots, &e->base, &e->count, &e->hnp, &e->hlen, &e->htok, &e->hdraws, &e->hstatus}) v->assign(nseq, 0);
    for (int b = 0; b < nseq; b++) e->slots[b] = b;
    int r = 0;
#define SA(p, bytes) \
    if ((r = dalloc(c, &e->p, (bytes)))) { delete e; return r; }
    SA(tgt, (size_t)nseq * (K + 1) * V * 4);
    SA(drf, (size_t)nseq * K * V * 4);
    SA(anchor, (size_t)nseq * H * 4);
    SA(vhid, (size_t)nseq * K * H * 4);
    SA(pack, ((size_t)nseq * (6 + K)) * 4);
    e->acc_len = e->pack;
    e->acc_tok = e->pack + nseq;
    e->acc_draws = e->pack + 2 * nseq;
    e->acc_status = e->pack + 3 * nseq;
    e->props = (uint32_t*)(e->pack + 4 * nseq);
    e->limit = e->pack + (size_t)nseq * (4 + K);
    e->pstat = e->pack + (size_t)nseq * (5 + K);
    SA(nprop, nseq * 4);
    SA(acc_flags, nseq * 4);
    SA(seeds, nseq * 8);
    SA(offs, nseq * 8);
    SA(offs_k, (size_t)K * nseq * 8);
    SA(src, (size_t)2 * g.max_batch * sizeof(void*));
    SA(dst, (size_t)2 * g.max_batch * sizeof(void*));
#undef SA
    if ((r = e->cand.alloc(c, nseq * (K + 1), nseq))) {
        delete e;
        return r;
    }
    *out = e;
    return 0;
}

// Row b takes a new request of `full` context tokens (cached + prompt): fresh output,
// statistics, candidates and keystream, and the token budget min(max_new_tokens,
// available) of prepare_session (engine.rs:288-297); a zero budget finishes at once
// with ContextLimit (GenerationSession::new, engine.rs:771).  Returns the budget.
int session_row_reset(aarh_session* e, int b, int full, int max_new_tokens) {
    e->live[b] = 1;
    e->available[b] = e->c->cfg.max_seq_len - full;
    e->max_new[b] = std::min(max_new_tokens, e->available[b]);
    e->finished[b] = e->max_new[b] <= 0;
    e->finish[b] = e->max_new[b] <= 0 ? AARH_FINISH_CONTEXT_LIMIT : AARH_FINISH_MAX_TOKENS;
    e->out[b].clear();
    e->stats[b] = aarh_spec_stats{};
    e->hoffs[b] = 0;
    e->cand.out_ids[b].clear();
    e->cand.out_probs[b].clear();
    return e->max_new[b];
}

// Prefill of rows[i]'s prompt tail (S0 tokens each, [n][S0]) from position `from`, in
// forwards of at most `chunk` tokens per row (prepare_session_with_chunk_size,
// engine.rs:300-307); the last row's logits and hidden state seed the first round.
int session_prefill(aarh_session* e, const int32_t* rows, int n, const uint32_t* prompts, int S0, int from, int chunk) {
    aarh_ctx* c = e->c;
    const int K = e->K, V = c->V, H = c->H;
    chunk = std::max(1, std::min(chunk, c->Mmax / n));
    std::vector<uint32_t> ids;
    std::vector<int32_t> offs(n);
    int r;
    for (int i = 0; i < n; i++) c->kv_len[rows[i]] = from;
    for (int p0 = 0; p0 < S0; p0 += chunk) {
        const int S = std::min(chunk, S0 - p0);
        ids.resize((size_t)n * S);
        for (int i = 0; i < n; i++) {
            offs[i] = from + p0;
            for (int s2 = 0; s2 < S; s2++) ids[(size_t)i * S + s2] = prompts[(size_t)i * S0 + p0 + s2];
        }
        int mk = 0;
        if ((r = stage_rows(c, ids.data(), rows, offs.data(), n, S, &mk)) ||
            (r = forward_dev(c, c->d_ids, c->d_pos0, c->d_slot, n, S, mk, c->logits, rm(n * S, 0, V), c->hidden)))
            return r;
        for (int i = 0; i < n; i++) c->kv_len[rows[i]] = from + p0 + S;
        if (p0 + S == S0) {
            std::vector<const float*> ls(n), hsrc(n);
            std::vector<float*> ld(n), hd(n);
            for (int i = 0; i < n; i++) {
                ls[i] = c->logits + ((size_t)i * S + S - 1) * V;
                ld[i] = e->tgt + (size_t)rows[i] * (K + 1) * V;
                hsrc[i] = c->hidden + ((size_t)i * S + S - 1) * H;
                hd[i] = e->anchor + (size_t)rows[i] * H;
            }
            if ((r = copy_rows_host_lists(e, ls, ld, V)) || (r = copy_rows_host_lists(e, hsrc, hd, H))) return r;
        }
    }
    return 0;
}

}  // namespace

extern "C" {

int aarh_session_begin(aarh_ctx* c, const uint32_t* prompts, int nseq, int prompt_len, int cached_len,
                       int max_new_tokens, int num_draft_tokens, const aarh_sampler* s, const uint64_t* seeds,
                       aarh_session** out) {
    if (!c || !s || !out) return AARH_ERR_CONFIG;
    *out = nullptr;
    const auto& g = c->cfg;
    if (nseq <= 0 || nseq > g.max_batch) return fail(c, AARH_ERR_SHAPE, "nseq %d exceeds max_batch", nseq);
    if (prompt_len <= 0) return fail(c, AARH_ERR_SHAPE, "prompt must be non-empty");
    if (cached_len < 0) return fail(c, AARH_ERR_SHAPE, "negative cached length");
    for (int b = 0; b < nseq; b++)
        if (c->kv_len[b] < cached_len)
            return fail(c, AARH_ERR_SHAPE, "slot %d holds %d cached tokens, fewer than %d", b, c->kv_len[b], cached_len);
    const int full = cached_len + prompt_len;
    if (full >= g.max_seq_len)
        return fail(c, AARH_ERR_SHAPE, "prompt has %d tokens but model context limit is %d", full, g.max_seq_len);
    aarh_session* e = nullptr;
    int r = session_create(c, nseq, num_draft_tokens, s, &e);
    if (r) return r;
    std::vector<uint64_t> hs(nseq);
    for (int b = 0; b < nseq; b++) hs[b] = seeds ? seeds[b] : 0;
    if (hipMemcpy(e->seeds, hs.data(), nseq * 8, hipMemcpyHostToDevice) != hipSuccess) {
        delete e;
        return fail(c, AARH_ERR_DEVICE, "seed upload failed");
    }
    int budget = 0;
    for (int b = 0; b < nseq; b++) budget = session_row_reset(e, b, full, max_new_tokens);
    if (budget > 0) {
        // ---- prefill of the uncached prompt tail, chunked so rows stay within max_rows ----
        if ((r = session_prefill(e, e->slots.data(), nseq, prompts, prompt_len, cached_len, c->Mmax))) {
            delete e;
            return r;
        }
    }
    *out = e;
    return 0;
}

int aarh_session_open(aarh_ctx* c, int capacity, int num_draft_tokens, const aarh_sampler* s, aarh_session** out) {
    if (!c || !s || !out) return AARH_ERR_CONFIG;
    *out = nullptr;
    return session_create(c, capacity, num_draft_tokens, s, out);
}

int aarh_session_admit(aarh_session* e, int row, const uint32_t* prompt, int prompt_len, int max_new_tokens,
                       uint64_t seed, int prefill_chunk) {
    if (!e) return AARH_ERR_CONFIG;
    aarh_ctx* c = e->c;
    if (prefill_chunk <= 0) return fail(c, AARH_ERR_CONFIG, "prefill chunk size must be greater than zero");
    if (row < 0 || row >= e->nseq) return fail(c, AARH_ERR_SHAPE, "row %d outside the session's %d rows", row, e->nseq);
    if (e->live[row]) return fail(c, AARH_ERR_CONFIG, "row %d holds a request that has not been retired", row);
    if (prompt_len <= 0) return fail(c, AARH_ERR_SHAPE, "prompt must be non-empty");
    if (!prompt) return fail(c, AARH_ERR_CONFIG, "null prompt");
    if (max_new_tokens < 0) return fail(c, AARH_ERR_SHAPE, "negative max_new_tokens");
    const int msl = c->cfg.max_seq_len;
    if (prompt_len >= msl) return fail(c, AARH_ERR_SHAPE, "prompt has %d tokens but model max_seq_len is %d", prompt_len, msl);
    int r = stage_copy(c, e->seeds + row, &seed, 8);
    if (r) return r;
    if (session_row_reset(e, row, prompt_len, max_new_tokens) <= 0) {
        c->kv_len[row] = 0;
        return 0;
    }
    const int32_t rows[1] = {row};
    if ((r = session_prefill(e, rows, 1, prompt, prompt_len, 0, prefill_chunk))) {
        // the row stays free: the request failed before it joined (admit_job, batching.rs:471-482)
        e->live[row] = 0;
        e->finished[row] = 1;
        c->kv_len[row] = 0;
        return r;
    }
    return 0;
}

int aarh_session_retire(aarh_session* e, int row) {
    if (!e) return AARH_ERR_CONFIG;
    if (row < 0 || row >= e->nseq) return fail(e->c, AARH_ERR_SHAPE, "row %d outside the session's %d rows", row, e->nseq);
    // the request leaves (completed or cancelled, batching.rs:363-367, 405-432): its row and
    // KV slot are free; a free row rides along in later rounds as padding at position 0
    e->live[row] = 0;
    e->finished[row] = 1;
    e->finish[row] = AARH_FINISH_MAX_TOKENS;
    e->max_new[row] = e->available[row] = 0;
    e->out[row].clear();
    e->stats[row] = aarh_spec_stats{};
    e->cand.out_ids[row].clear();
    e->cand.out_probs[row].clear();
    e->c->kv_len[row] = 0;
    return 0;
}

int aarh_session_rows(aarh_session* e, int32_t* state) {
    if (!e || !state) return AARH_ERR_CONFIG;
    for (int b = 0; b < e->nseq; b++) state[b] = !e->live[b] ? 0 : !e->finished[b] ? 1 : 2;
    return 0;
}

int aarh_session_step(aarh_session* e, int max_rounds, int32_t* all_done) {
    if (!e) return AARH_ERR_CONFIG;
    for (int i = 0; i < max_rounds; i++) {
        bool any = false;
        for (int b = 0; b < e->nseq; b++)
            if (!e->finished[b]) any = true;
        if (!any) break;
        int r = session_round(e);
        if (r) return r;
    }
    if (all_done) {
        *all_done = 1;
        for (int b = 0; b < e->nseq; b++)
            if (!e->finished[b]) *all_done = 0;
    }
    return 0;
}

int aarh_session_result(aarh_session* e, uint32_t* out_tokens, int32_t out_cap, int32_t* out_len, int32_t* finish_reason,
                        aarh_spec_stats* stats) {
    if (!e) return AARH_ERR_CONFIG;
    for (int b = 0; b < e->nseq; b++) {
        const int n = (int)e->out[b].size();
        if (out_len) out_len[b] = n;
        if (out_tokens)
            for (int i = 0; i < n && i < out_cap; i++) out_tokens[(size_t)b * out_cap + i] = e->out[b][i];
        int fin = e->finish[b];
        if (e->live[b] && n == e->available[b] && fin == AARH_FINISH_MAX_TOKENS) fin = AARH_FINISH_CONTEXT_LIMIT;
        if (finish_reason) finish_reason[b] = fin;
        if (stats) {
            stats[b] = e->stats[b];
            stats[b].draft_tokens_rejected =
                std::max(0, stats[b].draft_tokens_proposed - stats[b].draft_tokens_accepted);
        }
    }
    return 0;
}

int aarh_session_candidates(aarh_session* e, uint32_t* ids, float* probs, int32_t cap) {
    if (!e || cap < 0) return AARH_ERR_CONFIG;
    e->cand.copy_out(e->nseq, cap, ids, probs);
    return 0;
}

int aarh_session_rng_offsets(aarh_session* e, uint64_t* out) {
    if (!e || !out) return AARH_ERR_CONFIG;
    for (int b = 0; b < e->nseq; b++) out[b] = e->hoffs[b];
    return 0;
}

int aarh_session_set_rng_offsets(aarh_session* e, const uint64_t* offsets) {
    if (!e || !offsets) return AARH_ERR_CONFIG;
    for (int b = 0; b < e->nseq; b++) e->hoffs[b] = offsets[b];
    return 0;
}

void aarh_session_end(aarh_session* e) { delete e; }

int aarh_mtp_generate(aarh_ctx* c, const uint32_t* prompts, int nseq, int prompt_len, int max_new_tokens,
                      int num_draft_tokens, const aarh_sampler* s, const uint64_t* seeds, uint32_t* out_tokens,
                      int32_t* out_len, int32_t* finish_reason, aarh_spec_stats* stats) {
    if (!c) return AARH_ERR_CONFIG;
    for (int b = 0; b < nseq && b < c->cfg.max_batch; b++) c->kv_len[b] = 0;
    aarh_session* e = nullptr;
    int r = aarh_session_begin(c, prompts, nseq, prompt_len, 0, max_new_tokens, num_draft_tokens, s, seeds, &e);
    if (r) return r;
    int32_t done = 0;
    r = aarh_session_step(e, 1 << 30, &done);
    if (!r) r = aarh_session_result(e, out_tokens, max_new_tokens, out_len, finish_reason, stats);
    aarh_session_end(e);
    return r;
}

}  // extern "C"

// ===========================================================================
// Engine: SpeculativeEngine::generate_with_callback (speculative.rs:175-516)
// with an external draft model (second context), nseq requests in lock-step
// rounds.  Draft forwards, target verify, replays and the fused acceptance run
// on the device; the host keeps the per-request bookkeeping (commits, finish
// reasons, statistics, cache lengths).
// ===========================================================================
namespace {

struct XSession {
    aarh_ctx *c = nullptr, *d = nullptr;  // target, draft
    int nseq = 0, K = 0, max_new = 0, available = 0;
    bool greedy = true;
    aarh_sampler samp{};
    float *tgt = nullptr;  // [nseq][K+1][V] target rows T[i] for proposal i (T[np] = bonus row)
    float *drf = nullptr;  // [nseq][K][V] draft logits before proposal p (drf[b][0] = draft_next)
    uint32_t* props = nullptr;
    int32_t *acc_len = nullptr, *acc_tok = nullptr, *acc_draws = nullptr, *acc_status = nullptr, *nprop = nullptr;
    uint32_t* acc_flags = nullptr;
    uint64_t *seeds = nullptr, *offs = nullptr;
    const float** src = nullptr;
    float** dst = nullptr;
    std::vector<uint64_t> hoffs;
    std::vector<char> finished;
    std::vector<std::vector<uint32_t>> out;
    std::vector<int32_t> finish, pending, np, tbase, dbase, hlen, htok, hdraws, hstatus;
    std::vector<aarh_spec_stats> stats;
    std::vector<uint32_t> hprops;
    CandBuf cand;

    ~XSession() {
        cand.release();
        for (void* p : {(void*)tgt, (void*)drf, (void*)props, (void*)acc_len, (void*)acc_tok, (void*)acc_draws,
                        (void*)acc_status, (void*)nprop, (void*)acc_flags, (void*)seeds, (void*)offs, (void*)src,
                        (void*)dst})
            if (p) (void)hipFree(p);
    }
};

// Copy device rows src[i] -> dst[i] (n floats each) on ctx c's stream; waits.
int copy_rows_lists(XSession* e, aarh_ctx* c, const std::vector<const float*>& s, const std::vector<float*>& d, int n) {
    if (s.empty()) return 0;
    const int rows = (int)s.size();
    for (int r0 = 0; r0 < rows; r0 += 2 * e->c->cfg.max_batch) {
        const int nr = std::min(rows - r0, 2 * e->c->cfg.max_batch);
        HIPCHK(c, hipMemcpyAsync(e->src, s.data() + r0, nr * sizeof(void*), hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, hipMemcpyAsync(e->dst, d.data() + r0, nr * sizeof(void*), hipMemcpyHostToDevice, c->stream));
        KCHK(c, launch_copy_rows(e->src, e->dst, nr, n, c->stream));
        if (int r = sync_stream(c)) return r;
    }
    return 0;
}

// One ragged batch: sequence seqs[j] feeds rows[j] (<= S) ids at offset off[j] on
// its own slot; rows past rows[j] repeat the last id (padding, truncated by the
// cache length set afterwards).  Logits of (j, s) land in x->logits row j*S + s.
int ragged_forward(aarh_ctx* x, const std::vector<int>& seqs, const std::vector<std::vector<uint32_t>>& ids,
                   const std::vector<int>& off, int* S_out) {
    const int n = (int)seqs.size();
    int S = 1;
    for (const auto& v : ids) S = std::max(S, (int)v.size());
    std::vector<uint32_t> flat((size_t)n * S);
    std::vector<int32_t> sl(n), of(n);
    for (int j = 0; j < n; j++) {
        sl[j] = seqs[j];
        of[j] = off[j];
        for (int s2 = 0; s2 < S; s2++) flat[(size_t)j * S + s2] = ids[j][std::min(s2, (int)ids[j].size() - 1)];
    }
    int mk = 0, r;
    if ((r = stage_rows(x, flat.data(), sl.data(), of.data(), n, S, &mk, PAD_SLACK))) return r;
    if ((r = forward_dev(x, x->d_ids, x->d_pos0, x->d_slot, n, S, mk, x->logits, rm(n * S, 0, x->V), nullptr))) return r;
    for (int j = 0; j < n; j++) x->kv_len[seqs[j]] = off[j] + (int)ids[j].size();
    *S_out = S;
    return 0;
}

// Sample one token per sequence from rows drf[b][p] (draft proposal p); active[b]:
// the sequence proposes at p (its distribution must be valid).
int sample_draft_rows(XSession* e, int p, const std::vector<char>& active) {
    aarh_ctx* c = e->c;
    const int nseq = e->nseq, K = e->K, V = c->V;
    int r;
    if (e->greedy) {
        KCHK(c, launch_argmax_rows(e->drf + (size_t)p * V, (long long)K * V, nseq, V, (int32_t*)e->props + p, K, nullptr,
                                   c->stream));
    } else {
        std::vector<uint64_t> o(nseq);
        for (int b = 0; b < nseq; b++) o[b] = e->hoffs[b] + p;
        HIPCHK(c, hipMemcpyAsync(e->offs, o.data(), nseq * 8, hipMemcpyHostToDevice, c->stream));
        if ((r = aarh_accept_sample(c, e->drf + (size_t)p * V, K, nullptr, nullptr, nullptr, nseq, 0, V, 1, &e->samp,
                                    e->seeds, e->offs, nullptr, e->acc_len, e->acc_tok, e->acc_flags, e->acc_draws,
                                    e->acc_status, nullptr)))
            return r;
        if ((r = sync_stream(c))) return r;
        std::vector<int32_t> t(nseq), st(nseq);
        HIPCHK(c, hipMemcpy(t.data(), e->acc_tok, nseq * 4, hipMemcpyDeviceToHost));
        HIPCHK(c, hipMemcpy(st.data(), e->acc_status, nseq * 4, hipMemcpyDeviceToHost));
        for (int b = 0; b < nseq; b++) {
            // rows of requests that sit this step out are sampled too and ignored
            if (active[b] && st[b] != 0)
                return fail(c, AARH_ERR_CONFIG, "proposal distribution is invalid (zero mass or does not sum to one)");
            e->hprops[(size_t)b * K + p] = (uint32_t)(st[b] ? 0 : t[b]);
        }
        HIPCHK(c, hipMemcpy(e->props, e->hprops.data(), (size_t)nseq * K * 4, hipMemcpyHostToDevice));
    }
    if ((r = sync_stream(c))) return r;
    std::vector<uint32_t> t((size_t)nseq * K);
    HIPCHK(c, hipMemcpy(t.data(), e->props, t.size() * 4, hipMemcpyDeviceToHost));
    for (int b = 0; b < nseq; b++) e->hprops[(size_t)b * K + p] = t[(size_t)b * K + p];
    return 0;
}

// One round of speculative.rs:251-509 for every unfinished request.
int xsession_round(XSession* e) {
    aarh_ctx *c = e->c, *d = e->d;
    const int nseq = e->nseq, K = e->K, V = c->V;
    int r;
    std::vector<int> count(nseq, 0);
    std::vector<char> alive(nseq, 0);
    int Kr = 0;
    for (int b = 0; b < nseq; b++) {
        if (e->finished[b]) continue;
        count[b] = std::min(K, e->max_new - (int)e->out[b].size());
        alive[b] = 1;
        e->np[b] = 0;
        e->tbase[b] = c->kv_len[b];
        e->dbase[b] = d->kv_len[b];
        Kr = std::max(Kr, count[b]);
    }
    // ---- draft proposals (speculative.rs:267-304) ----
    for (int p = 0; p < Kr; p++) {
        std::vector<char> act(nseq);
        for (int b = 0; b < nseq; b++) act[b] = alive[b] && p < count[b];
        if ((r = sample_draft_rows(e, p, act))) return r;
        std::vector<int> fs, fo;
        std::vector<std::vector<uint32_t>> fi;
        for (int b = 0; b < nseq; b++) {
            if (!alive[b] || p >= count[b]) continue;
            const uint32_t tok = e->hprops[(size_t)b * K + p];
            e->np[b]++;
            e->stats[b].draft_tokens_proposed++;
            if (tok == EOS_ID) {
                alive[b] = 0;
                continue;
            }
            fs.push_back(b);
            fo.push_back(d->kv_len[b]);
            fi.push_back({tok});
            e->stats[b].draft_decode_forwards++;
        }
        if (fs.empty()) continue;
        int S = 0;
        if ((r = ragged_forward(d, fs, fi, fo, &S))) return r;
        std::vector<const float*> ls;
        std::vector<float*> ld;
        for (size_t j = 0; j < fs.size(); j++)
            if (p + 1 < count[fs[j]] ) {
                ls.push_back(d->logits + j * (size_t)S * V);
                ld.push_back(e->drf + ((size_t)fs[j] * K + p + 1) * V);
            }
        if ((r = copy_rows_lists(e, d, ls, ld, V))) return r;
    }
    // ---- target verify of [pending?] + proposals (speculative.rs:306-323) ----
    std::vector<int> vs, vo;
    std::vector<std::vector<uint32_t>> vi;
    for (int b = 0; b < nseq; b++) {
        if (e->finished[b]) continue;
        std::vector<uint32_t> ids;
        if (e->pending[b] >= 0) ids.push_back((uint32_t)e->pending[b]);
        for (int i = 0; i < e->np[b]; i++) ids.push_back(e->hprops[(size_t)b * K + i]);
        vs.push_back(b);
        vo.push_back(e->tbase[b]);
        vi.push_back(ids);
        e->stats[b].rounds++;
        e->stats[b].target_decode_forwards++;
    }
    if (vs.empty()) return 0;
    {
        int S = 0;
        if ((r = ragged_forward(c, vs, vi, vo, &S))) return r;
        // rows -> T[i]: with a pending token verify row i is T[i]; without, T[0] is
        // target_next (already in place) and verify row i is T[i + 1]
        std::vector<const float*> ls;
        std::vector<float*> ld;
        for (size_t j = 0; j < vs.size(); j++) {
            const int b = vs[j], shift = e->pending[b] >= 0 ? 0 : 1;
            for (int s2 = 0; s2 < (int)vi[j].size(); s2++) {
                ls.push_back(c->logits + (j * (size_t)S + s2) * V);
                ld.push_back(e->tgt + ((size_t)b * (K + 1) + s2 + shift) * V);
            }
        }
        if ((r = copy_rows_lists(e, c, ls, ld, V))) return r;
    }
    // ---- acceptance with bonus (speculative.rs:329-501) ----
    {
        std::vector<uint64_t> o(nseq);
        std::vector<int32_t> npv(nseq);
        for (int b = 0; b < nseq; b++) {
            o[b] = e->hoffs[b] + e->np[b];
            npv[b] = e->finished[b] ? 0 : e->np[b];
        }
        HIPCHK(c, hipMemcpyAsync(e->offs, o.data(), nseq * 8, hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, hipMemcpyAsync(e->nprop, npv.data(), nseq * 4, hipMemcpyHostToDevice, c->stream));
        // the top candidates (output metadata) run beside the acceptance kernel
        if ((r = e->cand.launch(c, e->tgt, nseq * (K + 1), V, e->samp))) return r;
        r = aarh_accept_sample(c, e->tgt, K + 1, e->drf, e->props, e->nprop, nseq, K, V, 1, &e->samp, e->seeds,
                               e->offs, nullptr, e->acc_len, e->acc_tok, e->acc_flags, e->acc_draws, e->acc_status,
                               nullptr);
        // join the side stream on every path: its kernel reads tgt, which later work rewrites
        const int rj = e->cand.join(c);
        if (r || (r = rj) || (r = sync_stream(c))) return r;
        if ((r = e->cand.fetch(c, nseq * (K + 1)))) return r;
        HIPCHK(c, hipMemcpy(e->hlen.data(), e->acc_len, nseq * 4, hipMemcpyDeviceToHost));
        HIPCHK(c, hipMemcpy(e->htok.data(), e->acc_tok, nseq * 4, hipMemcpyDeviceToHost));
        HIPCHK(c, hipMemcpy(e->hdraws.data(), e->acc_draws, nseq * 4, hipMemcpyDeviceToHost));
        HIPCHK(c, hipMemcpy(e->hstatus.data(), e->acc_status, nseq * 4, hipMemcpyDeviceToHost));
    }
    // ---- commit, rollback, replay ----
    std::vector<int> ts, to, ds, dof;
    std::vector<std::vector<uint32_t>> ti, di;
    for (size_t j = 0; j < vs.size(); j++) {
        const int b = vs[j];
        if (e->hstatus[b] != 0)
            return fail(c, AARH_ERR_CONFIG, "speculative residual distribution has zero probability mass");
        if (!e->greedy) e->hoffs[b] += e->np[b] + e->hdraws[b];
        const int npb = e->np[b], acc = e->hlen[b], hp = e->pending[b] >= 0 ? 1 : 0;
        const std::vector<uint32_t>& tin = vi[j];
        e->pending[b] = -1;
        bool done = false;
        for (int i = 0; i < acc && !done; i++) {
            e->stats[b].draft_tokens_accepted++;
            const uint32_t t = e->hprops[(size_t)b * K + i];
            if (t == EOS_ID) {
                e->finish[b] = AARH_FINISH_EOS;
                done = true;
                break;
            }
            e->out[b].push_back(t);
            e->cand.commit(b, b * (K + 1) + i);
            if ((int)e->out[b].size() == e->max_new) done = true;
        }
        if (done) {
            e->finished[b] = 1;
            continue;
        }
        if (acc < npb) {
            // rejection at acc: restore both caches, replay the accepted prefix
            const uint32_t repl = (uint32_t)e->htok[b];
            c->kv_len[b] = e->tbase[b];
            d->kv_len[b] = e->dbase[b];
            if (hp + acc > 0) {
                ts.push_back(b);
                to.push_back(e->tbase[b]);
                ti.emplace_back(tin.begin(), tin.begin() + hp + acc);
            }
            if (acc > 0) e->stats[b].draft_decode_forwards++;
            if (repl == EOS_ID) {
                e->finish[b] = AARH_FINISH_EOS;
                e->finished[b] = 1;
                continue;
            }
            e->out[b].push_back(repl);
            e->cand.commit(b, b * (K + 1) + acc);
            // draft: accepted prefix replay + the replacement, one launch (two reference forwards)
            std::vector<uint32_t> dr(e->hprops.begin() + (size_t)b * K, e->hprops.begin() + (size_t)b * K + acc);
            dr.push_back(repl);
            ds.push_back(b);
            dof.push_back(e->dbase[b]);
            di.push_back(dr);
            e->stats[b].draft_decode_forwards++;
            e->pending[b] = (int)repl;
        } else {
            // every proposal accepted: target cache keeps them, bonus from T[np]
            c->kv_len[b] = e->tbase[b] + hp + npb;
            const uint32_t bonus = (uint32_t)e->htok[b];
            if (bonus == EOS_ID) {
                e->finish[b] = AARH_FINISH_EOS;
                e->finished[b] = 1;
                continue;
            }
            e->out[b].push_back(bonus);
            e->cand.commit(b, b * (K + 1) + npb);
            ds.push_back(b);
            dof.push_back(d->kv_len[b]);
            di.push_back({bonus});
            e->stats[b].draft_decode_forwards++;
            e->pending[b] = (int)bonus;
        }
        if ((int)e->out[b].size() >= e->max_new) e->finished[b] = 1;
    }
    if (!ts.empty()) {
        int S = 0;
        if ((r = ragged_forward(c, ts, ti, to, &S))) return r;
    }
    if (!ds.empty()) {
        int S = 0;
        if ((r = ragged_forward(d, ds, di, dof, &S))) return r;
        std::vector<const float*> ls;
        std::vector<float*> ld;
        for (size_t j = 0; j < ds.size(); j++) {
            ls.push_back(d->logits + (j * (size_t)S + di[j].size() - 1) * V);
            ld.push_back(e->drf + (size_t)ds[j] * K * V);  // draft_next = proposal 0's logits
        }
        if ((r = copy_rows_lists(e, d, ls, ld, V))) return r;
    }
    return 0;
}

}  // namespace

// The external-draft engine as a session (round-by-round driving, keystream positions).
struct aarh_spec_session {
    XSession e;
    int max_new_tokens = 0;  // the caller's budget: row capacity of the results
};

namespace {

int spec_begin(aarh_ctx* c, aarh_ctx* d, const uint32_t* prompts, int nseq, int prompt_len, int max_new_tokens,
               int num_draft_tokens, const aarh_sampler* s, const uint64_t* seeds, XSession& e) {
    if (!c || !d || !s) return AARH_ERR_CONFIG;
    if (num_draft_tokens <= 0) return fail(c, AARH_ERR_CONFIG, "num_draft_tokens must be greater than zero");
    if (num_draft_tokens >= PAD_SLACK)
        return fail(c, AARH_ERR_UNSUPPORTED, "num_draft_tokens must be below %d on the device path", PAD_SLACK);
    if (c->device != d->device) return fail(c, AARH_ERR_CONFIG, "draft and target models must use the same device");
    if (c->V != d->V) return fail(c, AARH_ERR_CONFIG, "draft and target vocabularies differ (%d vs %d)", d->V, c->V);
    if (nseq <= 0 || nseq > c->cfg.max_batch || nseq > d->cfg.max_batch)
        return fail(c, AARH_ERR_SHAPE, "nseq %d exceeds max_batch", nseq);
    if (prompt_len <= 0) return fail(c, AARH_ERR_SHAPE, "prompt must be non-empty");
    if (!prompts) return fail(c, AARH_ERR_CONFIG, "null prompts");
    if (max_new_tokens < 0) return fail(c, AARH_ERR_SHAPE, "negative max_new_tokens");
    const int max_seq = std::min(c->cfg.max_seq_len, d->cfg.max_seq_len);
    if (prompt_len >= max_seq)
        return fail(c, AARH_ERR_SHAPE, "prompt has %d tokens but speculative context limit is %d (target=%d, draft=%d)",
                    prompt_len, max_seq, c->cfg.max_seq_len, d->cfg.max_seq_len);
    const bool greedy = s->greedy || !(s->temperature > 1.1920929e-07f);
    const int K = num_draft_tokens, V = c->V;
    if (nseq * (K + 1) > c->Mmax || nseq * (K + 1) > d->Mmax)
        return fail(c, AARH_ERR_SHAPE, "nseq x (draft tokens + 1) exceeds max_rows");
    e.c = c;
    e.d = d;
    e.nseq = nseq;
    e.K = K;
    e.greedy = greedy;
    e.samp = *s;
    e.available = max_seq - prompt_len;
    e.max_new = std::min(max_new_tokens, e.available);
    e.hoffs.assign(nseq, 0);
    e.finished.assign(nseq, 0);
    e.out.assign(nseq, {});
    e.finish.assign(nseq, AARH_FINISH_MAX_TOKENS);
    e.stats.assign(nseq, aarh_spec_stats{});
    e.hprops.assign((size_t)nseq * K, 0);
    for (auto* v : {&e.np, &e.tbase, &e.dbase, &e.hlen, &e.htok, &e.hdraws, &e.hstatus}) v->assign(nseq, 0);
    e.pending.assign(nseq, -1);
    int r = 0;
#define XA(p, bytes) \
    if ((r = dalloc(c, &e.p, (bytes)))) return r;
    XA(tgt, (size_t)nseq * (K + 1) * V * 4);
    XA(drf, (size_t)nseq * K * V * 4);
    XA(props, (size_t)nseq * K * 4);
    XA(acc_len, nseq * 4);
    XA(acc_tok, nseq * 4);
    XA(acc_draws, nseq * 4);
    XA(acc_status, nseq * 4);
    XA(nprop, nseq * 4);
    XA(acc_flags, nseq * 4);
    XA(seeds, nseq * 8);
    XA(offs, nseq * 8);
    XA(src, (size_t)2 * c->cfg.max_batch * sizeof(void*));
    XA(dst, (size_t)2 * c->cfg.max_batch * sizeof(void*));
#undef XA
    if ((r = e.cand.alloc(c, nseq * (K + 1), nseq))) return r;
    // rows of requests that sit out a step are sampled too (and ignored): keep them finite
    HIPCHK(c, hipMemset(e.tgt, 0, (size_t)nseq * (K + 1) * V * 4));
    HIPCHK(c, hipMemset(e.drf, 0, (size_t)nseq * K * V * 4));
    {
        std::vector<uint64_t> hs(nseq);
        for (int b = 0; b < nseq; b++) hs[b] = seeds ? seeds[b] : 0;
        HIPCHK(c, hipMemcpy(e.seeds, hs.data(), nseq * 8, hipMemcpyHostToDevice));
    }
    if (e.max_new > 0) {
        // prefill both models (speculative.rs:236-247), chunked to max_rows
        for (aarh_ctx* x : {c, d}) {
            const int chunk = std::max(1, x->Mmax / nseq);
            std::vector<int> seqs(nseq), off(nseq);
            for (int b = 0; b < nseq; b++) {
                seqs[b] = b;
                x->kv_len[b] = 0;
            }
            for (int p0 = 0; p0 < prompt_len; p0 += chunk) {
                const int S = std::min(chunk, prompt_len - p0);
                std::vector<std::vector<uint32_t>> ids(nseq);
                for (int b = 0; b < nseq; b++) {
                    off[b] = p0;
                    ids[b].assign(prompts + (size_t)b * prompt_len + p0, prompts + (size_t)b * prompt_len + p0 + S);
                }
                int Sx = 0;
                if ((r = ragged_forward(x, seqs, ids, off, &Sx))) return r;
                if (p0 + S == prompt_len) {
                    std::vector<const float*> ls(nseq);
                    std::vector<float*> ld(nseq);
                    for (int b = 0; b < nseq; b++) {
                        ls[b] = x->logits + ((size_t)b * Sx + S - 1) * V;
                        ld[b] = x == c ? e.tgt + (size_t)b * (K + 1) * V : e.drf + (size_t)b * K * V;
                    }
                    if ((r = copy_rows_lists(&e, x, ls, ld, V))) return r;
                }
            }
        }
    } else {
        for (int b = 0; b < nseq; b++) {
            e.finish[b] = AARH_FINISH_CONTEXT_LIMIT;
            e.finished[b] = 1;
        }
    }
    return 0;
}

}  // namespace

extern "C" int aarh_spec_session_begin(aarh_ctx* c, aarh_ctx* d, const uint32_t* prompts, int nseq, int prompt_len,
                                       int max_new_tokens, int num_draft_tokens, const aarh_sampler* s,
                                       const uint64_t* seeds, aarh_spec_session** out) {
    if (!out) return fail(c, AARH_ERR_CONFIG, "null session pointer");
    *out = nullptr;
    auto* ss = new aarh_spec_session();
    ss->max_new_tokens = max_new_tokens;
    const int r = spec_begin(c, d, prompts, nseq, prompt_len, max_new_tokens, num_draft_tokens, s, seeds, ss->e);
    if (r) {
        delete ss;
        return r;
    }
    *out = ss;
    return 0;
}

extern "C" int aarh_spec_session_step(aarh_spec_session* ss, int max_rounds, int32_t* all_done) {
    if (!ss) return AARH_ERR_CONFIG;
    XSession& e = ss->e;
    for (int i = 0; i < max_rounds; i++) {
        bool any = false;
        for (int b = 0; b < e.nseq; b++)
            if (!e.finished[b]) any = true;
        if (!any) break;
        if (int r = xsession_round(&e)) return r;
    }
    if (all_done) {
        *all_done = 1;
        for (int b = 0; b < e.nseq; b++)
            if (!e.finished[b]) *all_done = 0;
    }
    return 0;
}

extern "C" int aarh_spec_session_result(aarh_spec_session* ss, uint32_t* out_tokens, int32_t out_cap,
                                        int32_t* out_len, int32_t* finish_reason, aarh_spec_stats* stats) {
    if (!ss) return AARH_ERR_CONFIG;
    const XSession& e = ss->e;
    for (int b = 0; b < e.nseq; b++) {
        const int n = (int)e.out[b].size();
        if (out_len) out_len[b] = n;
        if (out_tokens)
            for (int i = 0; i < n && i < out_cap; i++) out_tokens[(size_t)b * out_cap + i] = e.out[b][i];
        int fin = e.finish[b];
        if (e.finished[b] && n == e.available && fin == AARH_FINISH_MAX_TOKENS) fin = AARH_FINISH_CONTEXT_LIMIT;
        if (finish_reason) finish_reason[b] = fin;
        if (stats) {
            stats[b] = e.stats[b];
            stats[b].draft_tokens_rejected =
                std::max(0, stats[b].draft_tokens_proposed - stats[b].draft_tokens_accepted);
        }
    }
    return 0;
}

extern "C" int aarh_spec_session_candidates(aarh_spec_session* ss, uint32_t* ids, float* probs, int32_t out_cap) {
    if (!ss) return AARH_ERR_CONFIG;
    ss->e.cand.copy_out(ss->e.nseq, out_cap, ids, probs);
    return 0;
}

extern "C" int aarh_spec_session_rng_offsets(aarh_spec_session* ss, uint64_t* out) {
    if (!ss || !out) return AARH_ERR_CONFIG;
    for (int b = 0; b < ss->e.nseq; b++) out[b] = ss->e.hoffs[b];
    return 0;
}

extern "C" int aarh_spec_session_set_rng_offsets(aarh_spec_session* ss, const uint64_t* offsets) {
    if (!ss || !offsets) return AARH_ERR_CONFIG;
    for (int b = 0; b < ss->e.nseq; b++) ss->e.hoffs[b] = offsets[b];
    return 0;
}

extern "C" void aarh_spec_session_end(aarh_spec_session* ss) {
    if (!ss) return;
    (void)hipStreamSynchronize(ss->e.c->stream);
    (void)hipStreamSynchronize(ss->e.d->stream);
    if (ss->e.c->side) (void)hipStreamSynchronize(ss->e.c->side);
    delete ss;
}

extern "C" int aarh_spec_generate(aarh_ctx* c, aarh_ctx* d, const uint32_t* prompts, int nseq, int prompt_len,
                                  int max_new_tokens, int num_draft_tokens, const aarh_sampler* s,
                                  const uint64_t* seeds, uint32_t* out_tokens, int32_t* out_len,
                                  int32_t* finish_reason, aarh_spec_stats* stats, uint32_t* out_cand_ids,
                                  float* out_cand_probs) {
    aarh_spec_session* ss = nullptr;
    int r = aarh_spec_session_begin(c, d, prompts, nseq, prompt_len, max_new_tokens, num_draft_tokens, s, seeds, &ss);
    if (r) return r;
    int32_t done = 0;
    while (!done && !r) r = aarh_spec_session_step(ss, 1 << 20, &done);
    if (!r) r = aarh_spec_session_result(ss, out_tokens, max_new_tokens, out_len, finish_reason, stats);
    if (!r) r = aarh_spec_session_candidates(ss, out_cand_ids, out_cand_probs, max_new_tokens);
    aarh_spec_session_end(ss);
    return r;
}
