// Kernel argument blocks and launchers of libaarambh_hip (host + device view).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

namespace aarh {

enum WFmt { WF_F32 = 0, WF_BF16 = 1, WF_INT8 = 2, WF_INT4 = 3 };
enum KvFmt { KV_F32 = 0, KV_F16 = 1, KV_INT8 = 2 };

// Element offset of V (dim d, token t) in the cache of head hb (= slot * n_kv + kv head).
// INT8 / fp16 caches keep V^T in 32-token blocks, [head][cap/32][hd][32]: the 32 tokens x
// hd dims a decode wave reads per step are one contiguous run (cap is a multiple of 32).
// f32 caches (MTP head scratch) keep [head][hd][cap].
__host__ __device__ inline size_t vt_off(size_t hb, int d, int t, int cap, int hd, int kv_fmt) {
    if (kv_fmt == KV_F32) return (hb * hd + d) * (size_t)cap + t;
    return ((hb * (size_t)(cap >> 5) + (t >> 5)) * hd + d) * 32 + (t & 31);
}

// Element offset of K (token t, dim d) in the cache of head hb.  INT8 / fp16 caches with
// head_dim 128 store each 32-token block (32 x 128 elements, contiguous) in the order the
// decode wave loads it: 16-byte chunk (ts, c) of lane (lg, lr) holds token row
// 8 (lr / 4) + 4 ts + lr % 4, dims 32 lg + c * (16 / esize) ..; one load instruction then
// reads 1 KiB contiguous.  Other caches are row-major [head][cap][hd].
__host__ __device__ inline size_t k_off(size_t hb, int t, int d, int cap, int hd, int kv_fmt) {
    if (kv_fmt == KV_F32 || hd != 128) return (hb * cap + t) * (size_t)hd + d;
    const int r = t & 31, ts = (r >> 2) & 1, lr = ((r >> 3) << 2) | (r & 3), lane = ((d >> 5) << 4) | lr;
    const int per = kv_fmt == KV_INT8 ? 16 : 8, nc = 32 / per;  // elements per chunk, chunks per lane row
    const int c = (d & 31) / per, j = d & (per - 1);
    return (hb * cap + (t & ~31)) * 128 + ((size_t)(ts * nc + c) * 64 + lane) * per + j;
}
enum Epi { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV = 3 };

enum { ACCEPT_FLAG_RATIO_NEAR = 1u, ACCEPT_FLAG_CDF_NEAR = 2u, ACCEPT_FLAG_TOPP_NEAR = 8u };

// Acceptance scratch: ACC_RS_WORDS 32-bit words of distribution parameters per
// logits row, and one arrival counter per sequence (zero between launches).
static constexpr int ACC_RS_WORDS = 12;
// Capacity of the statically allocated scratch of aarh_accept_sample_static.
static constexpr int ACC_STATIC_ROWS = 4096;
static constexpr int ACC_STATIC_SEQS = 1024;

// Dynamic LDS a kernel may request: 160 KiB per workgroup on gfx950 minus room
// for the kernels' static LDS.
static constexpr size_t MAX_DYN_LDS = 160 * 1024 - 4096;

// Kernel timing for the runtime's per-class profile: while `stop` is set, the
// instrumented launches record `start` at the first dispatch's start and `stop`
// at each dispatch's end (hipExtLaunchKernelGGL), so the profile holds kernel
// durations without launch gaps.
struct LaunchTiming {
    hipEvent_t start, stop;
    int launches;
};
extern thread_local LaunchTiming g_launch_timing;

template <typename... Args, typename F = void (*)(Args...)>
inline void launch_timed(F kernel, const dim3& grid, const dim3& block, uint32_t shmem, hipStream_t stream,
                         Args... args) {
    LaunchTiming& t = g_launch_timing;
    if (t.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, t.launches == 0 ? t.start : nullptr, t.stop, 0u,
                              args...);
        t.launches++;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream, args...);
    }
}

// Records the message of a failing HIP call (read by the runtime's error path).
int note_error(hipError_t e);
const char* last_launch_error();

// Rows of an activation block are indexed m = seq * S + s (S rows per sequence).
struct RowMap {
    int S;               // rows per sequence
    long long seq_stride; // elements between consecutive sequences
    long long row_stride; // elements between consecutive rows of a sequence
};

__host__ __device__ inline long long row_off(const RowMap& r, int m) {
    return (long long)(m / r.S) * r.seq_stride + (long long)(m % r.S) * r.row_stride;
}

// An activation matrix written once, by its producer, in the operand format of
// the quantised GEMV that consumes it: fp16 (bf16 for BF16 weights) hi and lo
// halves of x * norm_w, in MFMA k-slot order.  Layout in 16-byte entries:
//   index = ((((mt * G + g) * 4 + t) * 4 + lg) * EPB + e)
// for row chunk mt (16 rows), 128-column group g, k-step t (8 columns), lane
// group lg (32 columns); EPB = 2*mp entries for mp <= 8 (hi of row r at e = r,
// lo at e = mp + r: the two halves occupy MFMA rows), 32 for mp = 16 (hi at
// e = r, lo at 16 + r: the halves are two MFMAs; 16-row chunks also feed the
// many-row GEMM).  The slot of column c inside an entry is frag_slot(fmt,
// c % 8).  Sums of squares of the raw values over 16-column tiles go to
// ssq[m * ssq_ld + c / 16] for the consumer's RMSNorm (a row's partials are contiguous).

struct XFrag {
    uint16_t* buf;        // null: the consumer reads f32 rows (no fragments)
    int fmt;              // consumer weight format (WF_INT4 / WF_INT8 / WF_BF16)
    int mp;               // 4, 8 or 16 activation rows per MFMA row tile
    int G;                // consumer K / 128
    const float* norm_w;  // consumer RMSNorm weight (null: none)
    float* ssq;           // 16-column partial sums of squares (null: none)
    int ssq_ld;           // row stride of ssq (16-column tiles per row)
};

__host__ __device__ inline int frag_epb(int mp) { return mp <= 8 ? 2 * mp : 32; }

// k-slot j of an 8-column block holds column frag_elem(fmt, j): the order in
// which the weight dequantisation of each format emits B elements.
__host__ __device__ inline int frag_elem(int fmt, int j) {
    if (fmt == WF_INT4) return (j >> 1) | ((j & 1) << 2);
    if (fmt == WF_INT8) return (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1);
    return j;
}
__host__ __device__ inline int frag_slot(int fmt, int e) {
    if (fmt == WF_INT4) return ((e & 3) << 1) | (e >> 2);
    if (fmt == WF_INT8) return (e & 4) | ((e & 1) << 1) | ((e >> 1) & 1);
    return e;
}

// RoPE part of the fused QKV epilogue: rotated queries and the new K / V rows
// (appended to the cache by the attention kernel).
struct QkvEpi {
    int n_heads, n_kv, hd;
    int S;                 // rows per sequence
    const int* pos0;       // [nseq] position of row s == 0
    const float* rope_cos;
    const float* rope_sin; // [max_seq][hd/2]
    float* q_out;          // [M][n_heads*hd] rotated queries
    float* kv_out;         // [M][2][n_kv*hd] rotated keys, then values
};

struct GemvArgs {
    int fmt;
    const uint8_t* w;     // tiled weights (BF16/INT8/INT4) or row-major f32
    const uint32_t* sz;   // INT4: fp16 scale | fp16 zero << 16, per (tile, group, row)
    const float* rscale;  // INT8: per-row scales
    int N, K;
    int M;                // activation rows of this launch (<= 16)
    int m_base;           // index of its first row in the row maps
    float* gpart;         // many-row GEMM: split-K partial tiles (scratch)
    unsigned* gcnt;       // many-row GEMM: arrival counters, zero between launches
    long long gpart_elems;
    const float* x;       // input activations (f32 rows: F32 weights, hidden_out)
    RowMap xmap;
    const uint16_t* xf;   // input fragments (quantised formats, XFrag layout)
    int mp;               // their row-tile size
    const float* norm_w;  // RMSNorm weight fused into the input (null: none)
    const float* ssq_in;  // 16-column partial sums of squares of the raw input
    int ssq_ld;
    float eps;
    float* hidden_out;    // optional normalised input copy [rows][K]
    int epi;
    float* out;           // STORE / SWIGLU output
    RowMap omap;
    float* resid;         // RESID target [rows][N] (row stride ldr)
    int ldr;
    XFrag fo;             // RESID / SWIGLU: fragments of the result for its consumer
    QkvEpi qkv;
};

struct AttnArgs {
    int nseq, S, n_heads, n_kv, hd;
    const int* pos0;
    const int* slot;
    const float* q;       // [M][n_heads*hd]
    int kv_fmt, cap;
    const void* kc;
    const void* vc;
    const uint16_t* ks;
    const uint16_t* vs;
    const float* knew;    // [M][2][n_kv*hd] this launch's K and V rows, appended by the kernel
    float scale;
    int chunk;            // tokens per workgroup
    int nchunks;
    int rows_per_tile;    // query rows (token x group-head) per workgroup
    int ntiles;
    XFrag fo;             // fragments of the output for the wo projection
    float* part;          // scratch partials
    unsigned* counters;   // [nseq*n_kv*ntiles]
    float* out;           // [M][n_heads*hd]
};

struct AcceptArgs {
    const float* target;
    int target_rows;
    const float* draft;
    const uint32_t* draft_tokens;
    const int32_t* n_proposals;
    int B, K, V;
    int bonus, greedy;
    float temperature;
    int top_k;            // <= 0: none
    float top_p;          // outside (0, 1): none
    const uint64_t* seeds;
    const uint64_t* word_offsets;
    const float* uniforms;
    uint32_t* rstat;      // [B * (target_rows + K)][ACC_RS_WORDS] row parameters (scratch)
    unsigned* counters;   // [B] arrival counters, zero between launches
    int chunk;            // set by the launcher
    int32_t* out_accept_len;
    int32_t* out_token;
    uint32_t* out_flags;
    int32_t* out_draws;
    int32_t* out_status;
};

int launch_accept(const AcceptArgs& a, hipStream_t stream);

// Top-n candidates of each row's sampling distribution (greedy: one-hot at the
// argmax; else filtered_probs: softmax at T after top-k, then top-p, with exact
// sequential normalisers).
static constexpr int CAND_MAX = 5;  // engine.rs:70 top_candidates
struct CandArgs {
    const float* logits;  // [rows][ld]
    long long ld;
    int rows, V, n;
    int greedy;
    float temperature;
    int top_k;
    float top_p;
    int chunk;            // set by the launcher
    uint32_t* ids;        // [rows][n]
    float* probs;         // [rows][n]
};
int launch_candidates(const CandArgs& a, hipStream_t stream);
// Statically allocated acceptance scratch (one copy per GPU): set-up on `device`
// (current) resolves its address once; accept_static_scratch returns it.
int accept_static_init(int device, hipStream_t stream);
int accept_static_scratch(int device, uint32_t** rstat, unsigned** counters);
int launch_zero_u32(uint32_t* p, int n, hipStream_t stream);
int launch_gemv(const GemvArgs& a, hipStream_t stream);
// Many-row variant (M > 16, fragments with mp = 16, all rows in one launch).
int launch_gemm(const GemvArgs& a, hipStream_t stream);
int launch_attention(const AttnArgs& a, hipStream_t stream);
bool attention_uses_mfma(int kv_fmt, int hd);

// misc kernels
int launch_embed(const void* table, int table_fmt, int H, const uint32_t* ids, int M, float* x,
                 const XFrag& fo, hipStream_t stream);
int launch_mtp_prep(const float* anchor, long long anchor_stride, const void* table, int table_fmt,
                    const uint32_t* ids, int ids_stride, int nseq, int L, int H, const float* trunk_w,
                    const float* token_w, float eps, float* x, const XFrag& fo, hipStream_t stream);
int launch_norm_rows(const float* x, RowMap xmap, int M, int H, const float* w, float eps, float* out,
                     const XFrag& fo, hipStream_t stream);
int launch_quantise_tiled(const float* w, int N, int K, int fmt, uint8_t* tiled, uint32_t* sz,
                          float* rscale, int row_offset, int N_total, int interleave_gu,
                          hipStream_t stream);
int launch_repack_int4(const uint8_t* packed, const uint16_t* sc, const uint16_t* zr, int N, int K,
                       uint8_t* tiled, uint32_t* sz, int row_offset, int N_total, int interleave_gu,
                       hipStream_t stream);
int launch_repack_int8(const int8_t* codes, const float* sc, int N, int K, uint8_t* tiled,
                       float* rscale, int row_offset, int N_total, int interleave_gu,
                       hipStream_t stream);
int launch_synth_fill(float* out, long long n, unsigned long long seed, unsigned stream_id, float std,
                      hipStream_t stream);
int launch_to_bf16(const float* src, uint16_t* dst, long long n, hipStream_t stream);
int launch_kv_fill_synthetic(void* kc, void* vc, uint16_t* ks, uint16_t* vs, int kv_fmt, int slot,
                             int n_kv, int hd, int cap, int len, unsigned long long seed, int layer,
                             hipStream_t stream);
int launch_argmax_rows(const float* x, long long ld, int rows, int V, int32_t* out, int out_stride, float* gap,
                       hipStream_t stream);
int launch_copy_rows(const float* const* src, float* const* dst, int rows, int n, hipStream_t stream);
int launch_mtp_verify_rows(const uint32_t* props, int K, int Kr, int nseq, const int32_t* limit, uint32_t eos,
                           uint32_t* ids, int32_t* nprop, const uint64_t* obase, uint64_t* offs, hipStream_t stream);
int launch_sampled_props(const int32_t* tok, const int32_t* status, uint32_t* props, int K, int p, int nseq,
                         const int32_t* limit, uint32_t eos, int32_t* pstat, hipStream_t stream);
int launch_fill_f32(float* p, long long n, float v, hipStream_t stream);

// ---------------------------------------------------------------------------
// Latent attention (MLA) + fine-grained MoE decoder kernels (lat.hip)
// ---------------------------------------------------------------------------
struct MlaArgs {
    int nseq, S;                 // sequences x rows per sequence (M = nseq * S)
    int nh, nope, rd, lat;       // heads, nope / rope / latent widths (v width: vd)
    int vd;
    const int* pos0;             // [nseq] position of row 0
    const int* slot;             // [nseq] cache slot
    const float* raw;            // [M][raw_ld]: q (nh*(nope+rd)) | kv_a (lat) | k_rope (rd)
    int raw_ld;
    const float* rope_cos;
    const float* rope_sin;       // [positions][rd/2]
    const _Float16* upk_hi;      // up_k as fp16 hi + lo pairs, per head transposed: [nh][lat][nope]
    const _Float16* upk_lo;
    const _Float16* upv_hi;      // up_v as fp16 hi + lo pairs: [nh][vd][lat]
    const _Float16* upv_lo;
    const float* kvn_w;          // [lat] latent RMSNorm weight
    float eps;
    float* q;                    // [M][nh][lat+rd]: absorbed q_lat | rotated q_rope
    _Float16* kc;                // [slots][cap][lat+rd]: c_kv | k_rope
    _Float16* vt;                // [slots][cap/32][lat][32]: c_kv transposed per 32-token block
    int cap;
    float scale;                 // 1/sqrt(nope + rd)
    int chunk, nchunks, ntiles;  // tokens per chunk, chunks, 16-row query tiles per sequence
    int tiles_per_wg;            // query tiles per attention workgroup (1..mla_tiles_per_wg_max())
    float* part;                 // [nseq][ntiles][nchunks][16][lat+4] chunk partials (m, l, pad, pad, o)
    float* olat;                 // [M][nh][lat] merged latent attention output
    XFrag fo;                    // fragments of the attention output for o_proj
    float* out;                  // [M][nh*vd] f32 attention output rows (null: fragments only)
};
int launch_mla_qprep(const MlaArgs& a, hipStream_t stream);
int launch_mla_kvprep(const MlaArgs& a, hipStream_t stream);
int launch_mla_attn(const MlaArgs& a, hipStream_t stream);
int launch_mla_out(const MlaArgs& a, hipStream_t stream);
bool mla_supported(int lat, int rd, int vd, int nope);
int mla_tiles_per_wg_max();

struct MoeArgs {
    int M, E, K, NS;             // rows, routed experts, top-k, shared experts
    int H, D;                    // hidden, fine expert width
    const float* logits;         // [M][lld] router logits (first E columns)
    int lld;
    int* cnt;                    // [E+NS] assignments per expert
    int* off;                    // [E+NS+1] their offsets
    int* arow;                   // [A] token row of each assignment (A = M*(K+NS))
    float* aw;                   // [A] its dispatch weight (1 for shared experts)
    int* rowmap;                 // [M][K+NS] assignments of a row: routed in expert order, then shared
    int fmt;                     // expert weight format (WF_INT4 / WF_INT8 / WF_BF16)
    const uint8_t* gu;           // tiled [(E+NS)*2D][H], gate/up rows interleaved 8 + 8 per tile
    const uint32_t* gu_sz;
    const float* gu_rs;
    const uint8_t* dn;           // tiled [(E+NS)*H][D]
    const uint32_t* dn_sz;
    const float* dn_rs;
    const float* xn;             // [M][H] normed FFN input (norm2)
    float* h;                    // [A][D] SwiGLU activations per assignment
    float* y;                    // [A][H] expert outputs per assignment (unweighted)
    float* x;                    // [M][H] residual stream
    XFrag fo;                    // fragments of the new x for the next consumer
    float* gap;                  // [M] running min of (k-th - (k+1)-th) router logit (null: none)
    unsigned long long* selm;    // [M] experts selected per row (bit e), written by the ranking
    float* wsel;                 // [M][64] dispatch weight of (row, selected expert)
    int* chunk_e;                // [cmax] expert of each 16-assignment chunk (written by the routing)
    int* chunk_r0;               // [cmax] its first assignment within the expert
    int* nchunk;                 // [1] number of chunks
    int cmax;                    // chunk capacity: M*K/16 + E + NS*ceil(M/16)
    int bpe;                     // expert projection: workgroups per chunk (tile-step slices)
};
int launch_moe_route(const MoeArgs& a, hipStream_t stream);
int launch_moe_ffn(const MoeArgs& a, int phase, hipStream_t stream);
int moe_tiles_per_step(int fmt);  // weight tiles per step of the expert projection
int launch_moe_combine(const MoeArgs& a, hipStream_t stream);
// fp16 hi + lo split of a row-major f32 matrix [N][K] (tblk > 0: row n = b * tblk + i,
// column k goes to ((b * K + k) * tblk + i)).
int launch_split_hilo(const float* src, _Float16* hi, _Float16* lo, int N, int K, int tblk, hipStream_t stream);
// Row-major f32 copy of a tiled quantised matrix (the values its GEMV multiplies
// by); tblk > 0 writes row n = b * tblk + i, column k at ((b * K + k) * tblk + i).
int launch_dequant_tiled(const uint8_t* tiled, const uint32_t* sz, const float* rscale, int fmt, int N, int K,
                         float* out, int tblk, hipStream_t stream);
int launch_lat_kv_fill_synthetic(_Float16* kc, _Float16* vt, int slot, int lat, int rd, int cap, int len,
                                 unsigned long long seed, int layer, hipStream_t stream);

}  // namespace aarh
