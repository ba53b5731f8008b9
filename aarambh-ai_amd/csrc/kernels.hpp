// Kernel argument blocks and launchers of libaarambh_hip (host + device view).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aarh {

enum WFmt { WF_F32 = 0, WF_BF16 = 1, WF_INT8 = 2, WF_INT4 = 3 };
enum KvFmt { KV_F32 = 0, KV_F16 = 1, KV_INT8 = 2 };
enum Epi { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV = 3 };

enum { ACCEPT_FLAG_RATIO_NEAR = 1u, ACCEPT_FLAG_CDF_NEAR = 2u };

// Dynamic LDS a kernel may request: 160 KiB per workgroup on gfx950 minus room
// for the kernels' static LDS.
static constexpr size_t MAX_DYN_LDS = 160 * 1024 - 4096;

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

// Cache-append part of the fused QKV epilogue (RoPE + KV write).
struct QkvEpi {
    int n_heads, n_kv, hd;
    const int* pos0;    // [nseq] position of row s == 0
    const int* slot;    // [nseq] cache slot of each sequence
    const float* rope_cos;
    const float* rope_sin; // [max_seq][hd/2]
    float* q_out;          // [M][n_heads*hd] rotated queries
    int kv_fmt;
    int cap;               // tokens per slot
    void* kc;              // K [slot][n_kv][cap][hd]
    void* vc;              // V [slot][n_kv][hd][cap]  (transposed)
    uint16_t* ks;          // INT8 K scales [slot][n_kv][cap] (fp16)
    uint16_t* vs;          // INT8 V scales
};

struct GemvArgs {
    int fmt;
    const uint8_t* w;     // tiled weights (BF16/INT8/INT4) or row-major f32
    const uint32_t* sz;   // INT4: fp16 scale | fp16 zero << 16, per (tile, group, row)
    const float* rscale;  // INT8: per-row scales
    int N, K, M;
    int S;                // k-splits (workgroups per 128-row group)
    int split;            // 1: activations as fp16/bf16 hi+lo rows
    const float* x;       // input activations
    RowMap xmap;
    const float* norm_w;  // RMSNorm weight fused as prologue (null: none)
    const float* ssq_part;
    int n_ssq;
    float eps;
    float* hidden_out;    // optional normalised input copy [M][K]
    float* part;          // [S][M][N] split-K partial sums
    unsigned* counters;   // [N/128], zero between launches
    int epi;
    float* out;           // STORE / SWIGLU output
    RowMap omap;
    float* resid;         // RESID target [M][N] (row stride ldr)
    int ldr;
    float* ssq_out;       // RESID: [N/128][M]
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
    float scale;
    int chunk;            // tokens per workgroup
    int nchunks;
    int rows_per_tile;    // query rows (token x group-head) per workgroup
    int ntiles;
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
    const uint64_t* seeds;
    const uint64_t* word_offsets;
    const float* uniforms;
    float* row_max;
    float* row_sum;
    int32_t* row_argmax;
    unsigned* counters;
    int32_t* out_accept_len;
    int32_t* out_token;
    uint32_t* out_flags;
    int32_t* out_draws;
    int32_t* out_status;
};

int launch_accept(const AcceptArgs& a, hipStream_t stream);
int launch_gemv(const GemvArgs& a, hipStream_t stream);
int launch_attention(const AttnArgs& a, hipStream_t stream);
bool attention_uses_mfma(int kv_fmt, int hd);

// misc kernels
int launch_embed(const void* table, int table_fmt, int H, const uint32_t* ids, int M, float* x,
                 float* ssq_part, hipStream_t stream);
int launch_mtp_prep(const float* anchor, long long anchor_stride, const void* table, int table_fmt,
                    const uint32_t* ids, int ids_stride, int nseq, int L, int H, const float* trunk_w,
                    const float* token_w, float eps, float* x, float* ssq_part, hipStream_t stream);
int launch_norm_rows(const float* x, RowMap xmap, int M, int H, const float* w, float eps, float* out,
                     hipStream_t stream);
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
int launch_fill_f32(float* p, long long n, float v, hipStream_t stream);

}  // namespace aarh
