// Small kernels around the verify forward: embedding gather, MTP local
// sequence preparation, row RMSNorm, weight quantisation / repacking into the
// tiled GEMV layout, synthetic weights and KV contents, row argmax.
#include <float.h>
#include <stdio.h>

#include "device_common.hpp"
#include "kernels.hpp"
#include "frag.hpp"

namespace aarh {

static constexpr int MT_THREADS = 256;
static constexpr int RW_THREADS = 512;    // row kernels over a hidden-width row (one pass of ROW_U loads at 4096)
static constexpr int WIDE_THREADS = 1024; // row kernels over a vocabulary-width row
static constexpr int WIDE_U = 32;         // their loads in flight per thread (32768 floats per pass)

static thread_local char g_last_err[256] = "";
thread_local LaunchTiming g_launch_timing = {nullptr, nullptr, 0};

int note_error(hipError_t e) {
    if (e == hipSuccess) return 0;
    snprintf(g_last_err, sizeof(g_last_err), "%s", hipGetErrorString(e));
    return 1;
}

const char* last_launch_error() { return g_last_err; }

__device__ inline float load_table(const void* table, int fmt, size_t idx) {
    if (fmt == WF_BF16) return bf16_to_f32(((const uint16_t*)table)[idx]);
    return ((const float*)table)[idx];
}

__device__ inline float block_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    v = wave_sum_f32(v);
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float s = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) s += red[w];
    return s;
}

// TokenEmbedding::forward (model/src/embedding.rs:26-28) + split sums of
// squares over 128-column groups for the first RMSNorm.
// Fragments + 16-column sums of squares of row m of an activation matrix whose
// f32 values are already in `row` (one workgroup per row).
__device__ __forceinline__ void emit_row_fragments(const XFrag& fo, const float* row, int m, int H) {
    if (!fo.buf) return;
    for (int k = threadIdx.x; k < H; k += blockDim.x) frag_put(fo, m, k, row[k]);
    if (fo.ssq)
        for (int q = threadIdx.x; q < (H >> 4); q += blockDim.x) {
            float ss = 0.f;
#pragma unroll
            for (int n = 0; n < 16; n++) ss += row[q * 16 + n] * row[q * 16 + n];
            fo.ssq[(size_t)m * fo.ssq_ld + q] = ss;
        }
}

// The row kernels below keep their row in LDS (dynamic, H floats) for the
// fragment / sum-of-squares pass, so it is not re-read from global memory after
// its stores; the barrier before that pass waits for LDS only.
static constexpr int ROW_LDS_MAX = 16384;  // floats of one row held in LDS (64 KiB)
static constexpr int ROW_U = 8;            // loads a thread issues before the first store

__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__global__ void embed_kernel(const void* table, int fmt, int H, const uint32_t* ids, float* x, XFrag fo) {
    extern __shared__ float rowbuf[];
    const int m = blockIdx.x;
    const size_t base = (size_t)ids[m] * H;
    if (fmt == WF_BF16 && (H & 7) == 0) {
        // 16-byte loads of 8 bf16 values (the row starts 16-byte aligned)
        const int nc = H >> 3;
        const uint4* src = (const uint4*)((const uint16_t*)table + base);
        for (int c0 = threadIdx.x; c0 < nc; c0 += ROW_U * blockDim.x) {
            uint4 v[ROW_U];
#pragma unroll
            for (int u = 0; u < ROW_U; u++) {
                const int c = c0 + u * blockDim.x;
                v[u] = c < nc ? src[c] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < ROW_U; u++) {
                const int c = c0 + u * blockDim.x;
                if (c < nc) {
                    const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
                    float f[8];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        f[2 * j] = __uint_as_float(w[j] << 16);
                        f[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
                    }
                    const float4 lo = make_float4(f[0], f[1], f[2], f[3]), hi = make_float4(f[4], f[5], f[6], f[7]);
                    float4* xo = (float4*)(x + (size_t)m * H + 8 * c);
                    xo[0] = lo;
                    xo[1] = hi;
                    ((float4*)(rowbuf + 8 * c))[0] = lo;
                    ((float4*)(rowbuf + 8 * c))[1] = hi;
                }
            }
        }
        lds_barrier();
        emit_row_fragments(fo, rowbuf, m, H);
        return;
    }
    // ROW_U loads in flight per thread before their stores (the stores to x could
    // alias the table as far as the compiler knows, so it would not reorder them)
    for (int k0 = threadIdx.x; k0 < H; k0 += ROW_U * blockDim.x) {
        float v[ROW_U];
#pragma unroll
        for (int u = 0; u < ROW_U; u++) {
            const int k = k0 + u * blockDim.x;
            v[u] = k < H ? load_table(table, fmt, base + k) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < ROW_U; u++) {
            const int k = k0 + u * blockDim.x;
            if (k < H) {
                x[(size_t)m * H + k] = v[u];
                rowbuf[k] = v[u];
            }
        }
    }
    lds_barrier();
    emit_row_fragments(fo, rowbuf, m, H);
}

int launch_embed(const void* table, int table_fmt, int H, const uint32_t* ids, int M, float* x, const XFrag& fo,
                 hipStream_t stream) {
    if (H > ROW_LDS_MAX) return 2;
    (void)hipGetLastError();
    hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(RW_THREADS), (unsigned)(H * sizeof(float)), stream, table,
                       table_fmt, H, ids, x, fo);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// MtpHead::local_sequence (nn/src/mtp.rs:247-293): row 0 = trunk_norm(anchor),
// rows 1.. = token_norm(embedding(ids)); one workgroup per output row.
__global__ void mtp_prep_kernel(const float* anchor, long long anchor_stride, const void* table, int fmt,
                                const uint32_t* ids, int ids_stride, int L, int H, const float* trunk_w,
                                const float* token_w, float eps, float* x, XFrag fo) {
    extern __shared__ float rowbuf[];  // [H] row, then [H] norm weight
    __shared__ float red[16];
    const int row = blockIdx.x;
    const int seq = row / L, l = row % L;
    float* out = x + (size_t)row * H;
    const float* w = l == 0 ? trunk_w : token_w;
    float ss = 0.f;
    const size_t tbase = l == 0 ? 0 : (size_t)ids[(size_t)seq * ids_stride + l - 1] * H;
    float* wbuf = rowbuf + H;
    // the row and the norm weight in one round trip
    for (int k0 = threadIdx.x; k0 < H; k0 += ROW_U * blockDim.x) {
        float v[ROW_U], wv[ROW_U];
#pragma unroll
        for (int u = 0; u < ROW_U; u++) {
            const int k = k0 + u * blockDim.x;
            v[u] = k >= H ? 0.f : l == 0 ? anchor[(size_t)seq * anchor_stride + k] : load_table(table, fmt, tbase + k);
            wv[u] = k < H ? w[k] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < ROW_U; u++) {
            const int k = k0 + u * blockDim.x;
            if (k < H) {
                rowbuf[k] = v[u];
                wbuf[k] = wv[u];
                ss += v[u] * v[u];
            }
        }
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    for (int k = threadIdx.x; k < H; k += blockDim.x) {
        const float o = rowbuf[k] * inv * wbuf[k];
        out[k] = o;
        rowbuf[k] = o;
    }
    lds_barrier();
    emit_row_fragments(fo, rowbuf, row, H);
}

int launch_mtp_prep(const float* anchor, long long anchor_stride, const void* table, int table_fmt,
                    const uint32_t* ids, int ids_stride, int nseq, int L, int H, const float* trunk_w,
                    const float* token_w, float eps, float* x, const XFrag& fo, hipStream_t stream) {
    if (2 * H > ROW_LDS_MAX) return 2;  // row + norm weight in LDS
    (void)hipGetLastError();
    hipLaunchKernelGGL(mtp_prep_kernel, dim3(nseq * L), dim3(RW_THREADS), (unsigned)(2 * H * sizeof(float)), stream,
                       anchor, anchor_stride,
                       table, table_fmt, ids, ids_stride, L, H, trunk_w, token_w, eps, x, fo);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// RMSNorm of selected rows (nn/src/norm.rs:17-19), plus fragments of the result.
__global__ void norm_rows_kernel(const float* x, RowMap xmap, int H, const float* w, float eps, float* out, XFrag fo) {
    extern __shared__ float rowbuf[];  // [H] row, then [H] norm weight
    __shared__ float red[16];
    const int m = blockIdx.x;
    const float* r = x + row_off(xmap, m);
    float* wbuf = rowbuf + H;
    float ss = 0.f;
    // the row and the norm weight in one round trip
    for (int k0 = threadIdx.x; k0 < H; k0 += ROW_U * blockDim.x) {
        float v[ROW_U], wv[ROW_U];
#pragma unroll
        for (int u = 0; u < ROW_U; u++) {
            const int k = k0 + u * blockDim.x;
            v[u] = k < H ? r[k] : 0.f;
            wv[u] = k < H ? w[k] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < ROW_U; u++) {
            const int k = k0 + u * blockDim.x;
            if (k < H) {
                rowbuf[k] = v[u];
                wbuf[k] = wv[u];
                ss += v[u] * v[u];
            }
        }
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    for (int k = threadIdx.x; k < H; k += blockDim.x) {
        const float o = rowbuf[k] * inv * wbuf[k];
        out[(size_t)m * H + k] = o;
        rowbuf[k] = o;
    }
    lds_barrier();
    emit_row_fragments(fo, rowbuf, m, H);
}

int launch_norm_rows(const float* x, RowMap xmap, int M, int H, const float* w, float eps, float* out,
                     const XFrag& fo, hipStream_t stream) {
    if (2 * H > ROW_LDS_MAX) return 2;  // row + norm weight in LDS
    (void)hipGetLastError();
    hipLaunchKernelGGL(norm_rows_kernel, dim3(M), dim3(RW_THREADS), (unsigned)(2 * H * sizeof(float)), stream, x, xmap,
                       H, w, eps, out, fo);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// Destination row of source row n inside a fused matrix.  interleave 1/2 puts
// gate/up row f at row row_offset + (f/8)*16 + f%8 (+8 for up) so a 16-row tile
// holds 8 matching gate and up rows.  interleave = hd (>= 16) pairs RoPE dims within a
// head of hd rows: tile j of the head holds dims 8j..8j+7 (rows 0-7) and
// hd/2 + 8j.. (rows 8-15), so the rotation of a pair stays inside one tile.
__device__ __forceinline__ int dest_row(int n, int row_offset, int interleave) {
    if (interleave == 0) return row_offset + n;
    if (interleave >= 16) {
        const int hd = interleave, half = hd >> 1;
        const int head = n / hd, d = n % hd;
        const int p = ((d % half) >> 3) * 16 + (d & 7) + (d >= half ? 8 : 0);
        return row_offset + head * hd + p;
    }
    return row_offset + (n >> 3) * 16 + (n & 7) + (interleave == 2 ? 8 : 0);
}

// INT4 g128 quantisation (quant/src/int4.rs:7-41, codes from the f32 scale,
// scale/zero stored fp16) straight into the tiled layout.  One wave per
// (row, group); lane l holds columns 2l, 2l+1.
__global__ void quant_int4_kernel(const float* w, int N, int K, uint8_t* tiled, uint32_t* sz,
                                  int row_offset, int interleave) {
    const int G = K >> 7;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (wave >= N * G) return;
    const int lane = threadIdx.x & 63;
    const int n = wave / G, g = wave % G;
    const float* src = w + (size_t)n * K + g * 128;
    float v0 = src[2 * lane], v1 = src[2 * lane + 1];
    float mn = fminf(v0, v1), mx = fmaxf(v0, v1);
    for (int d = 32; d >= 1; d >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, d, 64));
        mx = fmaxf(mx, __shfl_xor(mx, d, 64));
    }
    float sc = fabsf(mx - mn) <= FLT_EPSILON ? 1.0f : (mx - mn) / 15.0f;
    float z = roundf(-mn / sc);
    float q0 = fminf(fmaxf(roundf(v0 / sc + z), 0.0f), 15.0f);
    float q1 = fminf(fmaxf(roundf(v1 / sc + z), 0.0f), 15.0f);
    const int dn = dest_row(n, row_offset, interleave);
    const int nt = dn >> 4, r = dn & 15;
    const int j = lane >> 4, c2 = lane & 15;  // columns 2*lane = 32*j + 2*c2
    const size_t tile = (size_t)nt * G + g;
    tiled[tile * 1024 + 16 * (j * 16 + r) + c2] = (uint8_t)(((int)q0 & 15) | (((int)q1 & 15) << 4));
    if (lane == 0) {
        uint16_t sh = __builtin_bit_cast(uint16_t, (_Float16)sc);
        uint16_t zh = __builtin_bit_cast(uint16_t, (_Float16)z);
        sz[tile * 16 + r] = (uint32_t)sh | ((uint32_t)zh << 16);
    }
}

// Per-output-row symmetric INT8 (quant/src/qat.rs:155-169), tiled.
__global__ void quant_int8_kernel(const float* w, int N, int K, uint8_t* tiled, float* rscale, int row_offset,
                                  int interleave) {
    __shared__ float red[MT_THREADS / 64];
    const int n = blockIdx.x;
    const float* src = w + (size_t)n * K;
    float mx = 0.f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) mx = fmaxf(mx, fabsf(src[k]));
    mx = wave_max_f32(mx);
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (lane == 0) red[wid] = mx;
    __syncthreads();
    float m = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) m = fmaxf(m, red[i]);
    float sc = m / 127.0f;
    if (m <= FLT_EPSILON) sc = 1.0f;
    const int dn = dest_row(n, row_offset, interleave);
    const int nt = dn >> 4, r = dn & 15, G = K >> 7;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        int g = k >> 7, kk = k & 127, j = kk >> 5, c = kk & 31;
        float q = fminf(fmaxf(roundf(src[k] / sc), -127.0f), 127.0f);
        tiled[((size_t)nt * G + g) * 2048 + tile_byte(j * 16 + r, c)] = (uint8_t)(int8_t)q;
    }
    if (threadIdx.x == 0) rscale[dn] = sc;
}

__global__ void quant_bf16_kernel(const float* w, int N, int K, uint8_t* tiled, int row_offset, int interleave) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K) return;
    const int n = (int)(i / K), k = (int)(i % K);
    const int dn = dest_row(n, row_offset, interleave);
    const int nt = dn >> 4, r = dn & 15, G = K >> 7;
    const int g = k >> 7, kk = k & 127, j = kk >> 5, c = kk & 31;
    *(uint16_t*)(tiled + ((size_t)nt * G + g) * 4096 + tile_byte(j * 16 + r, 2 * c)) = f32_to_bf16_rne(w[i]);
}

__global__ void copy_f32_rows_kernel(const float* w, int N, int K, float* dst, int row_offset, int interleave) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K) return;
    const int n = (int)(i / K), k = (int)(i % K);
    dst[(size_t)dest_row(n, row_offset, interleave) * K + k] = w[i];
}

int launch_quantise_tiled(const float* w, int N, int K, int fmt, uint8_t* tiled, uint32_t* sz, float* rscale,
                          int row_offset, int N_total, int interleave, hipStream_t stream) {
    (void)N_total;
    if (K % 128) return 2;
    if (fmt == WF_INT4) {
        const int waves = N * (K / 128);
        hipLaunchKernelGGL(quant_int4_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, w, N, K, tiled, sz,
                           row_offset, interleave);
    } else if (fmt == WF_INT8) {
        hipLaunchKernelGGL(quant_int8_kernel, dim3(N), dim3(MT_THREADS), 0, stream, w, N, K, tiled, rscale,
                           row_offset, interleave);
    } else if (fmt == WF_BF16) {
        const size_t n = (size_t)N * K;
        hipLaunchKernelGGL(quant_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, w, N, K,
                           tiled, row_offset, interleave);
    } else {
        const size_t n = (size_t)N * K;
        hipLaunchKernelGGL(copy_f32_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, w, N,
                           K, (float*)tiled, row_offset, interleave);
    }
    return note_error(hipGetLastError()) ? 4 : 0;
}

// Reference PackedInt4Tensor layout (row-major, two codes per byte, low
// nibble = even index, int4.rs:45-53) -> tiled layout.  One thread per byte.
__global__ void repack_int4_kernel(const uint8_t* packed, const uint16_t* sc, const uint16_t* zr, int N, int K,
                                   uint8_t* tiled, uint32_t* sz, int row_offset, int interleave) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nbytes = (size_t)N * K / 2;
    if (i >= nbytes) return;
    const int n = (int)(i / (K / 2)), kb = (int)(i % (K / 2));
    const int k = 2 * kb;
    const int dn = dest_row(n, row_offset, interleave);
    const int nt = dn >> 4, r = dn & 15, G = K >> 7;
    const int g = k >> 7, kk = k & 127, j = kk >> 5, c = kk & 31;
    const size_t tile = (size_t)nt * G + g;
    tiled[tile * 1024 + 16 * (j * 16 + r) + (c >> 1)] = packed[i];
    if (kk == 0) sz[tile * 16 + r] = (uint32_t)sc[(size_t)n * G + g] | ((uint32_t)zr[(size_t)n * G + g] << 16);
}

int launch_repack_int4(const uint8_t* packed, const uint16_t* sc, const uint16_t* zr, int N, int K, uint8_t* tiled,
                       uint32_t* sz, int row_offset, int N_total, int interleave, hipStream_t stream) {
    (void)N_total;
    const size_t nb = (size_t)N * K / 2;
    (void)hipGetLastError();
    hipLaunchKernelGGL(repack_int4_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, stream, packed, sc, zr,
                       N, K, tiled, sz, row_offset, interleave);
    return note_error(hipGetLastError()) ? 4 : 0;
}

__global__ void repack_int8_kernel(const int8_t* codes, const float* sc, int N, int K, uint8_t* tiled, float* rscale,
                                   int row_offset, int interleave) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K) return;
    const int n = (int)(i / K), k = (int)(i % K);
    const int dn = dest_row(n, row_offset, interleave);
    const int nt = dn >> 4, r = dn & 15, G = K >> 7;
    const int g = k >> 7, kk = k & 127, j = kk >> 5, c = kk & 31;
    tiled[((size_t)nt * G + g) * 2048 + tile_byte(j * 16 + r, c)] = (uint8_t)codes[i];
    if (k == 0) rscale[dn] = sc[n];
}

int launch_repack_int8(const int8_t* codes, const float* sc, int N, int K, uint8_t* tiled, float* rscale,
                       int row_offset, int N_total, int interleave, hipStream_t stream) {
    (void)N_total;
    const size_t n = (size_t)N * K;
    (void)hipGetLastError();
    hipLaunchKernelGGL(repack_int8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, codes, sc, N, K,
                       tiled, rscale, row_offset, interleave);
    return note_error(hipGetLastError()) ? 4 : 0;
}

__global__ void synth_fill_kernel(float* out, long long n, unsigned long long seed, unsigned stream, float std) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = (float)((double)synth_normal(seed, stream, (uint64_t)i) * (double)std);
}

int launch_synth_fill(float* out, long long n, unsigned long long seed, unsigned stream_id, float std,
                      hipStream_t stream) {
    (void)hipGetLastError();
    hipLaunchKernelGGL(synth_fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, out, n, seed,
                       stream_id, std);
    return note_error(hipGetLastError()) ? 4 : 0;
}

__global__ void to_bf16_kernel(const float* src, uint16_t* dst, long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = f32_to_bf16_rne(src[i]);
}

int launch_to_bf16(const float* src, uint16_t* dst, long long n, hipStream_t stream) {
    (void)hipGetLastError();
    hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, src, dst, n);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// Synthetic post-RoPE K/V contents for long-context benchmarks; one wave per
// (token, kv head, K|V).  Same values as the oracle's ref_kv_fill_synthetic.
__global__ void kv_fill_kernel(void* kc, void* vc, uint16_t* ks, uint16_t* vs, int kv_fmt, int slot, int n_kv,
                               int hd, int cap, int len, unsigned long long seed, int layer) {
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (wave >= len * n_kv * 2) return;
    const int lane = threadIdx.x & 63;
    const int which = wave & 1;
    const int th = wave >> 1;
    const int t = th / n_kv, h = th % n_kv;
    const uint32_t stream = 0x4B560000u + (uint32_t)(layer * 2 + which);
    const uint64_t off = ((uint64_t)t * n_kv + h) * hd;
    float v0 = lane < hd ? synth_normal(seed, stream, off + lane) : 0.f;
    float v1 = lane + 64 < hd ? synth_normal(seed, stream, off + lane + 64) : 0.f;
    const size_t hb = (size_t)slot * n_kv + h;
    if (kv_fmt == KV_INT8) {
        float amax = wave_max_f32(fmaxf(fabsf(v0), fabsf(v1)));
        float sc = amax <= FLT_EPSILON ? 1.0f : amax / 127.0f;
        int8_t q0 = (int8_t)fminf(fmaxf(roundf(v0 / sc), -127.f), 127.f);
        int8_t q1 = (int8_t)fminf(fmaxf(roundf(v1 / sc), -127.f), 127.f);
        uint16_t sh = __builtin_bit_cast(uint16_t, (_Float16)sc);
        if (which == 0) {
            int8_t* dst = (int8_t*)kc;
            if (lane < hd) dst[k_off(hb, t, lane, cap, hd, KV_INT8)] = q0;
            if (lane + 64 < hd) dst[k_off(hb, t, lane + 64, cap, hd, KV_INT8)] = q1;
            if (lane == 0) ks[hb * cap + t] = sh;
        } else {
            int8_t* dst = (int8_t*)vc;
            if (lane < hd) dst[vt_off(hb, lane, t, cap, hd, KV_INT8)] = q0;
            if (lane + 64 < hd) dst[vt_off(hb, lane + 64, t, cap, hd, KV_INT8)] = q1;
            if (lane == 0) vs[hb * cap + t] = sh;
        }
    } else if (kv_fmt == KV_F16) {
        if (which == 0) {
            _Float16* dst = (_Float16*)kc;
            if (lane < hd) dst[k_off(hb, t, lane, cap, hd, KV_F16)] = (_Float16)v0;
            if (lane + 64 < hd) dst[k_off(hb, t, lane + 64, cap, hd, KV_F16)] = (_Float16)v1;
        } else {
            _Float16* dst = (_Float16*)vc;
            if (lane < hd) dst[vt_off(hb, lane, t, cap, hd, KV_F16)] = (_Float16)v0;
            if (lane + 64 < hd) dst[vt_off(hb, lane + 64, t, cap, hd, KV_F16)] = (_Float16)v1;
        }
    } else {
        if (which == 0) {
            float* dst = (float*)kc + (hb * cap + t) * hd;
            if (lane < hd) dst[lane] = v0;
            if (lane + 64 < hd) dst[lane + 64] = v1;
        } else {
            float* dst = (float*)vc + hb * hd * cap + t;
            if (lane < hd) dst[(size_t)lane * cap] = v0;
            if (lane + 64 < hd) dst[(size_t)(lane + 64) * cap] = v1;
        }
    }
}

int launch_kv_fill_synthetic(void* kc, void* vc, uint16_t* ks, uint16_t* vs, int kv_fmt, int slot, int n_kv, int hd,
                             int cap, int len, unsigned long long seed, int layer, hipStream_t stream) {
    const int waves = len * n_kv * 2;
    if (waves == 0) return 0;
    (void)hipGetLastError();
    hipLaunchKernelGGL(kv_fill_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, kc, vc, ks, vs, kv_fmt, slot,
                       n_kv, hd, cap, len, seed, layer);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// argmax under f32::total_cmp keeping the last maximal index (sampler.rs:217-224),
// plus the top-2 value gap (greedy near-tie measure).
__global__ void argmax_rows_kernel(const float* x, long long ld, int V, int32_t* out, int out_stride, float* gap) {
    __shared__ int rk[16], ri[16];
    __shared__ float r1[16], r2[16];
    const float* row = x + (size_t)blockIdx.x * ld;
    int bk = INT_MIN, bi = 0;
    float t1 = -INFINITY, t2 = -INFINITY;
    // WIDE_U loads in flight per thread, then consumed in index order
    for (int j0 = threadIdx.x; j0 < V; j0 += WIDE_U * blockDim.x) {
        float vv[WIDE_U];
#pragma unroll
        for (int u = 0; u < WIDE_U; u++) {
            const int j = j0 + u * blockDim.x;
            vv[u] = j < V ? row[j] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < WIDE_U; u++) {
            const int j = j0 + u * blockDim.x;
            if (j < V) {
                const float v = vv[u];
                const int k = total_key(v);
                if (k >= bk) { bk = k; bi = j; }
                if (v > t1) { t2 = t1; t1 = v; } else if (v > t2) { t2 = v; }
            }
        }
    }
    for (int d = 32; d >= 1; d >>= 1) {
        int ok = __shfl_xor(bk, d, 64), oi = __shfl_xor(bi, d, 64);
        if (ok > bk || (ok == bk && oi > bi)) { bk = ok; bi = oi; }
        float o1 = __shfl_xor(t1, d, 64), o2 = __shfl_xor(t2, d, 64);
        float n1 = fmaxf(t1, o1);
        float n2 = fmaxf(fminf(t1, o1), fmaxf(t2, o2));
        t1 = n1; t2 = n2;
    }
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (lane == 0) { rk[wid] = bk; ri[wid] = bi; r1[wid] = t1; r2[wid] = t2; }
    __syncthreads();
    if (threadIdx.x == 0) {
        int k0 = rk[0], i0 = ri[0];
        float a1 = r1[0], a2 = r2[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) {
            if (rk[w] > k0 || (rk[w] == k0 && ri[w] > i0)) { k0 = rk[w]; i0 = ri[w]; }
            float n1 = fmaxf(a1, r1[w]);
            float n2 = fmaxf(fminf(a1, r1[w]), fmaxf(a2, r2[w]));
            a1 = n1; a2 = n2;
        }
        out[(size_t)blockIdx.x * out_stride] = i0;
        if (gap) gap[blockIdx.x] = a1 - a2;
    }
}

int launch_argmax_rows(const float* x, long long ld, int rows, int V, int32_t* out, int out_stride, float* gap,
                       hipStream_t stream) {
    (void)hipGetLastError();
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(WIDE_THREADS), 0, stream, x, ld, V, out, out_stride, gap);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// Row copies given as device arrays of (src, dst) pointers: one workgroup per row.
__global__ void copy_rows_kernel(const float* const* src, float* const* dst, int n) {
    const float* s = src[blockIdx.x];
    float* d = dst[blockIdx.x];
    for (int k0 = threadIdx.x; k0 < n; k0 += WIDE_U * blockDim.x) {
        float v[WIDE_U];
#pragma unroll
        for (int u = 0; u < WIDE_U; u++) {
            const int k = k0 + u * blockDim.x;
            v[u] = k < n ? s[k] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < WIDE_U; u++) {
            const int k = k0 + u * blockDim.x;
            if (k < n) d[k] = v[u];
        }
    }
}

int launch_copy_rows(const float* const* src, float* const* dst, int rows, int n, hipStream_t stream) {
    if (rows <= 0) return 0;
    (void)hipGetLastError();
    hipLaunchKernelGGL(copy_rows_kernel, dim3(rows), dim3(WIDE_THREADS), 0, stream, src, dst, n);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// Verify rows of a greedy MTP round (mtp_speculative.rs:211-221): row r of sequence b
// carries proposal min(r, K - 1) (rows past the proposals repeat the last one), and
// nprop[b] counts the proposals up to and including the first end-of-sequence id, at
// most limit[b] (0 for a finished sequence) -- the proposal loop of
// mtp_speculative.rs:169-209 that stops after an EOS proposal (:201-203).
__global__ void mtp_verify_rows_kernel(const uint32_t* props, int K, int Kr, int nseq, const int32_t* limit,
                                       uint32_t eos, uint32_t* ids, int32_t* nprop, const uint64_t* obase,
                                       uint64_t* offs) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nseq * Kr) return;
    const int b = i / Kr, r = i - b * Kr;
    ids[i] = props[(size_t)b * K + min(r, K - 1)];
    if (r == 0) {
        const int lim = min(limit[b], K);
        int np = 0;
        for (int p = 0; p < lim; p++) {
            np++;
            if (props[(size_t)b * K + p] == eos) break;
        }
        nprop[b] = np;
        // sampled rounds: the acceptance draws start after the np proposal draws
        if (offs) offs[b] = obase[b] + (uint64_t)np;
    }
}

int launch_mtp_verify_rows(const uint32_t* props, int K, int Kr, int nseq, const int32_t* limit, uint32_t eos,
                           uint32_t* ids, int32_t* nprop, const uint64_t* obase, uint64_t* offs, hipStream_t stream) {
    if (nseq <= 0 || Kr <= 0 || K <= 0 || (offs && !obase)) return 2;
    (void)hipGetLastError();
    hipLaunchKernelGGL(mtp_verify_rows_kernel, dim3((nseq * Kr + 255) / 256), dim3(256), 0, stream, props, K, Kr,
                       nseq, limit, eos, ids, nprop, obase, offs);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// Sampled MTP proposal p (mtp_speculative.rs:169-209): the token the sampling kernel
// drew for each sequence goes to props[b * K + p] (0 when its distribution was
// invalid).  A sequence whose proposal p counts -- p < limit[b] and no earlier
// proposal of the round is the end-of-sequence id, after which the reference stops
// proposing (:196-203) -- and whose distribution was invalid is flagged in pstat[b]
// (set at p = 0, accumulated after), which the host checks with the round's one
// read-back (sample_probabilities returns Err, sampler.rs:142-152).
__global__ void sampled_props_kernel(const int32_t* tok, const int32_t* status, uint32_t* props, int K, int p,
                                     int nseq, const int32_t* limit, uint32_t eos, int32_t* pstat) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nseq) return;
    const bool bad = status[b] != 0;
    props[(size_t)b * K + p] = bad ? 0u : (uint32_t)tok[b];
    bool after_eos = false;
    for (int j = 0; j < p; j++) after_eos |= props[(size_t)b * K + j] == eos;
    const int32_t flag = (bad && p < limit[b] && !after_eos) ? 1 : 0;
    pstat[b] = p == 0 ? flag : (pstat[b] | flag);
}

int launch_sampled_props(const int32_t* tok, const int32_t* status, uint32_t* props, int K, int p, int nseq,
                         const int32_t* limit, uint32_t eos, int32_t* pstat, hipStream_t stream) {
    if (nseq <= 0 || K <= 0 || p < 0 || p >= K) return 2;
    (void)hipGetLastError();
    hipLaunchKernelGGL(sampled_props_kernel, dim3((nseq + 255) / 256), dim3(256), 0, stream, tok, status, props, K, p,
                       nseq, limit, eos, pstat);
    return note_error(hipGetLastError()) ? 4 : 0;
}

__global__ void fill_f32_kernel(float* p, long long n, float v) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

int launch_fill_f32(float* p, long long n, float v, hipStream_t stream) {
    if (n <= 0) return 0;
    (void)hipGetLastError();
    hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p, n, v);
    return note_error(hipGetLastError()) ? 4 : 0;
}

}  // namespace aarh
