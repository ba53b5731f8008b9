// Quantised skinny GEMM for the verify forward on gfx950.
//
// Replaces QatLinear::forward (quant/src/qat.rs:315-348), i.e. y = x . W^T
// for every projection of the verify forward (attention.rs:170-222,
// ffn.rs:29-37, head.rs:47-49), with the weights kept quantised in HBM.
//
// Layout: W [N, K] is stored as 16-row x 128-column tiles, tile (nt, g) is a
// contiguous block (1 KiB INT4, 2 KiB INT8, 4 KiB BF16) in which lane l of a
// wave owns row l%16, columns 32*(l/16)..+32 of the group: one 16/32/64-byte
// load per lane, fully coalesced.  INT4 scale and zero (fp16) sit beside the
// tiles, one u32 per (tile, group, row).
//
// Work split: one workgroup (4 waves) per 16-row tile and the whole K; wave w
// takes groups w, w+4, ...  Nothing is exchanged between workgroups: the four
// wave partials are added in LDS in a fixed order and the workgroup runs the
// fused epilogue on its 16 output columns (store, residual add, SwiGLU of the
// 8 gate + 8 up rows of the tile, or RoPE of the 8 (d, d + hd/2) pairs of the
// tile + query / new K,V rows out).
//
// Compute: weights are dequantised in registers to EXACT fp16 integers (q - z
// for INT4, the code for INT8, magic-number 0x6400 conversion) or used as
// bf16.  Activations are read as f32 straight from L2 and split into fp16
// (bf16) hi + lo halves; both halves multiply the same weight fragment
// (two MFMAs), so products keep ~22 bits.  The INT4 group scale multiplies the
// fp32 group accumulator.  RMSNorm is fused: the workgroup multiplies x by the
// norm weight before the MFMA, accumulates sum(x^2) over the rows it reads
// (the full K) and scales the result rows by 1/rms at the end.
#include <float.h>

#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"
#include "frag.hpp"

namespace aarh {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

static constexpr int GT_NW = 8;         // waves per workgroup of the fragment GEMV
static constexpr int GT_PF = 4;         // its prefetch ring depth (items per wave)
static constexpr int GT_THREADS = 256;  // f32 GEMV workgroup
static constexpr int GT_MROWS = 16;     // activation rows per launch (one MFMA row tile)

template <int FMT>
struct FmtTraits;
template <>
struct FmtTraits<WF_INT4> {
    static constexpr int TILE_BYTES = 1024, LANE_WORDS = 4, PF = 8;
};
template <>
struct FmtTraits<WF_INT8> {
    static constexpr int TILE_BYTES = 2048, LANE_WORDS = 8, PF = 4;
};
template <>
struct FmtTraits<WF_BF16> {
    static constexpr int TILE_BYTES = 4096, LANE_WORDS = 16, PF = 2;
};

// Element of an 8-column block that k-slot j of an operand holds: the order in
// which the weight dequantisation below emits B elements.
template <int FMT>
__device__ __forceinline__ constexpr int slot_elem(int j) {
    if (FMT == WF_INT4) return (j >> 1) | ((j & 1) << 2);
    if (FMT == WF_INT8) return (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1);
    return j;
}

__device__ __forceinline__ half8_t int4_b_operand(uint32_t v, half2_t zz) {
    uint32_t p0 = (v & 0x000F000Fu) | 0x64006400u;
    uint32_t p1 = ((v >> 4) & 0x000F000Fu) | 0x64006400u;
    uint32_t p2 = ((v >> 8) & 0x000F000Fu) | 0x64006400u;
    uint32_t p3 = ((v >> 12) & 0x000F000Fu) | 0x64006400u;
    half2_t h0 = __builtin_bit_cast(half2_t, p0) - zz;
    half2_t h1 = __builtin_bit_cast(half2_t, p1) - zz;
    half2_t h2 = __builtin_bit_cast(half2_t, p2) - zz;
    half2_t h3 = __builtin_bit_cast(half2_t, p3) - zz;
    half8_t r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

__device__ __forceinline__ half8_t int8_b_operand(uint32_t d0, uint32_t d1) {
    const half2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    d0 ^= 0x80808080u;
    d1 ^= 0x80808080u;
    half2_t h0 = __builtin_bit_cast(half2_t, (d0 & 0x00FF00FFu) | 0x64006400u) - off;
    half2_t h1 = __builtin_bit_cast(half2_t, ((d0 >> 8) & 0x00FF00FFu) | 0x64006400u) - off;
    half2_t h2 = __builtin_bit_cast(half2_t, (d1 & 0x00FF00FFu) | 0x64006400u) - off;
    half2_t h3 = __builtin_bit_cast(half2_t, ((d1 >> 8) & 0x00FF00FFu) | 0x64006400u) - off;
    half8_t r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

// ---------------------------------------------------------------------------
// Epilogues on the reduced tile yt[m][n] (m < Mc activation rows of this
// chunk, n < 16 output columns nt*16 + n).
// ---------------------------------------------------------------------------
// Threads t0, t0 + stride, ... of the caller share the work; wave_only: the
// caller is a single wave (no workgroup barrier may be used).
template <int EPI>
__device__ void run_epilogue(const GemvArgs& a, float (*yt)[17], int nt, int Mc, int t0, int stride, bool wave_only) {
    const int tid = t0;
    if (EPI == EPI_STORE) {
        for (int idx = tid; idx < Mc * 16; idx += stride) {
            const int m = idx >> 4, n = idx & 15;
            a.out[row_off(a.omap, a.m_base + m) + nt * 16 + n] = yt[m][n];
        }
    } else if (EPI == EPI_RESID) {
        // x += y, and the new x as fragments + 16-column sums of squares for the next RMSNorm
        for (int idx = tid; idx < Mc * 16; idx += stride) {
            const int m = idx >> 4, n = idx & 15;
            float* p = a.resid + (size_t)(a.m_base + m) * a.ldr + nt * 16 + n;
            const float xn = *p + yt[m][n];
            *p = xn;
            yt[m][n] = xn;
            if (a.fo.buf) frag_put(a.fo, a.m_base + m, nt * 16 + n, xn);
        }
        if (a.fo.ssq) {
            if (wave_only) {
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's LDS writes are done
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
            } else {
                __syncthreads();
            }
            if (tid < Mc) {
                float ss = 0.f;
#pragma unroll
                for (int n = 0; n < 16; n++) ss += yt[tid][n] * yt[tid][n];
                a.fo.ssq[(size_t)nt * a.fo.ssq_rows + a.m_base + tid] = ss;
            }
        }
    } else if (EPI == EPI_SWIGLU) {
        // rows 0-7 of the tile are gate rows, 8-15 the matching up rows (ffn columns nt*8 + r)
        for (int idx = tid; idx < Mc * 8; idx += stride) {
            const int m = idx >> 3, r = idx & 7;
            const float g = yt[m][r], u = yt[m][8 + r];
            const float silu = g / (1.0f + expf(-g));
            const float h = silu * u;
            a.out[row_off(a.omap, a.m_base + m) + nt * 8 + r] = h;
            if (a.fo.buf) frag_put(a.fo, a.m_base + m, nt * 8 + r, h);
        }
    } else {
        // QKV: the tile holds dims d = 8j + r (rows r < 8) and d + hd/2 (rows 8 + r) of one head.
        const QkvEpi& e = a.qkv;
        const int hd = e.hd, half = hd >> 1;
        const int QD = e.n_heads * hd, KD = e.n_kv * hd;
        const int row0 = nt * 16;
        const int head = row0 / hd, j = (row0 % hd) >> 4;
        const bool is_q = row0 < QD, is_k = !is_q && row0 < QD + KD;
        for (int idx = tid; idx < Mc * 8; idx += stride) {
            const int m = idx >> 3, r = idx & 7;
            const int mg = a.m_base + m;
            const int d1 = 8 * j + r, d2 = d1 + half;
            float y1 = yt[m][r], y2 = yt[m][8 + r];
            if (is_q || is_k) {
                // RoPE (rope.rs:107-126): half-split rotation at the row's position
                const int bs = mg / e.S, s = mg % e.S;
                const int pos = e.pos0[bs] + s;
                const float cs = e.rope_cos[(size_t)pos * half + d1], sn = e.rope_sin[(size_t)pos * half + d1];
                {
#pragma clang fp contract(off)
                    const float r1 = y1 * cs - y2 * sn;
                    const float r2 = y1 * sn + y2 * cs;
                    y1 = r1;
                    y2 = r2;
                }
            }
            float* dst;
            if (is_q) dst = e.q_out + (size_t)mg * QD + head * hd;
            else if (is_k) dst = e.kv_out + (size_t)mg * 2 * KD + (head - e.n_heads) * hd;
            else dst = e.kv_out + (size_t)mg * 2 * KD + KD + (head - e.n_heads - e.n_kv) * hd;
            dst[d1] = y1;
            dst[d2] = y2;
        }
    }
}

// Quantised GEMV over fragment inputs, persistent over 16-row weight tiles:
// workgroup b takes tiles b, b + grid, ...; wave w of the NW waves takes the
// groups w, w + NW, ... of each tile (ngp items per tile, padded to the ring
// depth PF; padding items are skipped).  A ring of PF slots holds, per item,
// the weight tile words and the lane's activation fragment entries, so weights
// (HBM) and fragments (L2) of the next PF items are in flight while one is
// computed, across tile boundaries.  Loads are buffer loads with wave-uniform
// offsets, issued unconditionally (indices clamped into range); only the
// arithmetic depends on whether a group is real: conditional loads would be
// merged with register copies that wait for ALL outstanding loads.
//
// No workgroup barrier inside the stream: at the end of a tile each wave
// leaves its partial in an LDS slot (two slots, by tile parity) and the last
// wave to arrive (LDS counter) adds the NW partials in wave order and runs
// the epilogue alone while the others go on.  A wave waits before reusing a
// slot until the epilogue two tiles back has released it.
template <int FMT, int MP, int EPI>
__global__ void __launch_bounds__(GT_NW * 64) gemv_tile_kernel(GemvArgs a) {
    constexpr int NW = GT_NW;
    constexpr bool RS = MP <= 8;        // hi / lo in MFMA rows
    constexpr int EA = RS ? 1 : 2;      // fragment entries per k-step per lane
    constexpr int EPB = RS ? 2 * MP : 32;
    typedef FmtTraits<FMT> T;
    constexpr int PF = GT_PF;
    __shared__ float4_t part_s[2][NW][64];
    __shared__ float yt_s[2][16][17];
    __shared__ float s_inv[16];
    __shared__ unsigned cnt_s[2], gen_s[2];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int G = a.K >> 7;
    const int Mc = a.M;
    const int ntiles = a.N >> 4;
    const int ngp = ((G + NW - 1) / NW + PF - 1) / PF * PF;  // items per tile per wave
    const int nmine = (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int mt = a.m_base >> 4;
    const int elane = RS ? min(lr, 2 * MP - 1) : 2 * lr;  // fragment entry of this lane
    const int glast = G - 1 - ((G - 1 - wid) % NW + NW) % NW;  // last real group of this wave (may be < 0)

    // ---- 1/rms of each row from the producer's 16-column partial sums ----
    if (tid < 2) {
        cnt_s[tid] = 0u;
        gen_s[tid] = 0u;
    }
    if (a.norm_w) {
        for (int m = wid; m < Mc; m += NW) {
            float ss = 0.f;
            for (int q = lane; q < (a.K >> 4); q += 64) ss += a.ssq_in[(size_t)q * a.ssq_rows + a.m_base + m];
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, 64);
            if (lane == 0) s_inv[m] = 1.0f / sqrtf(ss / (float)a.K + a.eps);
        }
    }
    __syncthreads();
    if (nmine <= 0) return;

    const __amdgpu_buffer_rsrc_t wr = coh_rsrc(a.w), fr = coh_rsrc(a.xf), zr = coh_rsrc(a.sz);
    const unsigned w_voff = (unsigned)lane * T::LANE_WORDS * 4u;
    const unsigned f_voff = (unsigned)(lg * EPB + elane) * 16u;
    const unsigned z_voff = (unsigned)lr * 4u;
    uint32_t wv[PF][T::LANE_WORDS];
    uint32_t szv[PF];
    uint4 av[PF][4][EA];
    // item (tile tl, slot gi) of this wave -> ring slot p
    auto load_item = [&](int p, int tl, int gi) {
        const int g = max(min(wid + NW * gi, glast), 0);
        const unsigned tile = (unsigned)((int)blockIdx.x + tl * (int)gridDim.x) * G + g;
        const int w_soff = (int)(tile * T::TILE_BYTES);
#pragma unroll
        for (int q = 0; q < T::LANE_WORDS / 4; q++) {
            const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)(w_voff + 16u * q), w_soff, 2));
            wv[p][4 * q + 0] = v[0];
            wv[p][4 * q + 1] = v[1];
            wv[p][4 * q + 2] = v[2];
            wv[p][4 * q + 3] = v[3];
        }
        if (FMT == WF_INT4) szv[p] = __builtin_amdgcn_raw_buffer_load_b32(zr, (int)z_voff, (int)(tile * 64u), 0);
        const int f_soff = (int)(((unsigned)mt * G + g) * 16u * EPB * 16u);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int e = 0; e < EA; e++)
                av[p][t][e] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                             fr, (int)(f_voff + 16u * e), f_soff + t * 4 * EPB * 16, 0));
    };
#pragma unroll
    for (int p = 0; p < PF; p++) load_item(p, 0, p);

    for (int tl = 0; tl < nmine; tl++) {
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
        for (int gi0 = 0; gi0 < ngp; gi0 += PF) {
            // items PF ahead: same tile, or the first slots of the next one (last tile: clamped)
            const bool wrap = gi0 + PF >= ngp;
            const int rtl = wrap ? min(tl + 1, nmine - 1) : tl;
            const int rgi0 = wrap ? 0 : gi0 + PF;
#pragma unroll
            for (int p = 0; p < PF; p++) {
                const int gi = gi0 + p;
                if (wid + NW * gi < G) {
                    if (FMT == WF_INT4) {
                        const uint32_t szw = szv[p];
                        const _Float16 zh = __builtin_bit_cast(_Float16, (uint16_t)(szw >> 16));
                        const float sc = (float)__builtin_bit_cast(_Float16, (uint16_t)(szw & 0xFFFFu));
                        const _Float16 zz = (_Float16)1024.0f + zh;
                        const half2_t zz2 = {zz, zz};
                        float4_t g4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int t = 0; t < 4; t++) {
                            const half8_t b = int4_b_operand(wv[p][t], zz2);
#pragma unroll
                            for (int e = 0; e < EA; e++)
                                g4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, av[p][t][e]), b, g4, 0, 0, 0);
                        }
                        acc += sc * g4;
                    } else if (FMT == WF_INT8) {
#pragma unroll
                        for (int t = 0; t < 4; t++) {
                            const half8_t b = int8_b_operand(wv[p][2 * t], wv[p][2 * t + 1]);
#pragma unroll
                            for (int e = 0; e < EA; e++)
                                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, av[p][t][e]), b, acc, 0, 0, 0);
                        }
                    } else {
#pragma unroll
                        for (int t = 0; t < 4; t++) {
                            const u32x4_t w4 = {wv[p][4 * t], wv[p][4 * t + 1], wv[p][4 * t + 2], wv[p][4 * t + 3]};
                            const bf16x8_t b = __builtin_bit_cast(bf16x8_t, w4);
#pragma unroll
                            for (int e = 0; e < EA; e++)
                                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[p][t][e]), b, acc, 0, 0, 0);
                        }
                    }
                }
                load_item(p, rtl, rgi0 + p);
            }
        }
        // ---- end of tile tl: partial -> slot, the last wave reduces + epilogue ----
        const int ps = tl & 1;
        while (__hip_atomic_load(&gen_s[ps], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != (unsigned)(tl >> 1))
            __builtin_amdgcn_s_sleep(1);
        part_s[ps][wid][lane] = acc;
        unsigned old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(&cnt_s[ps], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
        old = __shfl(old, 0, 64);
        if (old == NW - 1) {
            const int nt = (int)blockIdx.x + tl * (int)gridDim.x;
            float4_t sum = part_s[ps][0][lane];
#pragma unroll
            for (int w = 1; w < NW; w++) sum += part_s[ps][w][lane];
            float (*yt)[17] = yt_s[ps];
#pragma unroll
            for (int i = 0; i < 4; i++) yt[4 * lg + i][lr] = sum[i];
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            float y[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int idx = lane + 64 * q, m = idx >> 4, n = idx & 15;
                y[q] = 0.f;
                if (m < Mc) {
                    float v = RS ? yt[m][n] + yt[MP + m][n] : yt[m][n];
                    if (a.norm_w) v *= s_inv[m];
                    if (FMT == WF_INT8) v *= a.rscale[nt * 16 + n];
                    y[q] = v;
                }
            }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int idx = lane + 64 * q, m = idx >> 4, n = idx & 15;
                if (m < Mc) yt[m][n] = y[q];
            }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (EPI == EPI_STORE && a.hidden_out && nt == 0) {
                // final normed hidden state (model.rs:579-585), written once by tile 0
                for (int idx = lane; idx < Mc * a.K; idx += 64) {
                    const int m = idx / a.K, k = idx - m * a.K;
                    const float v = a.x[row_off(a.xmap, a.m_base + m) + k];
                    a.hidden_out[(size_t)(a.m_base + m) * a.K + k] = v * s_inv[m] * a.norm_w[k];
                }
            }
            run_epilogue<EPI>(a, yt, nt, Mc, lane, 64, true);
            if (lane == 0) {
                __hip_atomic_store(&cnt_s[ps], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                __hip_atomic_fetch_add(&gen_s[ps], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
    }
}

// Plain fp32 weights (the reference's CPU dtype, row-major, rows in the same
// order as the tiled formats): fp32 FMA dot products on the vector ALUs, one
// workgroup per 16-row tile; thread (r, c) owns weight row r and activation
// rows c, c+16, ...; x is staged in LDS 128 columns at a time.
__global__ void __launch_bounds__(GT_THREADS) gemv_f32_kernel(GemvArgs a) {
    __shared__ float xs[GT_MROWS][128 + 1];
    __shared__ float red[4][GT_MROWS][17];
    __shared__ float s_ssq[4][GT_MROWS];
    __shared__ float yt[GT_MROWS][17];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int nt = blockIdx.x;
    const int Mc = a.M;
    const int r = tid >> 4, c = tid & 15;
    const float* W = (const float*)a.w + (size_t)(nt * 16 + r) * a.K;
    float acc[2] = {0.f, 0.f};
    float ssq_part = 0.f;
    for (int k0 = 0; k0 < a.K; k0 += 128) {
        __syncthreads();
        for (int idx = tid; idx < Mc * 128; idx += GT_THREADS) {
            const int m = idx >> 7, k = idx & 127;
            const float v = a.x[row_off(a.xmap, a.m_base + m) + k0 + k];
            xs[m][k] = a.norm_w ? v * a.norm_w[k0 + k] : v;
        }
        // sum of squares of the raw rows: wave w covers rows w, w+4, ...
        if (a.norm_w) {
            for (int m = wid; m < Mc; m += 4) {
                const float* xr = a.x + row_off(a.xmap, a.m_base + m) + k0;
                const float v0 = xr[lane], v1 = xr[64 + lane];
                const float s = wave_sum_f32(v0 * v0 + v1 * v1);
                if (lane == 0) s_ssq[0][m] = (k0 == 0 ? 0.f : s_ssq[0][m]) + s;
            }
        }
        __syncthreads();
#pragma unroll
        for (int mi = 0; mi < GT_MROWS / 16; mi++) {
            const int m = c + 16 * mi;
            if (m < Mc) {
                float s = acc[mi];
                for (int k = 0; k < 128; k++) s = fmaf(W[k0 + k], xs[m][k], s);
                acc[mi] = s;
            }
        }
    }
    (void)ssq_part;
    __syncthreads();
#pragma unroll
    for (int mi = 0; mi < 1; mi++) {
        const int m = c + 16 * mi;
        if (m < Mc) {
            float y = acc[mi];
            if (a.norm_w) y *= 1.0f / sqrtf(s_ssq[0][m] / (float)a.K + a.eps);
            yt[m][r] = y;
        }
    }
    if (a.hidden_out && nt == 0) {
        for (int idx = tid; idx < Mc * a.K; idx += GT_THREADS) {
            const int m = idx / a.K, k = idx - m * a.K;
            const float inv = 1.0f / sqrtf(s_ssq[0][m] / (float)a.K + a.eps);
            const float v = a.x[row_off(a.xmap, a.m_base + m) + k];
            a.hidden_out[(size_t)(a.m_base + m) * a.K + k] = v * inv * a.norm_w[k];
        }
    }
    (void)red;
    __syncthreads();
    switch (a.epi) {
        case EPI_STORE: run_epilogue<EPI_STORE>(a, yt, nt, Mc, threadIdx.x, GT_THREADS, false); break;
        case EPI_RESID: run_epilogue<EPI_RESID>(a, yt, nt, Mc, threadIdx.x, GT_THREADS, false); break;
        case EPI_SWIGLU: run_epilogue<EPI_SWIGLU>(a, yt, nt, Mc, threadIdx.x, GT_THREADS, false); break;
        default: run_epilogue<EPI_QKV>(a, yt, nt, Mc, threadIdx.x, GT_THREADS, false); break;
    }
}

template <int FMT, int MP, int EPI>
static int launch_tile(const GemvArgs& a, hipStream_t stream) {
    static int grid_cap = 0;
    if (!grid_cap) {
        int dev = 0, cus = 0, per_cu = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)gemv_tile_kernel<FMT, MP, EPI>,
                                                           GT_NW * 64, 0);
        grid_cap = std::max(1, cus) * std::max(1, per_cu);
    }
    const int grid = std::min(a.N / 16, grid_cap);
    (void)hipGetLastError();
    hipLaunchKernelGGL((gemv_tile_kernel<FMT, MP, EPI>), dim3(grid), dim3(GT_NW * 64), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

template <int FMT, int MP>
static int launch_epi(const GemvArgs& a, hipStream_t stream) {
    switch (a.epi) {
        case EPI_STORE: return launch_tile<FMT, MP, EPI_STORE>(a, stream);
        case EPI_RESID: return launch_tile<FMT, MP, EPI_RESID>(a, stream);
        case EPI_SWIGLU: return launch_tile<FMT, MP, EPI_SWIGLU>(a, stream);
        default: return launch_tile<FMT, MP, EPI_QKV>(a, stream);
    }
}

template <int FMT>
static int launch_fmt(const GemvArgs& a, hipStream_t stream) {
    if (a.mp == 4) return launch_epi<FMT, 4>(a, stream);
    if (a.mp == 8) return launch_epi<FMT, 8>(a, stream);
    return launch_epi<FMT, 16>(a, stream);
}

int launch_gemv(const GemvArgs& a, hipStream_t stream) {
    if (a.N % 16 || a.K % 128 || a.M <= 0 || a.M > GT_MROWS) return 2;
    if (a.fmt != WF_F32 && (!a.xf || (a.mp != 4 && a.mp != 8 && a.mp != 16) || a.M > a.mp || (a.m_base & 15) ||
                            (a.norm_w && !a.ssq_in)))
        return 2;
    if (a.fmt == WF_F32) {
        (void)hipGetLastError();
        hipLaunchKernelGGL(gemv_f32_kernel, dim3(a.N / 16), dim3(GT_THREADS), 0, stream, a);
        return note_error(hipGetLastError()) ? 4 : 0;
    }
    switch (a.fmt) {
        case WF_INT4: return launch_fmt<WF_INT4>(a, stream);
        case WF_INT8: return launch_fmt<WF_INT8>(a, stream);
        case WF_BF16: return launch_fmt<WF_BF16>(a, stream);
    }
    return 3;
}

}  // namespace aarh
