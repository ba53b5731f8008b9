// Quantised skinny GEMM for the verify forward on gfx950.
//
// Replaces QatLinear::forward (quant/src/qat.rs:315-348), i.e. y = x . W^T
// for every projection of the verify forward (attention.rs:170-222,
// ffn.rs:29-37, head.rs:47-49), with the weights kept quantised in HBM.
//
// Layout: W [N, K] is stored as 16-row x 128-column tiles, tile (nt, g) is a
// contiguous block (1 KiB INT4, 2 KiB INT8, 4 KiB BF16) in which lane l of a
// wave owns row l%16, columns 32*(l/16)..+32 of the group: one 16/32/64-byte
// load per lane, 1-4 KiB per wave instruction, fully coalesced.  INT4 scale
// and zero (fp16) sit beside the tiles, one u32 per (tile, group, row).
//
// Compute: weights are dequantised in registers to EXACT fp16 integers
// (q - z for INT4, code for INT8: magic-number 0x6400 conversion) or used as
// bf16; activations are staged in LDS as fp16 (bf16) hi + lo rows, so one
// v_mfma_f32_16x16x32 tile holds 8 activation rows at ~22-bit precision
// (rows 8-15 of the A tile would otherwise be padding when M <= 8).  The
// INT4 group scale multiplies the fp32 group accumulator.  K is split over
// S workgroups per 128-row group; partials are summed in a fixed order by the
// last workgroup to arrive (atomic counter), which also runs the fused
// epilogue: plain store, residual add (+ sum of squares for the next
// RMSNorm), SwiGLU, or RoPE + KV-cache append for the QKV projection.
#include <float.h>

#include "device_common.hpp"
#include "kernels.hpp"

namespace aarh {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

static constexpr int GV_THREADS = 512;  // 8 waves x one 16-row tile = 128 rows per workgroup
static constexpr int LDS_PAD = 8;       // halves of padding per LDS row

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

// LDS slot of activation column k so that the A operand matches the order in
// which the weight dequantisation emits B elements.
template <int FMT>
__device__ __forceinline__ int a_slot(int k) {
    const int w = k & 7, blk = k & ~7;
    if (FMT == WF_INT4) return blk + (((w & 3) << 1) | (w >> 2));
    if (FMT == WF_INT8) return blk + ((w & 4) | ((w & 1) << 1) | ((w >> 1) & 1));
    return k;
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
// Epilogues (run by the last workgroup of a 128-row group on the reduced
// tile yt[M][128] in LDS).
// ---------------------------------------------------------------------------
__device__ void epi_store(const GemvArgs& a, float* yt, int rg) {
    for (int idx = threadIdx.x; idx < a.M * 128; idx += blockDim.x) {
        int m = idx >> 7, c = idx & 127;
        a.out[row_off(a.omap, m) + rg * 128 + c] = yt[idx];
    }
}

__device__ void epi_resid(const GemvArgs& a, float* yt, int rg) {
    for (int idx = threadIdx.x; idx < a.M * 128; idx += blockDim.x) {
        int m = idx >> 7, c = idx & 127;
        float* p = a.resid + (size_t)m * a.ldr + rg * 128 + c;
        float xn = *p + yt[idx];
        *p = xn;
        yt[idx] = xn;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int m = wid; m < a.M; m += nw) {
        float v0 = yt[m * 128 + lane], v1 = yt[m * 128 + 64 + lane];
        float s = wave_sum_f32(v0 * v0 + v1 * v1);
        if (lane == 0) a.ssq_out[(size_t)rg * a.M + m] = s;
    }
}

__device__ void epi_swiglu(const GemvArgs& a, float* yt, int rg) {
    // 128 rows = 8 tiles of (8 gate rows, 8 up rows) for 64 consecutive ffn columns.
    for (int idx = threadIdx.x; idx < a.M * 64; idx += blockDim.x) {
        int m = idx >> 6, j = idx & 63;
        int tt = j >> 3, w = j & 7;
        float g = yt[m * 128 + tt * 16 + w];
        float u = yt[m * 128 + tt * 16 + 8 + w];
        float silu = g / (1.0f + expf(-g));
        a.out[row_off(a.omap, m) + rg * 64 + j] = silu * u;
    }
}

__device__ void epi_qkv(const GemvArgs& a, float* yt, int rg) {
    const QkvEpi& e = a.qkv;
    const int hd = e.hd, half = hd >> 1;
    const int QD = e.n_heads * hd, KD = e.n_kv * hd;
    const int S = a.omap.S;
    // RoPE (rope.rs:107-126) on q and k columns, in place.
    for (int idx = threadIdx.x; idx < a.M * 64; idx += blockDim.x) {
        int m = idx >> 6, pp = idx & 63;
        int hs = pp / half, d = pp % half;
        int c1 = hs * hd + d, c2 = c1 + half;
        int n1 = rg * 128 + c1;
        if (n1 < QD + KD) {
            int bs = m / S, s = m % S;
            int pos = e.pos0[bs] + s;
            float cs = e.rope_cos[(size_t)pos * half + d], sn = e.rope_sin[(size_t)pos * half + d];
            float x1 = yt[m * 128 + c1], x2 = yt[m * 128 + c2];
            {
#pragma clang fp contract(off)
                float r1 = x1 * cs - x2 * sn;
                float r2 = x1 * sn + x2 * cs;
                yt[m * 128 + c1] = r1;
                yt[m * 128 + c2] = r2;
            }
        }
    }
    __syncthreads();
    if (e.kv_fmt != KV_INT8) {
        for (int idx = threadIdx.x; idx < a.M * 128; idx += blockDim.x) {
            int m = idx >> 7, c = idx & 127;
            int n = rg * 128 + c;
            float v = yt[idx];
            if (n < QD) {
                e.q_out[(size_t)m * QD + n] = v;
                continue;
            }
            int bs = m / S, s = m % S;
            int pos = e.pos0[bs] + s, sl = e.slot[bs];
            bool isk = n < QD + KD;
            int nn = isk ? n - QD : n - QD - KD;
            int kvh = nn / hd, d = nn % hd;
            size_t kidx = (((size_t)sl * e.n_kv + kvh) * e.cap + pos) * hd + d;
            size_t vidx = (((size_t)sl * e.n_kv + kvh) * hd + d) * e.cap + pos;
            if (e.kv_fmt == KV_F32) {
                if (isk) ((float*)e.kc)[kidx] = v;
                else ((float*)e.vc)[vidx] = v;
            } else {
                if (isk) ((_Float16*)e.kc)[kidx] = (_Float16)v;
                else ((_Float16*)e.vc)[vidx] = (_Float16)v;
            }
        }
        return;
    }
    // INT8 cache: per token, per kv-head absmax scale (stored fp16), codes from the f32 scale.
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int hpg = 128 / hd;
    for (int idx = threadIdx.x; idx < a.M * 128; idx += blockDim.x) {
        int m = idx >> 7, c = idx & 127;
        int n = rg * 128 + c;
        if (n < QD) e.q_out[(size_t)m * QD + n] = yt[idx];
    }
    for (int task = wid; task < a.M * hpg; task += nw) {
        int m = task / hpg, hs = task % hpg;
        int n0 = rg * 128 + hs * hd;
        if (n0 < QD) continue;
        int bs = m / S, s = m % S;
        int pos = e.pos0[bs] + s, sl = e.slot[bs];
        bool isk = n0 < QD + KD;
        int kvh = (isk ? n0 - QD : n0 - QD - KD) / hd;
        float v0 = lane < hd ? yt[m * 128 + hs * hd + lane] : 0.0f;
        float v1 = (lane + 64) < hd ? yt[m * 128 + hs * hd + lane + 64] : 0.0f;
        float amax = wave_max_f32(fmaxf(fabsf(v0), fabsf(v1)));
        float sc = amax <= FLT_EPSILON ? 1.0f : amax / 127.0f;
        int8_t q0 = (int8_t)fminf(fmaxf(roundf(v0 / sc), -127.0f), 127.0f);
        int8_t q1 = (int8_t)fminf(fmaxf(roundf(v1 / sc), -127.0f), 127.0f);
        _Float16 sch = (_Float16)sc;
        if (isk) {
            int8_t* kc = (int8_t*)e.kc + (((size_t)sl * e.n_kv + kvh) * e.cap + pos) * hd;
            if (lane < hd) kc[lane] = q0;
            if (lane + 64 < hd) kc[lane + 64] = q1;
            if (lane == 0) e.ks[((size_t)sl * e.n_kv + kvh) * e.cap + pos] = __builtin_bit_cast(uint16_t, sch);
        } else {
            int8_t* vc = (int8_t*)e.vc + ((size_t)sl * e.n_kv + kvh) * hd * e.cap + pos;
            if (lane < hd) vc[(size_t)lane * e.cap] = q0;
            if (lane + 64 < hd) vc[(size_t)(lane + 64) * e.cap] = q1;
            if (lane == 0) e.vs[((size_t)sl * e.n_kv + kvh) * e.cap + pos] = __builtin_bit_cast(uint16_t, sch);
        }
    }
}

__device__ void run_epilogue(const GemvArgs& a, float* yt, int rg) {
    switch (a.epi) {
        case EPI_STORE: epi_store(a, yt, rg); break;
        case EPI_RESID: epi_resid(a, yt, rg); break;
        case EPI_SWIGLU: epi_swiglu(a, yt, rg); break;
        default: epi_qkv(a, yt, rg); break;
    }
}

// ---------------------------------------------------------------------------
// Shared prologue: per-row inverse RMS from split partial sums of squares.
// ---------------------------------------------------------------------------
__device__ void prologue_inv_rms(const GemvArgs& a, float* s_inv) {
    if (!a.norm_w) return;
    // one wave per row: lane p loads partial p (n_ssq <= 64), one round trip
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int m = wid; m < a.M; m += nw) {
        float ss = 0.0f;
        for (int p = lane; p < a.n_ssq; p += 64) ss += a.ssq_part[(size_t)p * a.M + m];
        ss = wave_sum_f32(ss);
        if (lane == 0) s_inv[m] = 1.0f / sqrtf(ss / (float)a.K + a.eps);
    }
}

// Split-K: the last workgroup of a row group sums the S partials in order.
__device__ bool finish_partials(const GemvArgs& a, int rg, float* yt, unsigned* s_flag) {
    if (a.S == 1) return true;
    if (!arrive_last(&a.counters[rg], (unsigned)a.S, s_flag)) return false;
    for (int idx = threadIdx.x; idx < a.M * 128; idx += blockDim.x) {
        int m = idx >> 7, c = idx & 127;
        const float* p = a.part + (size_t)m * a.N + rg * 128 + c;
        const size_t stride = (size_t)a.M * a.N;
        float y = 0.0f;
        // batches of 8 independent coherent loads: one memory round trip per batch
        for (int s0 = 0; s0 < a.S; s0 += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = (s0 + j < a.S) ? ld_coh(p + (size_t)(s0 + j) * stride) : 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) y += v[j];
        }
        yt[idx] = y;
    }
    __syncthreads();
    return true;
}

__device__ __forceinline__ void map_block(const GemvArgs& a, int& rg, int& ks) {
    const int nrg = a.N >> 7;
    const int total = nrg * a.S;
    int bid = blockIdx.x, logical = bid;
    // Keep the S workgroups of one row group on one XCD (workgroups are dealt
    // round-robin over the 8 XCDs), so the split-K reduction stays in one L2.
    if ((total & 7) == 0) {
        int per = total >> 3;
        logical = (bid & 7) * per + (bid >> 3);
    }
    rg = logical / a.S;
    ks = logical % a.S;
}

template <int FMT, int MTMAX>
__global__ void __launch_bounds__(GV_THREADS) gemv_mfma_kernel(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ unsigned s_flag;
    typedef FmtTraits<FMT> T;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int G = a.K >> 7;
    int rg, ks;
    map_block(a, rg, ks);
    const int g0 = (ks * G) / a.S, g1 = ((ks + 1) * G) / a.S;
    const int ng = g1 - g0, KR = ng * 128, k0 = g0 * 128;
    const int MT = a.split ? (a.M + 7) >> 3 : (a.M + 15) >> 4;
    const int ldsrow = KR + LDS_PAD;
    uint16_t* At = (uint16_t*)smem;
    float* s_inv = (float*)(smem + (size_t)MT * 16 * ldsrow * 2);
    const int nt = rg * 8 + wid;

    float4_t acc[MTMAX];
#pragma unroll
    for (int mt = 0; mt < MTMAX; mt++) acc[mt] = (float4_t){0.f, 0.f, 0.f, 0.f};

    for (int gi = 0; gi < ng; gi += T::PF) {
        uint32_t wv[T::PF][T::LANE_WORDS];
        uint32_t szv[T::PF];
#pragma unroll
        for (int p = 0; p < T::PF; p++) {
            if (gi + p < ng) {
                const size_t tile = (size_t)nt * G + g0 + gi + p;
                const u32x4_t* src = (const u32x4_t*)(a.w + tile * T::TILE_BYTES + (size_t)lane * T::LANE_WORDS * 4);
#pragma unroll
                for (int q = 0; q < T::LANE_WORDS / 4; q++) {
                    u32x4_t v = __builtin_nontemporal_load(src + q);
                    wv[p][4 * q + 0] = v[0];
                    wv[p][4 * q + 1] = v[1];
                    wv[p][4 * q + 2] = v[2];
                    wv[p][4 * q + 3] = v[3];
                }
                if (FMT == WF_INT4) szv[p] = a.sz[tile * 16 + lr];
            }
        }
        if (gi == 0) {
            // Activation prologue overlaps the first weight loads.
            prologue_inv_rms(a, s_inv);
            if (a.norm_w) __syncthreads();
            const int rows = a.split ? MT * 8 : MT * 16;
            for (int idx = tid; idx < rows * KR; idx += GV_THREADS) {
                int m = idx / KR, k = idx - m * KR;
                float v = 0.0f;
                if (m < a.M) {
                    v = a.x[row_off(a.xmap, m) + k0 + k];
                    if (a.norm_w) v = v * s_inv[m] * a.norm_w[k0 + k];
                    if (a.hidden_out && rg == 0) a.hidden_out[(size_t)m * a.K + k0 + k] = v;
                }
                uint16_t hi, lo;
                if (FMT == WF_BF16) {
                    hi = f32_to_bf16_rne(v);
                    lo = f32_to_bf16_rne(v - bf16_to_f32(hi));
                } else {
                    _Float16 h = (_Float16)v;
                    hi = __builtin_bit_cast(uint16_t, h);
                    lo = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)h));
                }
                const int sl = a_slot<FMT>(k);
                if (a.split) {
                    const int mt = m >> 3, r = m & 7;
                    At[(size_t)(mt * 16 + r) * ldsrow + sl] = hi;
                    At[(size_t)(mt * 16 + 8 + r) * ldsrow + sl] = lo;
                } else {
                    At[(size_t)m * ldsrow + sl] = hi;
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int p = 0; p < T::PF; p++) {
            if (gi + p >= ng) break;
            const int gl = gi + p;
            if (FMT == WF_INT4) {
                const uint32_t szw = szv[p];
                const _Float16 zh = __builtin_bit_cast(_Float16, (uint16_t)(szw >> 16));
                const float sc = (float)__builtin_bit_cast(_Float16, (uint16_t)(szw & 0xFFFFu));
                const _Float16 zz = (_Float16)1024.0f + zh;
                const half2_t zz2 = {zz, zz};
                half8_t bop[4];
#pragma unroll
                for (int t = 0; t < 4; t++) bop[t] = int4_b_operand(wv[p][t], zz2);
#pragma unroll
                for (int mt = 0; mt < MTMAX; mt++) {
                    if (mt < MT) {
                    float4_t g4 = {0.f, 0.f, 0.f, 0.f};
                    const uint16_t* arow = At + (size_t)(mt * 16 + lr) * ldsrow + gl * 128 + 32 * lg;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        half8_t av = *(const half8_t*)(arow + 8 * t);
                        g4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bop[t], g4, 0, 0, 0);
                    }
                    acc[mt] += sc * g4;
                    }
                }
            } else if (FMT == WF_INT8) {
                half8_t bop[4];
#pragma unroll
                for (int t = 0; t < 4; t++) bop[t] = int8_b_operand(wv[p][2 * t], wv[p][2 * t + 1]);
#pragma unroll
                for (int mt = 0; mt < MTMAX; mt++) {
                    if (mt < MT) {
                    const uint16_t* arow = At + (size_t)(mt * 16 + lr) * ldsrow + gl * 128 + 32 * lg;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        half8_t av = *(const half8_t*)(arow + 8 * t);
                        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bop[t], acc[mt], 0, 0, 0);
                    }
                    }
                }
            } else {
                bf16x8_t bop[4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    u32x4_t w4 = {wv[p][4 * t], wv[p][4 * t + 1], wv[p][4 * t + 2], wv[p][4 * t + 3]};
                    bop[t] = __builtin_bit_cast(bf16x8_t, w4);
                }
#pragma unroll
                for (int mt = 0; mt < MTMAX; mt++) {
                    if (mt < MT) {
                    const uint16_t* arow = At + (size_t)(mt * 16 + lr) * ldsrow + gl * 128 + 32 * lg;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        bf16x8_t av = *(const bf16x8_t*)(arow + 8 * t);
                        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bop[t], acc[mt], 0, 0, 0);
                    }
                    }
                }
            }
        }
    }
    // ---- partial results ----
    const int ncol = nt * 16 + lr;
    const float rs = (FMT == WF_INT8) ? a.rscale[ncol] : 1.0f;
    __syncthreads();  // all waves finished reading At before it is reused as yt
    float* yt = (float*)smem;
#pragma unroll
    for (int mt = 0; mt < MTMAX; mt++) {
        if (mt >= MT) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v = acc[mt][i] * rs;
            int m;
            bool writer;
            if (a.split) {
                v += __shfl_xor(v, 32, 64);
                m = mt * 8 + 4 * lg + i;
                writer = lg < 2;
            } else {
                m = mt * 16 + 4 * lg + i;
                writer = true;
            }
            if (writer && m < a.M) {
                if (a.S == 1) yt[m * 128 + wid * 16 + lr] = v;
                else st_coh(&a.part[((size_t)ks * a.M + m) * a.N + ncol], v);
            }
        }
    }
    if (a.S == 1) __syncthreads();
    if (!finish_partials(a, rg, yt, &s_flag)) return;
    run_epilogue(a, yt, rg);
}

// Plain fp32 weights (the reference's CPU dtype): exact fp32 FMA dot products
// on the vector ALUs, same split-K / epilogue scheme.  Used by fp32 models.
__global__ void __launch_bounds__(GV_THREADS) gemv_f32_kernel(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ unsigned s_flag;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int G = a.K >> 7;
    int rg, ks;
    map_block(a, rg, ks);
    const int g0 = (ks * G) / a.S, g1 = ((ks + 1) * G) / a.S;
    const int KR = (g1 - g0) * 128, k0 = g0 * 128;
    float* xs = (float*)smem;                 // [M][KR]
    float* s_inv = xs + (size_t)a.M * KR;     // [M]
    prologue_inv_rms(a, s_inv);
    __syncthreads();
    for (int idx = tid; idx < a.M * KR; idx += GV_THREADS) {
        int m = idx / KR, k = idx - m * KR;
        float v = a.x[row_off(a.xmap, m) + k0 + k];
        if (a.norm_w) v = v * s_inv[m] * a.norm_w[k0 + k];
        if (a.hidden_out && rg == 0) a.hidden_out[(size_t)m * a.K + k0 + k] = v;
        xs[idx] = v;
    }
    __syncthreads();
    const float* W = (const float*)a.w;
    // each wave: 16 rows; lane covers k = lane, lane+64, ...
    float res[16][4];
    for (int r = 0; r < 16; r++)
        for (int m = 0; m < 4; m++) res[r][m] = 0.f;
    // rows processed in M-chunks of 4
    float* yt = (float*)(smem);  // reused after the loop
    for (int mb = 0; mb < a.M; mb += 4) {
        for (int r = 0; r < 16; r++) {
            const float* wr = W + (size_t)(rg * 128 + wid * 16 + r) * a.K + k0;
            float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
            for (int k = lane; k < KR; k += 64) {
                float w = wr[k];
                s0 = fmaf(xs[(mb + 0) * KR + k], w, s0);
                if (mb + 1 < a.M) s1 = fmaf(xs[(mb + 1) * KR + k], w, s1);
                if (mb + 2 < a.M) s2 = fmaf(xs[(mb + 2) * KR + k], w, s2);
                if (mb + 3 < a.M) s3 = fmaf(xs[(mb + 3) * KR + k], w, s3);
            }
            res[r][0] = wave_sum_f32(s0);
            res[r][1] = wave_sum_f32(s1);
            res[r][2] = wave_sum_f32(s2);
            res[r][3] = wave_sum_f32(s3);
        }
        if (a.S > 1 && lane < 16) {
            for (int mm = 0; mm < 4 && mb + mm < a.M; mm++) {
                float v = 0.f;
                for (int r = 0; r < 16; r++)
                    if (r == lane) v = res[r][mm];
                st_coh(&a.part[((size_t)ks * a.M + mb + mm) * a.N + rg * 128 + wid * 16 + lane], v);
            }
        }
        if (a.S == 1) {
            __syncthreads();
            if (lane < 16)
                for (int mm = 0; mm < 4 && mb + mm < a.M; mm++) {
                    float v = 0.f;
                    for (int r = 0; r < 16; r++)
                        if (r == lane) v = res[r][mm];
                    // stash into the tail of LDS beyond xs (yt region is written after loop)
                    s_inv[a.M + (mb + mm) * 128 + wid * 16 + lane] = v;
                }
        }
    }
    if (a.S == 1) {
        __syncthreads();
        for (int idx = tid; idx < a.M * 128; idx += GV_THREADS) yt[idx] = s_inv[a.M + idx];
        __syncthreads();
    }
    if (!finish_partials(a, rg, yt, &s_flag)) return;
    run_epilogue(a, yt, rg);
}

template <int FMT, int MTMAX>
static int launch_fmt(const GemvArgs& a, hipStream_t stream, size_t lds) {
    static bool attr = false;
    if (!attr) {
        if (note_error(hipFuncSetAttribute((const void*)gemv_mfma_kernel<FMT, MTMAX>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, MAX_DYN_LDS)))
            return 4;
        attr = true;
    }
    (void)hipGetLastError();
    hipLaunchKernelGGL((gemv_mfma_kernel<FMT, MTMAX>), dim3((a.N / 128) * a.S), dim3(GV_THREADS), lds,
                       stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

template <int FMT>
static int launch_mt(const GemvArgs& a, hipStream_t stream, size_t lds) {
    const int MT = a.split ? (a.M + 7) / 8 : (a.M + 15) / 16;
    if (MT <= 1) return launch_fmt<FMT, 1>(a, stream, lds);
    if (MT <= 4) return launch_fmt<FMT, 4>(a, stream, lds);
    if (MT <= 16) return launch_fmt<FMT, 16>(a, stream, lds);
    return 2;
}

int launch_gemv(const GemvArgs& a, hipStream_t stream) {
    if (a.N % 128 || a.K % 128 || a.M <= 0 || a.S <= 0 || a.S > a.K / 128) return 2;
    const int G = a.K / 128;
    const int maxng = (G + a.S - 1) / a.S;
    const int KR = maxng * 128;
    size_t yt = (size_t)a.M * 128 * 4;
    size_t lds;
    if (a.fmt == WF_F32) {
        lds = (size_t)a.M * KR * 4 + (size_t)a.M * 4 + (size_t)a.M * 128 * 4;
        if (lds < yt) lds = yt;
        if (lds > MAX_DYN_LDS) return 3;
        static bool attr = false;
        if (!attr) {
            if (note_error(hipFuncSetAttribute((const void*)gemv_f32_kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, MAX_DYN_LDS)))
                return 4;
            attr = true;
        }
        (void)hipGetLastError();
        hipLaunchKernelGGL(gemv_f32_kernel, dim3((a.N / 128) * a.S), dim3(GV_THREADS), lds, stream, a);
        return note_error(hipGetLastError()) ? 4 : 0;
    }
    const int MT = a.split ? (a.M + 7) / 8 : (a.M + 15) / 16;
    lds = (size_t)MT * 16 * (KR + LDS_PAD) * 2 + (size_t)a.M * 4;
    if (lds < yt) lds = yt;
    if (lds > MAX_DYN_LDS) return 3;
    switch (a.fmt) {
        case WF_INT4: return launch_mt<WF_INT4>(a, stream, lds);
        case WF_INT8: return launch_mt<WF_INT8>(a, stream, lds);
        case WF_BF16: return launch_mt<WF_BF16>(a, stream, lds);
    }
    return 3;
}

}  // namespace aarh
