// Quantised GEMM for verify batches of more than 16 rows (batch x draft rows)
// on gfx950.
//
// Replaces QatLinear::forward (quant/src/qat.rs:315-348) when the verify
// forward carries many sequences: y = x . W^T with the weights read from HBM
// once per 64 activation rows instead of once per 16.
//
// Block = 64 weight rows (4 tiles of 16) x 64 activation rows (4 row chunks of
// 16), 4 waves; wave w owns row chunk w against all 4 weight tiles, so one
// activation fragment read from LDS feeds 4 MFMAs.  The activation fragments
// (producer-written, hi + lo halves as two MFMAs) of each 128-column group are
// copied to LDS one group ahead (double buffer); the weight tiles of the next
// groups stream into a register ring.  Weights are dequantised in registers to
// exact fp16 integers (INT4 q - z, INT8 code) or used as bf16; the INT4 group
// scale multiplies the fp32 group accumulator.  Each wave then runs the fused
// epilogue on its 16 rows of each tile.
#include "epilogue.hpp"

namespace aarh {

static constexpr int GM_TILES = 4;  // weight tiles per block
static constexpr int GM_CH = 4;     // 16-row activation chunks per block (one per wave)

template <int FMT, int EPI>
__global__ void __launch_bounds__(256) gemm_kernel(GemvArgs a) {
    typedef FmtTraits<FMT> T;
    constexpr int GM_PW = 16 / T::LANE_WORDS > 0 ? 16 / T::LANE_WORDS : 1;  // weight ring depth (groups)
    constexpr int U = GM_PW > 2 ? GM_PW : 2;                                  // unroll: ring slots, x stages
    constexpr int EPB = 32;                       // fragment entries per (g, t, lg) with 16-row tiles
    constexpr int CHUNK_U4 = 4 * 4 * EPB;         // uint4 per (chunk, group) = 8 KiB
    __shared__ uint4 xs[2][GM_CH][CHUNK_U4];      // 64 KiB: two groups of activation fragments
    __shared__ float yt_s[GM_CH][16][17];
    __shared__ float s_inv[GM_CH * 16];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int G = a.K >> 7;
    const int ntiles = a.N >> 4;
    const int nchunks = (a.ssq_rows + 15) >> 4;   // fragment chunks allocated (rows of the buffers)
    const int bn = blockIdx.x, bm = blockIdx.y;
    const int nt0 = bn * GM_TILES;
    const int mt0 = bm * GM_CH;
    const int row0 = mt0 * 16;

    // ---- 1/rms of the block's rows from the producer's 16-column partial sums ----
    if (a.norm_w) {
        for (int r = wid; r < GM_CH * 16; r += 4) {
            const int m = row0 + r;
            float ss = 0.f;
            if (m < a.M)
                for (int q = lane; q < (a.K >> 4); q += 64) ss += a.ssq_in[(size_t)q * a.ssq_rows + m];
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, 64);
            if (lane == 0) s_inv[r] = 1.0f / sqrtf(ss / (float)a.K + a.eps);
        }
    }

    // ---- activation fragments of group g -> register stage (thread t copies 8 uint4) ----
    const __amdgpu_buffer_rsrc_t fr = coh_rsrc(a.xf), wr = coh_rsrc(a.w), zr = coh_rsrc(a.sz);
    // uint4 u of thread t: chunk u / 2 (uniform), entry t + 256 * (u % 2) of that chunk
    static_assert(CHUNK_U4 == 512, "two 256-thread passes per chunk");
    uint4 xstage[2][8];
    const unsigned x_voff = (unsigned)tid * 16u;
    auto load_x = [&](int st, int g) {
        g = min(g, G - 1);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int mt = min(mt0 + (u >> 1), nchunks - 1);
            const int soff = ((mt * G + g) * CHUNK_U4 + 256 * (u & 1)) * 16;
            xstage[st][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(fr, (int)x_voff, soff, 0));
        }
    };
    auto store_x = [&](int st, int buf) {
#pragma unroll
        for (int u = 0; u < 8; u++) xs[buf][u >> 1][tid + 256 * (u & 1)] = xstage[st][u];
    };

    // ---- weight ring: GM_PW groups x 4 tiles ----
    const unsigned w_voff = (unsigned)lane * T::LANE_WORDS * 4u;
    uint32_t wv[GM_PW][GM_TILES][T::LANE_WORDS];
    uint32_t szv[GM_PW][GM_TILES];
    auto load_w = [&](int p, int g) {
        g = min(g, G - 1);
#pragma unroll
        for (int j = 0; j < GM_TILES; j++) {
            const int nt = min(nt0 + j, ntiles - 1);
            const unsigned tile = (unsigned)nt * G + g;
#pragma unroll
            for (int q = 0; q < T::LANE_WORDS / 4; q++) {
                const u32x4_t v = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)(w_voff + 16u * q), (int)(tile * T::TILE_BYTES), 2));
                wv[p][j][4 * q + 0] = v[0];
                wv[p][j][4 * q + 1] = v[1];
                wv[p][j][4 * q + 2] = v[2];
                wv[p][j][4 * q + 3] = v[3];
            }
            if (FMT == WF_INT4) szv[p][j] = __builtin_amdgcn_raw_buffer_load_b32(zr, (int)(lr * 4), (int)(tile * 64u), 0);
        }
    };

#pragma unroll
    for (int p = 0; p < GM_PW; p++) load_w(p, p);
    // group g: loaded into stage g % 2 two groups ahead, copied to LDS buffer g % 2 one group ahead
    load_x(0, 0);
    load_x(1, 1);
    store_x(0, 0);
    __syncthreads();

    float4_t acc[GM_TILES], accl[GM_TILES];  // accl: lo-half products (INT8 / BF16)
#pragma unroll
    for (int j = 0; j < GM_TILES; j++) acc[j] = accl[j] = (float4_t){0.f, 0.f, 0.f, 0.f};

    for (int g0 = 0; g0 < G; g0 += U) {
#pragma unroll
        for (int p = 0; p < U; p++) {
            const int g = g0 + p;
            const int buf = p & 1;  // == g & 1 (U even)
            const int wp = p % GM_PW;
            if (g < G) {
                // stage `buf` (group g) is already in LDS: reuse it for group g + 2
                if (g + 2 < G) load_x(buf, g + 2);
                // A operands of this wave's chunk: 4 k-steps x (hi, lo)
                uint4 af[4][2];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int e = (t * 4 + lg) * EPB + 2 * lr;
                    af[t][0] = xs[buf][wid][e];
                    af[t][1] = xs[buf][wid][e + 1];
                }
                // k-step outer, tiles inner, hi and lo into separate accumulators: eight
                // independent MFMA chains keep the matrix pipe busy
                if (FMT == WF_INT4) {
                    half2_t zl2[GM_TILES], zh2[GM_TILES];
                    float sc[GM_TILES];
#pragma unroll
                    for (int j = 0; j < GM_TILES; j++) {
                        const uint32_t szw = szv[wp][j];
                        sc[j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(szw & 0xFFFFu));
                        int4_zero_operands(__builtin_bit_cast(_Float16, (uint16_t)(szw >> 16)), zl2[j], zh2[j]);
                    }
                    float4_t gh[GM_TILES], gl[GM_TILES];
#pragma unroll
                    for (int j = 0; j < GM_TILES; j++) gh[j] = gl[j] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int t = 0; t < 4; t++)
#pragma unroll
                        for (int j = 0; j < GM_TILES; j++) {
                            const half8_t b = int4_b_operand(wv[wp][j][t], zl2[j], zh2[j]);
                            gh[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af[t][0]), b, gh[j], 0, 0, 0);
                            gl[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af[t][1]), b, gl[j], 0, 0, 0);
                        }
#pragma unroll
                    for (int j = 0; j < GM_TILES; j++) acc[j] += sc[j] * (gh[j] + gl[j]);
                } else if (FMT == WF_INT8) {
#pragma unroll
                    for (int t = 0; t < 4; t++)
#pragma unroll
                        for (int j = 0; j < GM_TILES; j++) {
                            const half8_t b = int8_b_operand(wv[wp][j][2 * t], wv[wp][j][2 * t + 1]);
                            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af[t][0]), b, acc[j], 0, 0, 0);
                            accl[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af[t][1]), b, accl[j], 0, 0, 0);
                        }
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++)
#pragma unroll
                        for (int j = 0; j < GM_TILES; j++) {
                            const u32x4_t w4 = {wv[wp][j][4 * t], wv[wp][j][4 * t + 1], wv[wp][j][4 * t + 2], wv[wp][j][4 * t + 3]};
                            const bf16x8_t b = __builtin_bit_cast(bf16x8_t, w4);
                            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af[t][0]), b, acc[j], 0, 0, 0);
                            accl[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af[t][1]), b, accl[j], 0, 0, 0);
                        }
                }
                load_w(wp, g + GM_PW);
                // group g + 1 (loaded one iteration ago) -> the other LDS buffer, read after the barrier
                if (g + 1 < G) store_x(buf ^ 1, buf ^ 1);
                __syncthreads();
            }
        }
    }

    if (FMT != WF_INT4)
#pragma unroll
        for (int j = 0; j < GM_TILES; j++) acc[j] += accl[j];
    // ---- epilogue: wave w, row chunk mt0 + w, each of the 4 tiles ----
    const int mrow = row0 + wid * 16;
    const int Mc = min(16, a.M - mrow);
    if (Mc <= 0) return;
    float (*yt)[17] = yt_s[wid];
#pragma unroll
    for (int j = 0; j < GM_TILES; j++) {
        const int nt = nt0 + j;
        if (nt >= ntiles) break;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 4 * lg + i;
            float v = acc[j][i];
            if (a.norm_w) v *= s_inv[wid * 16 + r];
            if (FMT == WF_INT8) v *= a.rscale[nt * 16 + lr];
            yt[r][lr] = v;
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (EPI == EPI_STORE && a.hidden_out && nt == 0) {
            // final normed hidden state (model.rs:579-585), written by the blocks of tile 0
            for (int idx = lane; idx < Mc * a.K; idx += 64) {
                const int m = idx / a.K, k = idx - m * a.K;
                const float xv = a.x[row_off(a.xmap, mrow + m) + k];
                a.hidden_out[(size_t)(mrow + m) * a.K + k] = xv * s_inv[wid * 16 + m] * a.norm_w[k];
            }
        }
        run_epilogue<EPI>(a, yt, nt, Mc, mrow, lane, 64, true);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
}

template <int FMT, int EPI>
static int launch_e(const GemvArgs& a, hipStream_t stream) {
    const dim3 grid((a.N / 16 + GM_TILES - 1) / GM_TILES, (a.M + 16 * GM_CH - 1) / (16 * GM_CH));
    (void)hipGetLastError();
    hipLaunchKernelGGL((gemm_kernel<FMT, EPI>), grid, dim3(256), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

template <int FMT>
static int launch_f(const GemvArgs& a, hipStream_t stream) {
    switch (a.epi) {
        case EPI_STORE: return launch_e<FMT, EPI_STORE>(a, stream);
        case EPI_RESID: return launch_e<FMT, EPI_RESID>(a, stream);
        case EPI_SWIGLU: return launch_e<FMT, EPI_SWIGLU>(a, stream);
        default: return launch_e<FMT, EPI_QKV>(a, stream);
    }
}

int launch_gemm(const GemvArgs& a, hipStream_t stream) {
    if (a.N % 16 || a.K % 128 || a.M <= 0 || a.m_base != 0 || !a.xf || a.mp != 16 || (a.norm_w && !a.ssq_in))
        return 2;
    switch (a.fmt) {
        case WF_INT4: return launch_f<WF_INT4>(a, stream);
        case WF_INT8: return launch_f<WF_INT8>(a, stream);
        case WF_BF16: return launch_f<WF_BF16>(a, stream);
    }
    return 3;
}

}  // namespace aarh
