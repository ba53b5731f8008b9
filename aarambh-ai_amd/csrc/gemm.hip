// Quantised GEMM for verify batches of more than 16 rows (batch x draft rows)
// on gfx950.
//
// Replaces QatLinear::forward (quant/src/qat.rs:315-348) when the verify
// forward carries many sequences: y = x . W^T over M = batch * (k+1) rows,
// every projection of attention.rs:170-222, ffn.rs:29-37 and head.rs:47-49.
// At M = 128 (batch 32, k = 3) an INT4 weight byte feeds 256 MACs, above the
// MI355X ridge, so this kernel is MFMA-bound.  Activations arrive as hi + lo
// fp16 (bf16 for BF16 weights) fragments written by their producer (mp = 16
// layout: per (chunk, group, k-step, lane group) 16 hi entries then 16 lo);
// INT4 / INT8 codes are exact in fp16, so products keep ~22 bits.
//
// Block: 8 waves = WM (M) x WN = 8 / WM (N), WM = 2 or 1.  It covers MC = WM *
// CPW row chunks (16 rows each) x NT = WN * TPW weight tiles (16 rows each) over
// a contiguous range of 128-column groups (split-K).  Wave (wm, wn) owns CPW
// chunks x TPW tiles: per group 8 * CPW * TPW MFMAs 16x16x32, with each INT4
// weight word dequantised once per wave for CPW chunks.  At 32 rows and below
// the 1 x 8 shape with both chunks in every wave dequantises each weight word
// once for four MFMAs instead of two (the dequantisation is VALU work of the
// same order as the MFMAs it feeds).
//
// Data movement: a ring of NS LDS stages, one 128-column group each, filled by
// direct HBM/L2 -> LDS loads (buffer_load ... lds, no VGPRs): the activation
// fragments of the block's chunks (8 KiB per chunk), the weight tiles and the
// INT4 scale/zero words.  Every wave issues the same number of loads per
// stage, so `s_waitcnt vmcnt(L * (NS - 1))` + a barrier publishes stage g
// while stages g+1 .. g+NS-1 are in flight.  Each byte enters the CU once.
//
// Split-K partials go to scratch with coherent stores; the block that arrives
// last at its (M-block, N-block) counter adds the S partials in split order
// (deterministic) and runs the fused epilogue (store, residual add + next
// fragments, SwiGLU, RoPE + Q/K/V rows) on each 16 x 16 tile.
#include "epilogue.hpp"

namespace aarh {

static constexpr int GM_WAVES = 8;
static constexpr int GM_LDS_BUDGET = 150 * 1024;  // dynamic LDS for the stage ring

template <int FMT, int WM, int CPW, int TPW_>
struct GmCfg {
    typedef FmtTraits<FMT> T;
    static constexpr int WN = GM_WAVES / WM;                        // N-waves
    static constexpr int TPW = TPW_;                                // weight tiles per wave
    static constexpr int NT = WN * TPW;                             // weight tiles per block
    static constexpr int MC = WM * CPW;                             // row chunks per block
    static constexpr int A_BYTES = MC * 8192;                       // hi + lo fragments of one group
    static constexpr int W_BYTES = NT * T::TILE_BYTES;
    // scale/zero words of the block's tiles: one 64-lane load covers 16 tiles
    static constexpr int Z_LOADS = FMT == WF_INT4 ? (NT + 15) / 16 : 0;
    static constexpr int Z_BYTES = Z_LOADS * 1024;
    static constexpr int STAGE = A_BYTES + W_BYTES + Z_BYTES;
    // narrow 32-row blocks keep the ring small enough for two blocks per CU
    static constexpr int BUDGET = (MC == 2 && NT <= 8) ? 76 * 1024 : GM_LDS_BUDGET;
    static constexpr int NS_RAW = BUDGET / STAGE;
    static constexpr int NS = NS_RAW < 2 ? 2 : (NS_RAW > 4 ? 4 : NS_RAW);
    static constexpr int A_PW = MC * 8 / GM_WAVES;                  // 1 KiB activation pieces per wave
    static constexpr int W_PIECES = W_BYTES / 1024;
    static constexpr int W_PW = (W_PIECES + GM_WAVES - 1) / GM_WAVES;  // 1 KiB weight pieces per wave
    static constexpr int L = A_PW + W_PW + Z_LOADS;                 // loads per wave per stage
    static_assert(MC * 8 % GM_WAVES == 0, "activation pieces split over waves");
    static_assert(WM * WN == GM_WAVES, "wave grid");
    // the epilogue stages each wave's 16 CPW x (16 TPW + 4) f32 tile in the idle ring
    static_assert(GM_WAVES * 16 * CPW * (16 * TPW + 4) * 4 <= NS * STAGE, "epilogue tile exceeds the ring");
    static_assert(NS * STAGE <= GM_LDS_BUDGET, "stage ring exceeds LDS");
};

// K-split mode (KS, INT4 at 32 rows): wave w takes the block's groups w, w + 8, ... for
// all NT = 8 weight tiles of the block.  Its activation group goes to its own 16 KiB of
// LDS by direct loads (read once, by that wave), the weight and scale/zero words stream
// straight into registers, and each dequantised word feeds both row chunks.  The eight
// waves' partial tiles are then added in LDS in wave order and the block continues as
// a 1 x 8 block with one tile per wave (split-K exchange, epilogue).
static constexpr int KS_LDS = GM_WAVES * 16384;

template <int FMT, int EPI, int WM, int CPW, int TPW_, bool KS = false>
__global__ void __launch_bounds__(GM_WAVES * 64) gemm_kernel(GemvArgs a, int S, int gps) {
    static_assert(!KS || (FMT == WF_INT4 && WM == 1 && CPW == 2 && TPW_ == 1), "K-split mode: INT4, 1 x 8, 2 x 1");
    typedef FmtTraits<FMT> T;
    typedef GmCfg<FMT, WM, CPW, TPW_> C;
    constexpr int TPW = C::TPW, NT = C::NT, MC = C::MC, NS = C::NS, LW = T::LANE_WORDS;
    extern __shared__ __attribute__((aligned(1024))) char lds[];
    __shared__ float s_inv[MC * 16];
    __shared__ unsigned s_flag;

    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int wm = wid / C::WN, wn = wid % C::WN;
    const int G = a.K >> 7;
    const int ntiles = a.N >> 4;
    const int NB = (ntiles + NT - 1) / NT;
    const int nchunks = (a.M + 15) >> 4;
    int bid = blockIdx.x;
    const int s = bid % S;
    bid /= S;
    // (N-block, M-block): the M-blocks of one N-block sit 8 workgroups apart in launch
    // order (workgroups go round-robin to the 8 XCDs), so they run on one XCD at
    // about the same time and share its L2 for their common weight tiles.  N-blocks
    // in whole groups of 8 first, the remainder in order.
    const int MBK = (int)gridDim.x / (NB * S);
    const int full = NB / 8 * 8;
    int nb, mb;
    if (bid < full * MBK) {
        const int r = bid % (8 * MBK);
        mb = r / 8;
        nb = bid / (8 * MBK) * 8 + r % 8;
    } else {
        const int r = bid - full * MBK, w = NB - full;
        mb = r / w;
        nb = full + r % w;
    }
    const int g0 = s * gps, ng = min(G, g0 + gps) - g0;

    // 1/rms of the block's rows from the producer's 16-column partial sums (same
    // summation order as the GEMV kernel)
    // wave w takes rows w, w + 8, ...; the partials of all its rows are loaded
    // before any is summed (4 per row per lane per round trip).
    auto compute_inv = [&]() {
        constexpr int RPW = MC * 16 / GM_WAVES;
        const int nq = a.K >> 4;
        float ss[RPW];
        int mrow[RPW];
#pragma unroll
        for (int k = 0; k < RPW; k++) {
            ss[k] = 0.f;
            mrow[k] = min(mb * MC * 16 + wid + GM_WAVES * k, a.M - 1);
        }
        for (int q0 = lane; q0 < nq; q0 += 256) {
            float v[RPW][4];
#pragma unroll
            for (int k = 0; k < RPW; k++)
#pragma unroll
                for (int u = 0; u < 4; u++) v[k][u] = a.ssq_in[(size_t)mrow[k] * a.ssq_ld + min(q0 + 64 * u, nq - 1)];
#pragma unroll
            for (int k = 0; k < RPW; k++)
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (q0 + 64 * u < nq) ss[k] += v[k][u];
        }
#pragma unroll
        for (int k = 0; k < RPW; k++) {
            float t = ss[k];
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) t += __shfl_xor(t, d, 64);
            if (lane == 0) s_inv[wid + GM_WAVES * k] = 1.0f / sqrtf(t / (float)a.K + a.eps);
        }
        __syncthreads();
    };
    // K <= 4096 (one round of partials per lane), outside the K-split mode (whose
    // registers are spoken for): the partials are loaded before the K loop and summed
    // after it, so their round trip and the barrier stay off the loop's start (1/rms is
    // needed only by the epilogue)
    constexpr int RPW_INV = KS ? 1 : MC * 16 / GM_WAVES;
    float inv_v[RPW_INV][4];
    auto inv_load = [&]() {
        const int nq = a.K >> 4;
#pragma unroll
        for (int k = 0; k < RPW_INV; k++) {
            const int m = min(mb * MC * 16 + wid + GM_WAVES * k, a.M - 1);
#pragma unroll
            for (int u = 0; u < 4; u++) inv_v[k][u] = a.ssq_in[(size_t)m * a.ssq_ld + min(lane + 64 * u, nq - 1)];
        }
    };
    auto inv_finish = [&]() {
        const int nq = a.K >> 4;
#pragma unroll
        for (int k = 0; k < RPW_INV; k++) {
            float t = 0.f;
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (lane + 64 * u < nq) t += inv_v[k][u];
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) t += __shfl_xor(t, d, 64);
            if (lane == 0) s_inv[wid + GM_WAVES * k] = 1.0f / sqrtf(t / (float)a.K + a.eps);
        }
        __syncthreads();
    };
    if (EPI == EPI_STORE && a.hidden_out) {
        // final normed hidden state (model.rs:579-585): the NB * S blocks of this
        // M-block each write a slice of columns of its rows
        compute_inv();
        const int nq = NB * S, q = nb * S + s;
        const int cw = ((a.K + nq - 1) / nq + 3) & ~3;
        const int k0 = q * cw, kn = max(0, min(cw, a.K - k0));
        const int rows = min(MC * 16, a.M - mb * MC * 16);
        for (int idx = tid; idx < rows * (kn >> 2); idx += GM_WAVES * 64) {
            const int r = idx / (kn >> 2), k = k0 + 4 * (idx - r * (kn >> 2));
            const int m = mb * MC * 16 + r;
            const float4 v = *(const float4*)(a.x + row_off(a.xmap, m) + k);
            const float4 w = *(const float4*)(a.norm_w + k);
            const float si = s_inv[r];
            *(float4*)(a.hidden_out + (size_t)m * a.K + k) =
                make_float4(v.x * si * w.x, v.y * si * w.y, v.z * si * w.z, v.w * si * w.w);
        }
    }

    // ---- stage loads: this wave's pieces of group g into ring slot st ----
    const __amdgpu_buffer_rsrc_t wr = coh_rsrc(a.w), fr = coh_rsrc(a.xf), zr = coh_rsrc(a.sz);
    constexpr int WP = T::TILE_BYTES / 1024;  // 1 KiB pieces per tile
    int z_tile[C::Z_LOADS > 0 ? C::Z_LOADS : 1];
#pragma unroll
    for (int q = 0; q < C::Z_LOADS; q++) z_tile[q] = min(nb * NT + 16 * q + (lane >> 2), ntiles - 1);
    auto issue_stage = [&](int st, int g) {
        char* base = lds + st * C::STAGE;
#pragma unroll
        for (int q = 0; q < C::A_PW; q++) {
            const int pi = wid * C::A_PW + q, cc = pi >> 3, sub = pi & 7;  // block chunk, 1 KiB piece
            const int mt = min(mb * MC + cc, nchunks - 1);
            lds_dma16(fr, base + cc * 8192 + sub * 1024, lane * 16 + sub * 1024, (mt * G + g) * 8192);
        }
        // tile jj, piece sub: the sub-th KiB of the tile = every lane's sub-th 16-byte
        // chunk, read contiguously; the wave reading piece sub from LDS is conflict-free
#pragma unroll
        for (int q = 0; q < C::W_PW; q++) {
            // pieces not a multiple of the waves: the extra loads repeat a piece (same bytes, same place)
            const int pi = (wid * C::W_PW + q) % C::W_PIECES, jj = pi / WP, sub = pi % WP;
            const int nt = min(nb * NT + jj, ntiles - 1);
            lds_dma16<true>(wr, base + C::A_BYTES + jj * T::TILE_BYTES + sub * 1024, lane * 16 + sub * 1024,
                      (int)(((unsigned)nt * G + g) * T::TILE_BYTES));
        }
#pragma unroll
        for (int q = 0; q < C::Z_LOADS; q++)
            lds_dma16(zr, base + C::A_BYTES + C::W_BYTES + q * 1024,
                      (int)(((unsigned)z_tile[q] * G + g) * 64u + (lane & 3) * 16u), 0);
    };

    float4_t acc[CPW][TPW];
#pragma unroll
    for (int c = 0; c < CPW; c++)
#pragma unroll
        for (int j = 0; j < TPW; j++) acc[c][j] = (float4_t){0.f, 0.f, 0.f, 0.f};

    // ---- one group from ring slot st ----
    auto compute_stage = [&](int st) {
        const char* base = lds + st * C::STAGE;
        uint4 ah[CPW][4], al[CPW][4];
#pragma unroll
        for (int c = 0; c < CPW; c++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint4* e = (const uint4*)(base + ((((wm * CPW + c) * 4 + t) * 4 + lg) * 32) * 16);
                ah[c][t] = e[lr];
                al[c][t] = e[16 + lr];
            }
        uint32_t wv[TPW][LW];
#pragma unroll
        for (int j = 0; j < TPW; j++) {
            const char* w = base + C::A_BYTES + (wn * TPW + j) * T::TILE_BYTES;
#pragma unroll
            for (int q = 0; q < LW / 4; q++) {
                const uint4 v = ((const uint4*)(w + q * 1024))[lane];
                wv[j][4 * q + 0] = v.x;
                wv[j][4 * q + 1] = v.y;
                wv[j][4 * q + 2] = v.z;
                wv[j][4 * q + 3] = v.w;
            }
        }
        if (FMT == WF_INT4) {
            half2_t zl2[TPW], zh2[TPW];
            float sc[TPW];
#pragma unroll
            for (int j = 0; j < TPW; j++) {
                const uint32_t szw = ((const uint32_t*)(base + C::A_BYTES + C::W_BYTES))[(wn * TPW + j) * 16 + lr];
                sc[j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(szw & 0xFFFFu));
                int4_zero_operands(__builtin_bit_cast(_Float16, (uint16_t)(szw >> 16)), zl2[j], zh2[j]);
            }
            float4_t ga[CPW][TPW];
#pragma unroll
            for (int c = 0; c < CPW; c++)
#pragma unroll
                for (int j = 0; j < TPW; j++) ga[c][j] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int j = 0; j < TPW; j++) {
                    const half8_t b = int4_b_operand(wv[j][t], zl2[j], zh2[j]);
#pragma unroll
                    for (int c = 0; c < CPW; c++) {
                        ga[c][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, ah[c][t]), b,
                                                                          ga[c][j], 0, 0, 0);
                        ga[c][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, al[c][t]), b,
                                                                          ga[c][j], 0, 0, 0);
                    }
                }
#pragma unroll
            for (int c = 0; c < CPW; c++)
#pragma unroll
                for (int j = 0; j < TPW; j++) acc[c][j] += sc[j] * ga[c][j];
        } else if (FMT == WF_INT8) {
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int j = 0; j < TPW; j++) {
                    const half8_t b = int8_b_operand(wv[j][2 * t], wv[j][2 * t + 1]);
#pragma unroll
                    for (int c = 0; c < CPW; c++) {
                        acc[c][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, ah[c][t]), b,
                                                                           acc[c][j], 0, 0, 0);
                        acc[c][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, al[c][t]), b,
                                                                           acc[c][j], 0, 0, 0);
                    }
                }
        } else {
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int j = 0; j < TPW; j++) {
                    const u32x4_t w4 = {wv[j][4 * t], wv[j][4 * t + 1], wv[j][4 * t + 2], wv[j][4 * t + 3]};
                    const bf16x8_t b = __builtin_bit_cast(bf16x8_t, w4);
#pragma unroll
                    for (int c = 0; c < CPW; c++) {
                        acc[c][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ah[c][t]), b,
                                                                            acc[c][j], 0, 0, 0);
                        acc[c][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, al[c][t]), b,
                                                                            acc[c][j], 0, 0, 0);
                    }
                }
        }
    };

    // ---- pipeline.  NS >= 3: LA = NS - 2 stages in flight ahead of the one
    // computed, and the stage a load rewrites was last read two groups ago, so
    // the one barrier per group (after the wait) also orders every wave's reads
    // before the rewrite.  NS == 2: one stage ahead and a second barrier after
    // the compute.
    constexpr int LA = NS >= 3 ? NS - 2 : 1;
    // K-split state: this wave's LDS stage, tiles, group count, weight / scale words of
    // the current group in two halves of four tiles
    char* const aw = lds + wid * 16384;
    const int mt0 = min(mb * MC, nchunks - 1), mt1 = min(mb * MC + 1, nchunks - 1);
    const int ks_n = ng > wid ? (ng - wid + GM_WAVES - 1) / GM_WAVES : 0;
    int ks_nt[KS ? NT : 1];
    u32x4_t wA[KS ? 4 : 1], wB[KS ? 4 : 1];
    uint32_t zA[KS ? 4 : 1], zB[KS ? 4 : 1];
    float4_t racc[KS ? 2 : 1][KS ? NT : 1];
    auto ks_issue_a = [&](int g) {
#pragma unroll
        for (int sub = 0; sub < 8; sub++) {
            lds_dma16(fr, aw + sub * 1024, lane * 16 + sub * 1024, (mt0 * G + g) * 8192);
            lds_dma16(fr, aw + 8192 + sub * 1024, lane * 16 + sub * 1024, (mt1 * G + g) * 8192);
        }
    };
    auto ks_load_w = [&](u32x4_t (&w)[4], uint32_t (&z)[4], int g, int j0) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int nt = ks_nt[(j0 + q) % (KS ? NT : 1)];
            w[q] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                      wr, lane * 16, (int)(((unsigned)nt * G + g) * 1024u), 2));
            z[q] = __builtin_amdgcn_raw_buffer_load_b32(zr, lr * 4, (int)(((unsigned)nt * G + g) * 64u), 0);
        }
    };
    if constexpr (KS) {
#pragma unroll
        for (int j = 0; j < NT; j++) ks_nt[j] = min(nb * NT + j, ntiles - 1);
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int j = 0; j < NT; j++) racc[c][j] = (float4_t){0.f, 0.f, 0.f, 0.f};
        if (ks_n > 0) {
            ks_issue_a(g0 + wid);
            ks_load_w(wA, zA, g0 + wid, 0);
            ks_load_w(wB, zB, g0 + wid, 4);
        }
    } else {
#pragma unroll
        for (int i = 0; i < LA; i++) issue_stage(i, g0 + min(i, ng - 1));
    }
    // the epilogue's 1/rms while the first stages are in flight (loads complete in
    // order, so its wait also covers those stages: the loop's first wait is then free)
    const bool norm_rows = a.norm_w && !(EPI == EPI_STORE && a.hidden_out);
    const bool inv_late = !KS && norm_rows && a.K <= 4096;
    if (inv_late) inv_load();
    else if (norm_rows) compute_inv();
    // rows and tiles of this wave's epilogue; QKV positions loaded up front
    const int row0 = (mb * MC + wm * CPW) * 16, tile0 = nb * NT + wn * TPW;
    int mrw[CPW][4];  // activation row, clamped into range
    bool rok[CPW][4];
#pragma unroll
    for (int c = 0; c < CPW; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int chunk = mb * MC + wm * CPW + c, m = chunk * 16 + 4 * lg + i;
            rok[c][i] = chunk < nchunks && m < a.M;
            mrw[c][i] = min(m, a.M - 1);
        }
    int pos[CPW][4];
    if (EPI == EPI_QKV)
#pragma unroll
        for (int c = 0; c < CPW; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) pos[c][i] = a.qkv.pos0[mrw[c][i] / a.qkv.S] + mrw[c][i] % a.qkv.S;
    if constexpr (KS) {
        // four tiles (q) of one half against both chunks, then the group scale
        auto ks_half = [&](const uint4 (&ah)[2][4], const uint4 (&al)[2][4], const u32x4_t (&w)[4],
                           const uint32_t (&z)[4], int j0) {
            half2_t zl2[4], zh2[4];
            float sc[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                sc[q] = (float)__builtin_bit_cast(_Float16, (uint16_t)(z[q] & 0xFFFFu));
                int4_zero_operands(__builtin_bit_cast(_Float16, (uint16_t)(z[q] >> 16)), zl2[q], zh2[q]);
            }
            float4_t ga[2][4];
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int q = 0; q < 4; q++) ga[c][q] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const half8_t bop = int4_b_operand(w[q][t], zl2[q], zh2[q]);
#pragma unroll
                    for (int c = 0; c < 2; c++) {
                        ga[c][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, ah[c][t]), bop,
                                                                          ga[c][q], 0, 0, 0);
                        ga[c][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, al[c][t]), bop,
                                                                          ga[c][q], 0, 0, 0);
                    }
                }
            // interleave the dequantisation of the next words with the MFMAs of the last
#pragma unroll
            for (int k = 0; k < 32; k++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two VALU
            }
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int q = 0; q < 4; q++) racc[c][j0 + q] += sc[q] * ga[c][q];
        };
        for (int i = 0; i < ks_n; i++) {
            const int g = g0 + wid + GM_WAVES * i;
            wait_vmcnt<0>();  // this group's activation stage and weight words have landed
            uint4 ah[2][4], al[2][4];
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const uint4* e = (const uint4*)(aw + c * 8192 + ((t * 4 + lg) * 32) * 16);
                    ah[c][t] = e[lr];
                    al[c][t] = e[16 + lr];
                }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the stage has been read
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            const bool more = i + 1 < ks_n;
            if (more) ks_issue_a(g + GM_WAVES);
            ks_half(ah, al, wA, zA, 0);
            if (more) ks_load_w(wA, zA, g + GM_WAVES, 0);
            ks_half(ah, al, wB, zB, 4);
            if (more) ks_load_w(wB, zB, g + GM_WAVES, 4);
        }
        wait_vmcnt<0>();
        __syncthreads();  // every wave's stage is idle: the reduction reuses the LDS
        // the eight K-lanes' partial tiles, added in wave order; wave w keeps tile w
        float4_t* red = (float4_t*)lds;
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int j = 0; j < NT; j++) red[((wid * 2 + c) * NT + j) * 64 + lane] = racc[c][j];
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 2; c++) {
            float4_t t = red[((0 * 2 + c) * NT + wid) * 64 + lane];
#pragma unroll
            for (int w = 1; w < GM_WAVES; w++) t += red[((w * 2 + c) * NT + wid) * 64 + lane];
            acc[c][0] = t;
        }
    } else {
        for (int gi = 0; gi < ng; gi++) {
            issue_stage((gi + LA) % NS, g0 + min(gi + LA, ng - 1));  // past the end: harmless repeats
            wait_vmcnt<C::L * LA>();
            __syncthreads();
            compute_stage(gi % NS);
            if constexpr (NS == 2) __syncthreads();
        }
    }
    wait_vmcnt<0>();
    __syncthreads();  // every wave's stage loads have landed: the ring is free for the epilogue
    if (inv_late) inv_finish();

    // ---- epilogue inputs that do not depend on this kernel's products: loaded in the
    //      same round trip as the split-K partials (after the arrival, which waits for
    //      every outstanding access), or right away without a split ----
    int ntv[TPW];
    bool tok[TPW];
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const int nt = tile0 + j;
        tok[j] = nt < ntiles;
        ntv[j] = min(nt, ntiles - 1);
    }
    // RESID: unit u = (row r, 8-column half s8 of a tile) of the wave's region; the old
    // residual and the next consumer's norm weights of every unit of the lane
    constexpr int TR = 16 * CPW, TLD = 16 * TPW + 4;
    constexpr int RU = TR * 2 * TPW, RI = (RU + 63) / 64;
    float rs[TPW];
    float xres[EPI == EPI_RESID ? RI : 1][8], nres[EPI == EPI_RESID ? RI : 1][8];
    float qcs[EPI == EPI_QKV ? TPW : 1][CPW][4], qsn[EPI == EPI_QKV ? TPW : 1][CPW][4];
    auto load_epi_inputs = [&]() {
        if (FMT == WF_INT8)
#pragma unroll
            for (int j = 0; j < TPW; j++) rs[j] = a.rscale[ntv[j] * 16 + lr];
        if (EPI == EPI_RESID) {
#pragma unroll
            for (int it = 0; it < RI; it++) {
                const int u = lane + 64 * it;
                const int r = u / (2 * TPW), s8 = u % (2 * TPW), m = row0 + r, nt = tile0 + (s8 >> 1);
                const int col = nt * 16 + (s8 & 1) * 8;
                const bool ok = u < RU && m < a.M && nt < ntiles;
                const float* xr = a.resid + (size_t)min(m, a.M - 1) * a.ldr + min(col, a.N - 8);
                if (ok && ((uintptr_t)xr & 15) == 0) {
                    const float4_t x0 = *(const float4_t*)xr, x1 = *(const float4_t*)(xr + 4);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        xres[it][e] = x0[e];
                        xres[it][4 + e] = x1[e];
                    }
                } else if (ok) {
#pragma unroll
                    for (int e = 0; e < 8; e++) xres[it][e] = xr[e];
                }
                if (ok && a.fo.buf && a.fo.norm_w)
#pragma unroll
                    for (int e = 0; e < 8; e++) nres[it][e] = a.fo.norm_w[col + e];
            }
        }
        // QKV: RoPE cos / sin of every (tile, row) of the lane
        if (EPI == EPI_QKV) {
            const int half = a.qkv.hd >> 1;
#pragma unroll
            for (int j = 0; j < TPW; j++) {
                const int rowq = ntv[j] * 16;
                const int d1 = 8 * ((rowq % a.qkv.hd) >> 4) + (lr & 7);
#pragma unroll
                for (int c = 0; c < CPW; c++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        qcs[j][c][i] = a.qkv.rope_cos[(size_t)pos[c][i] * half + d1];
                        qsn[j][c][i] = a.qkv.rope_sin[(size_t)pos[c][i] * half + d1];
                    }
            }
        }
    };
    if (S == 1) load_epi_inputs();

    if (S > 1) {
        // ---- split-K: partial tiles out, the last block of the (mb, nb) pair adds them in order ----
        const size_t unit = (size_t)mb * NB + nb;
        const __amdgpu_buffer_rsrc_t pr = coh_rsrc(a.gpart + unit * S * (MC * NT * 256));
#pragma unroll
        for (int c = 0; c < CPW; c++)
#pragma unroll
            for (int j = 0; j < TPW; j++) {
                const unsigned o = ((unsigned)(s * MC * NT + (wm * CPW + c) * NT + wn * TPW + j) * 64u + lane) * 16u;
                st4_coh(pr, o, acc[c][j]);
            }
        if (!arrive_last(a.gcnt + unit, (unsigned)S, &s_flag)) return;
        load_epi_inputs();
        // the wave's CPW * TPW tiles x 4 splits in flight per round trip, added in split order
        const unsigned step = (unsigned)(MC * NT) * 1024u;
#pragma unroll
        for (int c = 0; c < CPW; c++)
#pragma unroll
            for (int j = 0; j < TPW; j++) acc[c][j] = (float4_t){0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < S; s0 += 4) {
            float4_t v[CPW][TPW][4];
#pragma unroll
            for (int c = 0; c < CPW; c++)
#pragma unroll
                for (int j = 0; j < TPW; j++) {
                    const unsigned o0 = ((unsigned)((wm * CPW + c) * NT + wn * TPW + j) * 64u + lane) * 16u;
#pragma unroll
                    for (int i = 0; i < 4; i++) v[c][j][i] = ld4_coh(pr, o0 + step * (unsigned)min(s0 + i, S - 1));
                }
#pragma unroll
            for (int c = 0; c < CPW; c++)
#pragma unroll
                for (int j = 0; j < TPW; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (s0 + i < S) acc[c][j] += v[c][j][i];
        }
    }

    // ---- epilogue in the MFMA layout: lane (lr, lg) of tile (c, j) holds rows
    //      4 lg + i of chunk c for weight row lr of tile j.  Its global inputs were
    //      loaded for all of the wave's tiles before the split-K exchange.
#pragma unroll
    for (int c = 0; c < CPW; c++)
#pragma unroll
        for (int j = 0; j < TPW; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = acc[c][j][i];
                if (a.norm_w) v *= s_inv[(wm * CPW + c) * 16 + 4 * lg + i];
                if (FMT == WF_INT8) v *= rs[j];
                acc[c][j][i] = v;
            }

    // ---- the wave's tile goes through LDS (the stage ring is idle now) so that
    //      every global access is a 16-byte run of 4 (f32) or 8 (fragment)
    //      consecutive columns of one row ----
    float* wt = (float*)lds + wid * TR * TLD;
    if (EPI == EPI_QKV) {
        // a tile holds dims d = 8 jh + r (weight rows r < 8) and d + hd/2 (rows 8 + r) of one
        // head; RoPE (rope.rs:107-126) pairs lane lr with lane lr ^ 8, each keeps its own output
        const QkvEpi& e = a.qkv;
        const int QD = e.n_heads * e.hd, KD = e.n_kv * e.hd;
#pragma unroll
        for (int j = 0; j < TPW; j++) {
            const bool rot = ntv[j] * 16 < QD + KD;
#pragma unroll
            for (int c = 0; c < CPW; c++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float mine = acc[c][j][i], other = __shfl_xor(mine, 8, 64);
                    float y1 = lr < 8 ? mine : other, y2 = lr < 8 ? other : mine;
                    if (rot) {
#pragma clang fp contract(off)
                        const float r1 = y1 * qcs[j][c][i] - y2 * qsn[j][c][i];
                        const float r2 = y1 * qsn[j][c][i] + y2 * qcs[j][c][i];
                        y1 = r1;
                        y2 = r2;
                    }
                    wt[(16 * c + 4 * lg + i) * TLD + 16 * j + lr] = lr < 8 ? y1 : y2;
                }
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < CPW; c++)
#pragma unroll
            for (int j = 0; j < TPW; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) wt[(16 * c + 4 * lg + i) * TLD + 16 * j + lr] = acc[c][j][i];
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's LDS writes are done
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    {
        if (EPI == EPI_SWIGLU) {
            // unit (row, tile): gate rows 0-7 and up rows 8-15 of the tile give h columns nt*8 .. +7
            for (int u = lane; u < TR * TPW; u += 64) {
                const int r = u / TPW, j = u % TPW, m = row0 + r, nt = tile0 + j;
                if (m >= a.M || nt >= ntiles) continue;
                const float4_t g0 = *(const float4_t*)(wt + r * TLD + 16 * j), g1 = *(const float4_t*)(wt + r * TLD + 16 * j + 4);
                const float4_t u0 = *(const float4_t*)(wt + r * TLD + 16 * j + 8), u1 = *(const float4_t*)(wt + r * TLD + 16 * j + 12);
                float h[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    h[e] = g0[e] / (1.0f + expf(-g0[e])) * u0[e];
                    h[4 + e] = g1[e] / (1.0f + expf(-g1[e])) * u1[e];
                }
                if (a.out) {  // f32 rows only for a consumer that reads them (f32 weights)
                    float* dst = a.out + row_off(a.omap, m) + nt * 8;
                    if (((uintptr_t)dst & 15) == 0) {
                        *(float4_t*)dst = (float4_t){h[0], h[1], h[2], h[3]};
                        *(float4_t*)(dst + 4) = (float4_t){h[4], h[5], h[6], h[7]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; e++) dst[e] = h[e];
                    }
                }
                if (a.fo.buf) {
                    if (a.fo.norm_w)
#pragma unroll
                        for (int e = 0; e < 8; e++) h[e] *= a.fo.norm_w[nt * 8 + e];
                    frag_put8_w(a.fo, m, nt * 8, h);
                }
            }
        } else if (EPI == EPI_STORE || EPI == EPI_RESID) {
            // unit (row, 8-column half of a tile); lanes 2q and 2q+1 hold the two halves of one tile row
#pragma unroll
            for (int it = 0; it < RI; it++) {  // RU is a multiple of 64 units, or 32
                const int u = lane + 64 * it;
                if (u >= RU) break;
                const int r = u / (2 * TPW), s8 = u % (2 * TPW), m = row0 + r, nt = tile0 + (s8 >> 1);
                const int col = nt * 16 + (s8 & 1) * 8;
                const bool ok = m < a.M && nt < ntiles;
                const float4_t v0 = *(const float4_t*)(wt + r * TLD + 8 * s8), v1 = *(const float4_t*)(wt + r * TLD + 8 * s8 + 4);
                float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                if (EPI == EPI_STORE) {
                    if (ok) {
                        float* dst = a.out + row_off(a.omap, m) + col;
                        if (((uintptr_t)dst & 15) == 0) {
                            *(float4_t*)dst = v0;
                            *(float4_t*)(dst + 4) = v1;
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; e++) dst[e] = v[e];
                        }
                    }
                } else {
                    // x += y (old x loaded before the split-K exchange); the new x as fragments
                    // for the next consumer and its 16-column sums of squares
                    float sq = 0.f;
                    if (ok) {
                        float* xr = a.resid + (size_t)m * a.ldr + col;
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            v[e] += xres[it][e];
                            sq += v[e] * v[e];
                        }
                        if (((uintptr_t)xr & 15) == 0) {
                            *(float4_t*)xr = (float4_t){v[0], v[1], v[2], v[3]};
                            *(float4_t*)(xr + 4) = (float4_t){v[4], v[5], v[6], v[7]};
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; e++) xr[e] = v[e];
                        }
                        if (a.fo.buf) {
                            if (a.fo.norm_w)
#pragma unroll
                                for (int e = 0; e < 8; e++) v[e] *= nres[it][e];
                            frag_put8_w(a.fo, m, col, v);
                        }
                    }
                    sq += __shfl_xor(sq, 1, 64);
                    if (a.fo.ssq && ok && (s8 & 1) == 0) a.fo.ssq[(size_t)m * a.fo.ssq_ld + nt] = sq;
                }
            }
        } else if (EPI == EPI_QKV) {
            // unit (row, tile): dims 8 jh .. +7 and 8 jh + hd/2 .. +7 of one head
            const QkvEpi& e = a.qkv;
            const int hd = e.hd, half = hd >> 1;
            const int QD = e.n_heads * hd, KD = e.n_kv * hd;
            for (int u = lane; u < TR * TPW; u += 64) {
                const int r = u / TPW, j = u % TPW, m = row0 + r, nt = tile0 + j;
                if (m >= a.M || nt >= ntiles) continue;
                const int rowq = nt * 16, head = rowq / hd, d0 = 8 * ((rowq % hd) >> 4);
                float* dst;
                if (rowq < QD) dst = e.q_out + (size_t)m * QD + head * hd;
                else if (rowq < QD + KD) dst = e.kv_out + (size_t)m * 2 * KD + (head - e.n_heads) * hd;
                else dst = e.kv_out + (size_t)m * 2 * KD + KD + (head - e.n_heads - e.n_kv) * hd;
                const float* src = wt + r * TLD + 16 * j;
                float* p1 = dst + d0;
                float* p2 = dst + d0 + half;
                if ((((uintptr_t)p1 | (uintptr_t)p2) & 15) == 0) {
                    *(float4_t*)p1 = *(const float4_t*)src;
                    *(float4_t*)(p1 + 4) = *(const float4_t*)(src + 4);
                    *(float4_t*)p2 = *(const float4_t*)(src + 8);
                    *(float4_t*)(p2 + 4) = *(const float4_t*)(src + 12);
                } else {
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        p1[q] = src[q];
                        p2[q] = src[8 + q];
                    }
                }
            }
        }
    }
}

static int cu_count() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (cus <= 0) cus = 256;
    }
    return cus;
}

template <int FMT, int EPI, int WM, int CPW, int TPW, bool KS = false>
static size_t ring_bytes() {
    typedef GmCfg<FMT, WM, CPW, TPW> C;
    return KS ? (size_t)KS_LDS : (size_t)C::NS * C::STAGE;
}

// Resident blocks per CU of one configuration (dynamic LDS attribute set on first use).
template <int FMT, int EPI, int WM, int CPW, int TPW, bool KS = false>
static int blocks_per_cu() {
    static int per_cu = 0;
    if (!per_cu) {
        const size_t lds = ring_bytes<FMT, EPI, WM, CPW, TPW, KS>();
        if (note_error(hipFuncSetAttribute((const void*)gemm_kernel<FMT, EPI, WM, CPW, TPW, KS>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds)))
            return 0;
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)gemm_kernel<FMT, EPI, WM, CPW, TPW, KS>,
                                                           GM_WAVES * 64, lds);
        per_cu = std::max(per_cu, 1);
    }
    return per_cu;
}

// Launch with a WM x (8 / WM) wave grid, CPW row chunks and TPW weight tiles per
// wave and S k-splits.
template <int FMT, int EPI, int WM, int CPW, int TPW, bool KS = false>
static int launch_cfg(const GemvArgs& a, int S, hipStream_t stream) {
    typedef GmCfg<FMT, WM, CPW, TPW> C;
    if (!blocks_per_cu<FMT, EPI, WM, CPW, TPW, KS>()) return 4;
    const int G = a.K >> 7;
    const int NB = (a.N / 16 + C::NT - 1) / C::NT;
    const int MB = ((a.M + 15) / 16 + C::MC - 1) / C::MC;
    S = std::max(1, std::min(S, G));
    while (S > 1 && (long long)NB * MB * S * C::MC * C::NT * 256 > (a.gpart ? a.gpart_elems : 0)) S--;
    const int gps = (G + S - 1) / S;
    S = (G + gps - 1) / gps;  // every split non-empty
    if (S > 1 && (!a.gcnt || NB * MB > 8192)) return 2;  // counters: 8192 per context
    const size_t lds = ring_bytes<FMT, EPI, WM, CPW, TPW, KS>();
    (void)hipGetLastError();
    launch_timed(gemm_kernel<FMT, EPI, WM, CPW, TPW, KS>, dim3(NB * MB * S), dim3(GM_WAVES * 64), (uint32_t)lds,
                 stream, a, S, gps);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// Launch plan: block shape (wm = 2: 2 x 4 waves with cpw = 1 or 2; wm = 1: 1 x 8
// waves with cpw = 2; wm = 0: the K-split mode, INT4 at 32 rows, 8 tiles per block),
// weight tiles per wave (tpw) and k-splits (S).
struct GmPlan {
    int wm, cpw, tpw, S;
};

// Measured best plans for the projection shapes of the 7B-class decoder
// (d_model 4096, 32 x 128 query heads, 8 kv heads, ffn 11008, INT4 g128; bf16
// LM head over a 32000 vocabulary) at 32 / 64 / 128 rows (replay and MTP
// batches; verify batches of 16 and 32 sequences x 4 rows).  At 128 rows the
// 1 x 8 wave shape (four 32-row blocks per weight tile) took the batch-32 verify
// step from 6.59 to 6.41 ms; at 32 rows it measured slower in the full model than
// the 2 x 4 plans, and the K-split mode (wm = 0) is faster for gate/up (25.4 against
// 28.1 us) and down (17.3 against 17.6 us).
struct GmTuned {
    int fmt, N, K;
    GmPlan plan[3];
};
static constexpr GmTuned GM_TUNED[] = {
    {WF_INT4, 6144, 4096, {{2, 1, 2, 4}, {2, 2, 2, 4}, {1, 2, 1, 1}}},
    {WF_INT4, 4096, 4096, {{2, 1, 1, 4}, {2, 2, 1, 4}, {1, 2, 1, 2}}},
    {WF_INT4, 22016, 4096, {{0, 2, 1, 1}, {2, 2, 3, 2}, {1, 2, 3, 1}}},
    {WF_INT4, 4096, 11008, {{0, 2, 1, 8}, {2, 2, 1, 4}, {1, 2, 1, 2}}},
    {WF_BF16, 32000, 4096, {{2, 1, 2, 1}, {2, 2, 2, 1}, {2, 2, 2, 1}}},
};

// Widest weight-tile count per wave whose stage ring fits the LDS budget.
template <int FMT, int WM>
static constexpr int max_tpw() {
    return FMT == WF_BF16 ? (WM == 1 ? 1 : 2) : (WM == 1 && FMT == WF_INT8 ? 3 : 4);
}

template <int FMT, int EPI, int WM, int CPW>
static int per_cu_of(int tpw) {
    constexpr int TM = max_tpw<FMT, WM>();
    if constexpr (TM >= 4)
        if (tpw >= 4) return blocks_per_cu<FMT, EPI, WM, CPW, 4>();
    if constexpr (TM >= 3)
        if (tpw >= 3) return blocks_per_cu<FMT, EPI, WM, CPW, 3>();
    if constexpr (TM >= 2)
        if (tpw >= 2) return blocks_per_cu<FMT, EPI, WM, CPW, 2>();
    return blocks_per_cu<FMT, EPI, WM, CPW, 1>();
}

template <int FMT, int EPI>
static int plan_capacity(int wm, int cpw, int tpw) {
    const int per_cu = wm == 1 ? per_cu_of<FMT, EPI, 1, 2>(tpw)
                     : cpw == 2 ? per_cu_of<FMT, EPI, 2, 2>(tpw) : per_cu_of<FMT, EPI, 2, 1>(tpw);
    return cu_count() * std::max(per_cu, 1);
}

// 64-row blocks above 32 rows, 32-row blocks otherwise (both block shapes).  Among
// the tile widths (4, 3, 2, 1 weight tiles per wave; 2, 1 for BF16) and splits whose
// blocks fit one dispatch round, the plan fills the round best (fill counted up to
// 2/3 of a one-block-per-CU round, 1/2 of a two-block one: beyond that wider blocks
// measured faster than more of them), then uses the fewest splits, then the widest
// tiles, then the 2 x 4 shape.
template <int FMT, int EPI>
static GmPlan plan_gemm(const GemvArgs& a) {
    const int G = a.K >> 7, ntiles = a.N / 16, chunks = (a.M + 15) / 16;
    for (const GmTuned& t : GM_TUNED)
        if (t.fmt == FMT && t.N == a.N && t.K == a.K) return t.plan[a.M <= 32 ? 0 : a.M <= 64 ? 1 : 2];
    GmPlan best{2, a.M > 32 ? 2 : 1, 1, 1};
    double bkey0 = -1.0;
    int bkey1 = 0, bkey2 = 0;
    for (int wm = 2; wm >= (a.M > 32 ? 2 : 1); wm--) {
        const int cpw = wm == 1 || a.M > 32 ? 2 : 1, wn = GM_WAVES / wm;
        for (int tpw = wm == 1 ? max_tpw<FMT, 1>() : max_tpw<FMT, 2>(); tpw >= 1; tpw--) {
            const int cap = plan_capacity<FMT, EPI>(wm, cpw, tpw);
            const int units = ((ntiles + wn * tpw - 1) / (wn * tpw)) * ((chunks + wm * cpw - 1) / (wm * cpw));
            for (int S = 1; S <= std::min(8, G); S++) {
                const int gps = (G + S - 1) / S;
                if ((G + gps - 1) / gps != S) continue;  // another S gives the same splits
                const long long blocks = (long long)units * S;
                if (blocks > cap) break;
                const double fill = std::min((double)blocks / cap, cap > cu_count() ? 0.5 : 0.66);
                const double key0 = std::floor(fill * 100.0 + 1e-9) / 100.0;
                const int key2 = wn * tpw;
                if (key0 > bkey0 || (key0 == bkey0 && (-S > bkey1 || (-S == bkey1 && key2 > bkey2)))) {
                    bkey0 = key0;
                    bkey1 = -S;
                    bkey2 = key2;
                    best = {wm, cpw, tpw, S};
                }
            }
        }
    }
    return best;
}

template <int FMT, int EPI, int WM, int CPW>
static int launch_tpw(const GemvArgs& a, int tpw, int S, hipStream_t stream) {
    constexpr int TM = max_tpw<FMT, WM>();
    if constexpr (TM >= 4)
        if (tpw >= 4) return launch_cfg<FMT, EPI, WM, CPW, 4>(a, S, stream);
    if constexpr (TM >= 3)
        if (tpw >= 3) return launch_cfg<FMT, EPI, WM, CPW, 3>(a, S, stream);
    if constexpr (TM >= 2)
        if (tpw >= 2) return launch_cfg<FMT, EPI, WM, CPW, 2>(a, S, stream);
    return launch_cfg<FMT, EPI, WM, CPW, 1>(a, S, stream);
}

template <int FMT, int EPI>
static int launch_plan(const GemvArgs& a, const GmPlan& p, hipStream_t stream) {
    if constexpr (FMT == WF_INT4)
        if (p.wm == 0 && a.M <= 32) return launch_cfg<FMT, EPI, 1, 2, 1, true>(a, p.S, stream);
    if (p.wm <= 1) return launch_tpw<FMT, EPI, 1, 2>(a, p.tpw, p.S, stream);
    if (p.cpw == 2) return launch_tpw<FMT, EPI, 2, 2>(a, p.tpw, p.S, stream);
    return launch_tpw<FMT, EPI, 2, 1>(a, p.tpw, p.S, stream);
}

template <int FMT, int EPI>
static int launch_m(const GemvArgs& a, hipStream_t stream) {
    return launch_plan<FMT, EPI>(a, plan_gemm<FMT, EPI>(a), stream);
}

template <int FMT>
static int launch_f(const GemvArgs& a, hipStream_t stream) {
    switch (a.epi) {
        case EPI_STORE: return launch_m<FMT, EPI_STORE>(a, stream);
        case EPI_RESID: return launch_m<FMT, EPI_RESID>(a, stream);
        case EPI_SWIGLU: return launch_m<FMT, EPI_SWIGLU>(a, stream);
        default: return launch_m<FMT, EPI_QKV>(a, stream);
    }
}

int launch_gemm(const GemvArgs& a, hipStream_t stream) {
    if (a.N % 16 || a.K % 128 || a.M <= 0 || a.m_base != 0 || !a.xf || a.mp != 16 || (a.norm_w && !a.ssq_in))
        return 2;
    if (a.hidden_out && (!a.norm_w || (a.xmap.seq_stride & 3) || (a.xmap.row_stride & 3) || ((uintptr_t)a.x & 15) ||
                         ((uintptr_t)a.hidden_out & 15) || (a.K & 3)))
        return 2;
    switch (a.fmt) {
        case WF_INT4: return launch_f<WF_INT4>(a, stream);
        case WF_INT8: return launch_f<WF_INT8>(a, stream);
        case WF_BF16: return launch_f<WF_BF16>(a, stream);
    }
    return 3;
}

}  // namespace aarh
