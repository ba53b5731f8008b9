// Quantised skinny GEMM for the verify forward on gfx950.
//
// Replaces QatLinear::forward (quant/src/qat.rs:315-348), i.e. y = x . W^T
// for every projection of the verify forward (attention.rs:170-222,
// ffn.rs:29-37, head.rs:47-49), with the weights kept quantised in HBM.
//
// Layout: W [N, K] is stored as 16-row x 128-column tiles, tile (nt, g) is a
// contiguous block (1 KiB INT4, 2 KiB INT8, 4 KiB BF16) in which lane l of a
// wave owns row l%16, columns 32*(l/16)..+32 of the group (16/32/64 bytes), cut
// into 16-byte chunks: chunk q of all 64 lanes is the q-th KiB of the tile, so
// each 16-byte load of the wave reads one contiguous KiB (tile_byte()).  INT4
// scale and zero (fp16) sit beside the tiles, one u32 per (tile, group, row).
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
#include "epilogue.hpp"

namespace aarh {

static constexpr int GT_NW = 8;         // waves per workgroup of the fragment GEMV
static constexpr int GT_PF = 4;         // its prefetch ring depth (items per wave)
static constexpr int GT_THREADS = 256;  // f32 GEMV workgroup
static constexpr int GT_MROWS = 16;     // activation rows per launch (one MFMA row tile)

// Quantised GEMV over fragment inputs, persistent over 16-row weight tiles:
// workgroup b takes tiles b, b + grid, ...; wave w of the NW waves takes the
// groups w, w + NW, ... of each tile (ngp items per tile, padded to the ring
// depth PF; padding items are skipped).  A ring of PF slots holds, per item,
// the weight tile words (and, on the L2 path, the lane's activation fragment
// entries), so the next PF items are in flight while one is computed, across
// tile boundaries.  Loads are buffer loads with wave-uniform offsets, issued
// unconditionally (indices clamped into range); only the arithmetic depends
// on whether a group is real: conditional loads would be merged with
// register copies that wait for ALL outstanding loads.
//
// Since a wave meets the same groups in every tile, with NGP > 0 (items per
// tile per wave known at compile time, MP <= 8) the wave loads the fragment
// entries of its groups into registers once (16 VGPRs per group) and the
// stream carries weights and scales only.  NGP == 0 reads the fragments of
// each item from L2 inside the ring (M > 8, or K beyond the register budget).
//
// No workgroup barrier inside the stream: at the end of a tile each wave
// leaves its partial in an LDS slot (two slots, by tile parity) and the last
// wave to arrive (LDS counter) adds the NW partials in wave order and runs
// the epilogue alone while the others go on.  A wave waits before reusing a
// slot until the epilogue two tiles back has released it.
template <int FMT, int MP, int EPI, int NGP>
__global__ void __launch_bounds__(GT_NW * 64) gemv_tile_kernel(GemvArgs a) {
    constexpr int NW = GT_NW;
    constexpr bool RS = MP <= 8;        // hi / lo in MFMA rows
    constexpr int EA = RS ? 1 : 2;      // fragment entries per k-step per lane
    constexpr int EPB = RS ? 2 * MP : 32;
    constexpr bool REG = NGP > 0;       // fragments held in registers
    static_assert(!REG || (RS && NGP % GT_PF == 0), "register fragments need MP <= 8 and whole rings");
    typedef FmtTraits<FMT> T;
    constexpr int PF = GT_PF;
    __shared__ float4_t part_s[2][NW][64];
    __shared__ float yt_s[2][16][17];
    __shared__ float s_inv[16];
    __shared__ unsigned cnt_s[2], gen_s[2];
    __shared__ float ep_pf[128];  // epilogue inputs of the last tile, loaded ahead by wave NW - 1
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int G = a.K >> 7;
    const int Mc = a.M;
    const int ntiles = a.N >> 4;
    const int ngp = REG ? NGP : ((G + NW - 1) / NW + PF - 1) / PF * PF;  // items per tile per wave
    const int nmine = (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int mt = a.m_base >> 4;
    const int elane = RS ? min(lr, 2 * MP - 1) : lr;  // fragment entry of this lane (lo: +16 at MP 16)
    const int glast = G - 1 - ((G - 1 - wid) % NW + NW) % NW;  // last real group of this wave (may be < 0)

    const __amdgpu_buffer_rsrc_t wr = coh_rsrc(a.w), fr = coh_rsrc(a.xf), zr = coh_rsrc(a.sz);
    const unsigned w_voff = (unsigned)lane * 16u;
    const unsigned f_voff = (unsigned)(lg * EPB + elane) * 16u;
    const unsigned z_voff = (unsigned)lr * 4u;
    uint32_t wv[PF][T::LANE_WORDS];
    uint32_t szv[PF];
    constexpr int NA = REG ? 1 : PF;
    uint4 av[NA][4][EA];  // L2 path: fragment ring
    // Register path.  MP == 8: one entry per k-step.  MP == 4 needs MFMA rows
    // 0..7 only, so k-steps 2j and 2j+1 share a register: rows 0..7 (lanes 0..7
    // of each 16-lane row) hold k-step 2j, rows 8..15 k-step 2j + 1.  The register
    // is the A operand of both k-steps; even k-steps accumulate into acc[0], whose
    // product rows 0..7 are right, odd ones into acc[1], whose rows 8..15 are
    // (rows of a 16x16 product: lanes 0..31 hold 0..7, lanes 32..63 hold 8..15).
    // The wave's partial takes acc[0] in lanes 0..31 and acc[1] in lanes 32..63;
    // the epilogue adds product rows r and 8 + r.
    constexpr bool PK = MP == 4;
    constexpr int NREG = PK ? 2 : 4;
    uint4 fa[REG ? NGP : 1][NREG];
    auto load_frag_reg = [&](uint4 (&f)[NREG], int g) {
        const int f_soff = (int)(((unsigned)mt * G + g) * 16u * EPB * 16u);
        const unsigned voff = PK ? (unsigned)((lg * EPB + (lr & 7)) * 16 + (lr >> 3) * 4 * EPB * 16) : f_voff;
#pragma unroll
        for (int j = 0; j < NREG; j++)
            f[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 fr, (int)voff, f_soff + (PK ? 2 : 1) * j * 4 * EPB * 16, 0));
    };
    auto unpack_frag = [&](const uint4 (&f)[NREG], uint4 (&o)[4][EA]) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            o[t][0] = f[PK ? t >> 1 : t];
        }
    };
    auto load_frag = [&](uint4 (&f)[4][EA], int g) {
        const int f_soff = (int)(((unsigned)mt * G + g) * 16u * EPB * 16u);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int e = 0; e < EA; e++)
                f[t][e] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        fr, (int)(f_voff + 256u * e), f_soff + t * 4 * EPB * 16, 0));
    };
    // item (tile tl, slot gi) of this wave -> ring slot p
    auto load_item = [&](int p, int tl, int gi) {
        const int g = max(min(wid + NW * gi, glast), 0);
        const unsigned tile = (unsigned)((int)blockIdx.x + tl * (int)gridDim.x) * G + g;
        const int w_soff = (int)(tile * T::TILE_BYTES);
#pragma unroll
        for (int q = 0; q < T::LANE_WORDS / 4; q++) {
            const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)w_voff, w_soff + 1024 * q, 2));
            wv[p][4 * q + 0] = v[0];
            wv[p][4 * q + 1] = v[1];
            wv[p][4 * q + 2] = v[2];
            wv[p][4 * q + 3] = v[3];
        }
        if (FMT == WF_INT4) szv[p] = __builtin_amdgcn_raw_buffer_load_b32(zr, (int)z_voff, (int)(tile * 64u), 0);
        if constexpr (!REG) load_frag(av[p], g);
    };
    // one item: weights of ring slot p times fragment entries f, added to acc[0]
    // (register-packed MP 4: even k-steps to acc[0], odd ones to acc[1])
    constexpr bool PKR = REG && PK;
    auto mma_item = [&](float4_t (&acc)[2], int p, const uint4 (&f)[4][EA]) {
        if (FMT == WF_INT4) {
            const uint32_t szw = szv[p];
            const float sc = (float)__builtin_bit_cast(_Float16, (uint16_t)(szw & 0xFFFFu));
            half2_t zl2, zh2;
            int4_zero_operands(__builtin_bit_cast(_Float16, (uint16_t)(szw >> 16)), zl2, zh2);
            float4_t g4[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};  // two independent chains
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const half8_t b = int4_b_operand(wv[p][t], zl2, zh2);
#pragma unroll
                for (int e = 0; e < EA; e++)
                    g4[(t + e) & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, f[t][e]), b,
                                                                             g4[(t + e) & 1], 0, 0, 0);
            }
            if (PKR) {
                acc[0] += sc * g4[0];
                acc[1] += sc * g4[1];
            } else {
                acc[0] += sc * (g4[0] + g4[1]);
            }
        } else if (FMT == WF_INT8) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const half8_t b = int8_b_operand(wv[p][2 * t], wv[p][2 * t + 1]);
#pragma unroll
                for (int e = 0; e < EA; e++)
                    acc[PKR ? t & 1 : 0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(half8_t, f[t][e]), b, acc[PKR ? t & 1 : 0], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const u32x4_t w4 = {wv[p][4 * t], wv[p][4 * t + 1], wv[p][4 * t + 2], wv[p][4 * t + 3]};
                const bf16x8_t b = __builtin_bit_cast(bf16x8_t, w4);
#pragma unroll
                for (int e = 0; e < EA; e++)
                    acc[PKR ? t & 1 : 0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8_t, f[t][e]), b, acc[PKR ? t & 1 : 0], 0, 0, 0);
            }
        }
    };
    // ---- the weight stream starts first: nothing below depends on it ----
    if (nmine > 0) {
#pragma unroll
        for (int p = 0; p < PF; p++) load_item(p, 0, p);
        if constexpr (REG) {
#pragma unroll
            for (int gi = 0; gi < NGP; gi++) load_frag_reg(fa[gi], max(min(wid + NW * gi, glast), 0));
        }
    }
    // ---- epilogue inputs of this workgroup's last tile, loaded now by the last wave
    //      (RESID: old x and the consumer's norm weight; QKV: RoPE cos / sin), so the
    //      final epilogue does not wait for them ----
    constexpr bool PF_EPI = EPI == EPI_RESID || EPI == EPI_QKV;
    float pf0 = 0.f, pf1 = 1.f;
    const int nt_last = (int)blockIdx.x + (nmine - 1) * (int)gridDim.x;
    if (PF_EPI && nmine > 0 && wid == NW - 1) {
        if (EPI == EPI_RESID) {
            if (lane < Mc * 16) {
                const int m = lane >> 4, n = lane & 15;
                pf0 = a.resid[(size_t)(a.m_base + m) * a.ldr + nt_last * 16 + n];
                if (a.fo.norm_w) pf1 = a.fo.norm_w[nt_last * 16 + n];
            }
        } else {
            const QkvEpi& e = a.qkv;
            const int half = e.hd >> 1, row0 = nt_last * 16;
            if (lane < Mc * 8 && row0 < e.n_heads * e.hd + e.n_kv * e.hd) {
                const int m = lane >> 3, r = lane & 7, mg = a.m_base + m;
                const int pos = e.pos0[mg / e.S] + mg % e.S, d1 = 8 * ((row0 % e.hd) >> 4) + r;
                pf0 = e.rope_cos[(size_t)pos * half + d1];
                pf1 = e.rope_sin[(size_t)pos * half + d1];
            }
        }
    }
    // ---- RMSNorm: 1/rms of each row from the producer's 16-column partial sums.
    //      Only the epilogues need it, so wave w loads the partials of row w (and
    //      w + NW) now and reduces them at the end of its first tile: no wait on the
    //      weight loads issued above.  Buffer loads past the row's K / 16 partials
    //      (or with no row) read 0. ----
    constexpr int SQL = 4;                  // partials per lane held in registers
    constexpr int SQR = MP > 8 ? 2 : 1;     // rows per wave (Mc <= NW * SQR)
    const int nq = a.K >> 4;
    const bool ss_late = a.norm_w && !a.hidden_out && nq <= 64 * SQL;
    float ssr[SQR][SQL];
#pragma unroll
    for (int j = 0; j < SQR; j++) {
        const int m = wid + NW * j;
        const bool has = ss_late && m < Mc;
        const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(has ? a.ssq_in + (size_t)(a.m_base + m) * a.ssq_ld : a.x), (short)0, has ? nq * 4 : 0,
            0x00020000);
#pragma unroll
        for (int i = 0; i < SQL; i++)
            ssr[j][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, (lane + 64 * i) * 4, 0, 0));
    }
    if (tid < 2) {
        cnt_s[tid] = 0u;
        gen_s[tid] = 0u;
    }
    if (a.norm_w && !ss_late) {
        for (int m = wid; m < Mc; m += NW) {
            float ss = 0.f;
            for (int q = lane; q < (a.K >> 4); q += 64) ss += a.ssq_in[(size_t)(a.m_base + m) * a.ssq_ld + q];
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, 64);
            if (lane == 0) s_inv[m] = 1.0f / sqrtf(ss / (float)a.K + a.eps);
        }
    }
    // LDS-only barrier: the weight loads above stay in flight
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (EPI == EPI_STORE && a.hidden_out) {
        // final normed hidden state (model.rs:579-585): workgroup b writes
        // columns [b*cw, (b+1)*cw) of every row, 4 at a time
        const int cw = ((a.K + (int)gridDim.x - 1) / (int)gridDim.x + 3) & ~3;
        const int k0 = (int)blockIdx.x * cw, kn = min(cw, a.K - k0);
        for (int idx = tid; idx < Mc * (kn >> 2); idx += NW * 64) {
            const int m = idx / (kn >> 2), k = k0 + 4 * (idx - m * (kn >> 2));
            const float4 v = *(const float4*)(a.x + row_off(a.xmap, a.m_base + m) + k);
            const float4 w = *(const float4*)(a.norm_w + k);
            const float si = s_inv[m];
            *(float4*)(a.hidden_out + (size_t)(a.m_base + m) * a.K + k) =
                make_float4(v.x * si * w.x, v.y * si * w.y, v.z * si * w.z, v.w * si * w.w);
        }
    }
    if (nmine <= 0) return;

    for (int tl = 0; tl < nmine; tl++) {
        float4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        if constexpr (REG) {
            const int ntl = min(tl + 1, nmine - 1);
#pragma unroll
            for (int gi = 0; gi < NGP; gi++) {
                if (wid + NW * gi < G) {
                    uint4 f[4][EA];
                    unpack_frag(fa[gi], f);
                    mma_item(acc, gi % PF, f);
                }
                // the slot's next item: PF further in this tile, or the head of the next one
                if (gi + PF < NGP)
                    load_item(gi % PF, tl, gi + PF);
                else
                    load_item(gi % PF, ntl, gi + PF - NGP);
            }
        } else {
            for (int gi0 = 0; gi0 < ngp; gi0 += PF) {
                // items PF ahead: same tile, or the first slots of the next one (last tile: clamped)
                const bool wrap = gi0 + PF >= ngp;
                const int rtl = wrap ? min(tl + 1, nmine - 1) : tl;
                const int rgi0 = wrap ? 0 : gi0 + PF;
#pragma unroll
                for (int p = 0; p < PF; p++) {
                    if (wid + NW * (gi0 + p) < G) mma_item(acc, p, av[p]);
                    load_item(p, rtl, rgi0 + p);
                }
            }
        }
        // ---- end of tile tl: partial -> slot, the last wave reduces + epilogue ----
        if (ss_late && tl == 0) {
            // written before this wave's first arrival (LDS operations of a wave run in order)
#pragma unroll
            for (int j = 0; j < SQR; j++) {
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < SQL; i++) {
                    asm volatile("" : "+v"(ssr[j][i]));  // keeps the sum here, not before the loop
                    ss += ssr[j][i];
                }
#pragma unroll
                for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, 64);
                const int m = wid + NW * j;
                if (lane == 0 && m < Mc) s_inv[m] = 1.0f / sqrtf(ss / (float)a.K + a.eps);
            }
        }
        const int ps = tl & 1;
        if (PF_EPI && wid == NW - 1 && tl == nmine - 1) {
            // written before this wave's arrival below (LDS operations of a wave run in order)
            ep_pf[lane] = pf0;
            ep_pf[64 + lane] = pf1;
        }
        while (__hip_atomic_load(&gen_s[ps], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != (unsigned)(tl >> 1))
            __builtin_amdgcn_s_sleep(1);
        part_s[ps][wid][lane] = PKR && lane >= 32 ? acc[1] : acc[0];
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
                    if (PKR) v += yt[8 + m][n] + yt[8 + MP + m][n];
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
            run_epilogue<EPI>(a, yt, nt, Mc, a.m_base, lane, 64, true, PF_EPI && tl == nmine - 1 ? ep_pf : nullptr);
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
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
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
        case EPI_STORE: run_epilogue<EPI_STORE>(a, yt, nt, Mc, a.m_base, threadIdx.x, GT_THREADS, false); break;
        case EPI_RESID: run_epilogue<EPI_RESID>(a, yt, nt, Mc, a.m_base, threadIdx.x, GT_THREADS, false); break;
        case EPI_SWIGLU: run_epilogue<EPI_SWIGLU>(a, yt, nt, Mc, a.m_base, threadIdx.x, GT_THREADS, false); break;
        default: run_epilogue<EPI_QKV>(a, yt, nt, Mc, a.m_base, threadIdx.x, GT_THREADS, false); break;
    }
}

template <int FMT, int MP, int EPI, int NGP>
static int launch_tile(const GemvArgs& a, hipStream_t stream) {
    static int grid_cap = 0;
    if (!grid_cap) {
        int dev = 0, cus = 0, per_cu = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)gemv_tile_kernel<FMT, MP, EPI, NGP>,
                                                           GT_NW * 64, 0);
        grid_cap = std::max(1, cus) * std::max(1, per_cu);
    }
    // Tiles spread evenly over the resident workgroups (no partial last round).
    const int ntiles = a.N / 16;
    const int per_wg = (ntiles + grid_cap - 1) / grid_cap;
    const int grid = (ntiles + per_wg - 1) / per_wg;
    (void)hipGetLastError();
    launch_timed(gemv_tile_kernel<FMT, MP, EPI, NGP>, dim3(grid), dim3(GT_NW * 64), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// Items per tile per wave for the register-fragment path: ceil(G / NW) groups
// rounded up to whole rings, while the fragments fit without spilling (8 VGPRs
// per group at MP 4, up to 12 groups; 16 at MP 8, up to 8 groups); 0 otherwise.
static int reg_items(const GemvArgs& a) {
    if (a.mp > 8) return 0;
    const int per_wave = ((a.K >> 7) + GT_NW - 1) / GT_NW;
    const int ngp = (per_wave + GT_PF - 1) / GT_PF * GT_PF;
    return ngp <= (a.mp == 4 ? 12 : 8) ? ngp : 0;
}

template <int FMT, int MP, int EPI>
static int launch_ngp(const GemvArgs& a, hipStream_t stream) {
    if constexpr (MP <= 8) {
        const int n = reg_items(a);
        if (n == 4) return launch_tile<FMT, MP, EPI, 4>(a, stream);
        if (n == 8) return launch_tile<FMT, MP, EPI, 8>(a, stream);
        if constexpr (MP == 4)
            if (n == 12) return launch_tile<FMT, MP, EPI, 12>(a, stream);
    }
    return launch_tile<FMT, MP, EPI, 0>(a, stream);
}

template <int FMT, int MP>
static int launch_epi(const GemvArgs& a, hipStream_t stream) {
    switch (a.epi) {
        case EPI_STORE: return launch_ngp<FMT, MP, EPI_STORE>(a, stream);
        case EPI_RESID: return launch_ngp<FMT, MP, EPI_RESID>(a, stream);
        case EPI_SWIGLU: return launch_ngp<FMT, MP, EPI_SWIGLU>(a, stream);
        default: return launch_ngp<FMT, MP, EPI_QKV>(a, stream);
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
    if (a.hidden_out && (!a.norm_w || (a.xmap.seq_stride & 3) || (a.xmap.row_stride & 3) || ((uintptr_t)a.x & 15) ||
                         ((uintptr_t)a.hidden_out & 15)))
        return 2;
    if (a.fmt == WF_F32) {
        (void)hipGetLastError();
        launch_timed(gemv_f32_kernel, dim3(a.N / 16), dim3(GT_THREADS), 0, stream, a);
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
