// Shared device pieces of the quantised GEMV / GEMM kernels: weight-format
// traits, in-register dequantisation to exact fp16 MFMA operands, and the
// fused epilogues applied to a 16-column output tile.
#pragma once
#include <float.h>

#include "device_common.hpp"
#include "frag.hpp"
#include "kernels.hpp"

namespace aarh {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

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

// INT4 word (nibbles n0..n7, column order) -> exact fp16 (q - z), element order
// [n0, n4, n1, n5, n2, n6, n3, n7].  Even nibbles: (v & 0x000F000F) | 0x6400
// is the fp16 1024 + q, minus zl = 1024 + z.  Odd nibbles stay in place:
// (v & 0x00F000F0) | 0x6400 is 1024 + 16 q, and fma(., 1/16, -zh) with
// zh = 64 + z gives q - z (every step exact in fp16).
// (x & m) | c in one VOP3 (the mask in a VGPR, the constant in an SGPR: gfx9
// VOP3 takes no literal operands).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "s"(c));
    return r;
}

__device__ __forceinline__ half8_t int4_b_operand(uint32_t v, half2_t zl, half2_t zh) {
    const half2_t s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const uint32_t v8 = v >> 8;
    const uint32_t lo = 0x000F000Fu, hi = 0x00F000F0u, magic = 0x64006400u;
    const half2_t h0 = __builtin_bit_cast(half2_t, and_or(v, lo, magic)) - zl;
    const half2_t h1 = __builtin_bit_cast(half2_t, and_or(v, hi, magic)) * s16 - zh;
    const half2_t h2 = __builtin_bit_cast(half2_t, and_or(v8, lo, magic)) - zl;
    const half2_t h3 = __builtin_bit_cast(half2_t, and_or(v8, hi, magic)) * s16 - zh;
    half8_t r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

// Zero-point operands of int4_b_operand for an fp16 zero z.
__device__ __forceinline__ void int4_zero_operands(_Float16 z, half2_t& zl, half2_t& zh) {
    const _Float16 l = (_Float16)1024.0f + z, h = (_Float16)64.0f + z;
    zl = (half2_t){l, l};
    zh = (half2_t){h, h};
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
// pf (optional, LDS): inputs of this tile loaded ahead by the caller, entry idx of
// the loop below: RESID pf[idx] = old x, pf[64 + idx] = consumer norm weight; QKV
// pf[idx] = cos, pf[64 + idx] = sin of the row's position (valid for idx < 64).
template <int EPI>
__device__ void run_epilogue(const GemvArgs& a, float (*yt)[17], int nt, int Mc, int mbase, int t0, int stride,
                             bool wave_only, const float* pf = nullptr) {
    const int tid = t0;
    if (EPI == EPI_STORE) {
        for (int idx = tid; idx < Mc * 16; idx += stride) {
            const int m = idx >> 4, n = idx & 15;
            a.out[row_off(a.omap, mbase + m) + nt * 16 + n] = yt[m][n];
        }
    } else if (EPI == EPI_RESID) {
        // x += y, and the new x as fragments + 16-column sums of squares for the next RMSNorm
        for (int idx = tid; idx < Mc * 16; idx += stride) {
            const int m = idx >> 4, n = idx & 15;
            float* p = a.resid + (size_t)(mbase + m) * a.ldr + nt * 16 + n;
            const bool pre = pf && idx < 64;
            const float xn = (pre ? pf[idx] : *p) + yt[m][n];
            *p = xn;
            yt[m][n] = xn;
            if (a.fo.buf) {
                if (pre) frag_put_w(a.fo, mbase + m, nt * 16 + n, xn * pf[64 + idx]);
                else frag_put(a.fo, mbase + m, nt * 16 + n, xn);
            }
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
                a.fo.ssq[(size_t)(mbase + tid) * a.fo.ssq_ld + nt] = ss;
            }
        }
    } else if (EPI == EPI_SWIGLU) {
        // rows 0-7 of the tile are gate rows, 8-15 the matching up rows (ffn columns nt*8 + r)
        for (int idx = tid; idx < Mc * 8; idx += stride) {
            const int m = idx >> 3, r = idx & 7;
            const float g = yt[m][r], u = yt[m][8 + r];
            const float silu = g / (1.0f + expf(-g));
            const float h = silu * u;
            if (a.out) a.out[row_off(a.omap, mbase + m) + nt * 8 + r] = h;
            if (a.fo.buf) frag_put(a.fo, mbase + m, nt * 8 + r, h);
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
            const int mg = mbase + m;
            const int d1 = 8 * j + r, d2 = d1 + half;
            float y1 = yt[m][r], y2 = yt[m][8 + r];
            if (is_q || is_k) {
                // RoPE (rope.rs:107-126): half-split rotation at the row's position
                float cs, sn;
                if (pf && idx < 64) {
                    cs = pf[idx];
                    sn = pf[64 + idx];
                } else {
                    const int bs = mg / e.S, s = mg % e.S;
                    const int pos = e.pos0[bs] + s;
                    cs = e.rope_cos[(size_t)pos * half + d1];
                    sn = e.rope_sin[(size_t)pos * half + d1];
                }
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


}  // namespace aarh
