// Device-side writer of XFrag activation fragments (see kernels.hpp).
#pragma once
#include "device_common.hpp"
#include "kernels.hpp"

namespace aarh {

// Store element (m, c) of an activation matrix (value x before the consumer's
// norm weight) into its fragment entries.  Rows past f.mp of a chunk with
// mp <= 8 are never consumed and are not written.
// v = x * norm_w[c] already applied.
__device__ __forceinline__ void frag_put_w(const XFrag& f, int m, int c, float v) {
    uint16_t hi, lo;
    if (f.fmt == WF_BF16) {
        hi = f32_to_bf16_rne(v);
        lo = f32_to_bf16_rne(v - bf16_to_f32(hi));
    } else {
        const _Float16 h = (_Float16)v;
        hi = __builtin_bit_cast(uint16_t, h);
        lo = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)h));
    }
    const int mt = m >> 4, r = m & 15;
    if (f.mp <= 8 && r >= f.mp) return;
    const int g = c >> 7, lg = (c >> 5) & 3, t = (c >> 3) & 3, j = frag_slot(f.fmt, c & 7);
    const int epb = frag_epb(f.mp);
    const size_t base = ((((size_t)mt * f.G + g) * 4 + t) * 4 + lg) * epb;
    const int ehi = r, elo = f.mp <= 8 ? f.mp + r : 16 + r;
    f.buf[(base + ehi) * 8 + j] = hi;
    f.buf[(base + elo) * 8 + j] = lo;
}

__device__ __forceinline__ void frag_put(const XFrag& f, int m, int c, float x) {
    frag_put_w(f, m, c, f.norm_w ? x * f.norm_w[c] : x);
}

// Columns c8 .. c8+7 (c8 a multiple of 8) of row m as one 16-byte hi entry and one
// 16-byte lo entry (values already multiplied by the consumer's norm weight).
__device__ __forceinline__ void frag_put8_w(const XFrag& f, int m, int c8, const float (&v)[8]) {
    typedef unsigned fr_u32x4_t __attribute__((ext_vector_type(4)));
    const int mt = m >> 4, r = m & 15;
    if (f.mp <= 8 && r >= f.mp) return;
    uint16_t hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        uint16_t h, l;
        if (f.fmt == WF_BF16) {
            h = f32_to_bf16_rne(v[e]);
            l = f32_to_bf16_rne(v[e] - bf16_to_f32(h));
        } else {
            const _Float16 hh = (_Float16)v[e];
            h = __builtin_bit_cast(uint16_t, hh);
            l = __builtin_bit_cast(uint16_t, (_Float16)(v[e] - (float)hh));
        }
        const int j = frag_slot(f.fmt, e);
        hi[j] = h;
        lo[j] = l;
    }
    const int g = c8 >> 7, lg = (c8 >> 5) & 3, t = (c8 >> 3) & 3;
    const size_t base = ((((size_t)mt * f.G + g) * 4 + t) * 4 + lg) * frag_epb(f.mp);
    const int ehi = r, elo = f.mp <= 8 ? f.mp + r : 16 + r;
    fr_u32x4_t wh, wl;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        wh[q] = (uint32_t)hi[2 * q] | ((uint32_t)hi[2 * q + 1] << 16);
        wl[q] = (uint32_t)lo[2 * q] | ((uint32_t)lo[2 * q + 1] << 16);
    }
    *(fr_u32x4_t*)(f.buf + (base + ehi) * 8) = wh;
    *(fr_u32x4_t*)(f.buf + (base + elo) * 8) = wl;
}

}  // namespace aarh
