// Verify / decode attention over the KV cache on gfx950.
//
// Replaces GroupedQueryAttention's attend step (nn/src/attention.rs:196-217)
// and the CPU kernel it dispatches to (kernel/src/cpu/parallel_attn.rs:190-233):
// causal softmax(q k^T * scale) v with shift kv_len - q_len, query head h
// reading kv head h % n_kv (repeat_heads, attention.rs:415-428).
//
// One workgroup handles (sequence, kv head, query-row tile, token chunk): all
// S x (n_heads/n_kv) query rows of a kv head share one read of the chunk's
// K/V (INT8 codes x fp16 per-token scale, fp16 or f32), which is dequantised
// once into LDS.  Each wave owns a fixed set of query rows: scores for 64
// tokens (one per lane), wave-wide online softmax, P.V with lanes over the
// head dimension.  Chunks are merged in a fixed order by the last workgroup
// of the (sequence, kv head, tile) (atomic counter) -- no KV is re-read.
#include <float.h>

#include "device_common.hpp"
#include "kernels.hpp"

namespace aarh {

static constexpr int AT_THREADS = 256;  // 4 waves
static constexpr int AT_TOK = 64;       // tokens per LDS sub-block
static constexpr int AT_MAXR = 32;      // query rows per workgroup
static constexpr int AT_MAXHD = 128;

__global__ void __launch_bounds__(AT_THREADS) attn_kernel(AttnArgs a) {
    __shared__ float qs[AT_MAXR][AT_MAXHD];
    __shared__ float ks[AT_TOK][AT_MAXHD + 1];
    __shared__ float vs[AT_TOK][AT_MAXHD + 1];
    __shared__ float ps[AT_MAXR][AT_TOK];
    __shared__ unsigned s_last;

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int hd = a.hd, G = a.n_heads / a.n_kv;
    const int R_total = a.S * G;
    int bid = blockIdx.x;
    const int chunk = bid % a.nchunks;
    bid /= a.nchunks;
    const int tile = bid % a.ntiles;
    bid /= a.ntiles;
    const int kvh = bid % a.n_kv;
    const int seq = bid / a.n_kv;
    const int r0 = tile * a.rows_per_tile;
    const int R = min(a.rows_per_tile, R_total - r0);
    const int pos0 = a.pos0[seq];
    const int kv_len = pos0 + a.S;
    const int sl = a.slot[seq];
    const int QD = a.n_heads * hd;

    // query rows: r -> (s = r / G, g = r % G), head h = kvh + g * n_kv
    for (int idx = tid; idx < R * hd; idx += AT_THREADS) {
        int r = idx / hd, d = idx % hd;
        int rr = r0 + r;
        int s = rr / G, g = rr % G;
        int h = kvh + g * a.n_kv;
        qs[r][d] = a.q[(size_t)(seq * a.S + s) * QD + h * hd + d];
    }

    const int t_begin = chunk * a.chunk;
    const int t_end = min(kv_len, t_begin + a.chunk);
    // per-wave rows: r = wid + 4*j
    float mrow[AT_MAXR / 4], lrow[AT_MAXR / 4];
    float o0[AT_MAXR / 4], o1[AT_MAXR / 4];
#pragma unroll
    for (int j = 0; j < AT_MAXR / 4; j++) {
        mrow[j] = -INFINITY;
        lrow[j] = 0.f;
        o0[j] = 0.f;
        o1[j] = 0.f;
    }
    const size_t head_base = (size_t)sl * a.n_kv + kvh;
    for (int tb = t_begin; tb < t_end; tb += AT_TOK) {
        const int nt = min(AT_TOK, t_end - tb);
        __syncthreads();
        // dequantise the K and V sub-block into LDS as f32 (effective cache values)
        for (int idx = tid; idx < nt * hd; idx += AT_THREADS) {
            int t = idx / hd, d = idx % hd;
            int tt = tb + t;
            float kv_, vv_;
            if (a.kv_fmt == KV_INT8) {
                float ksc = (float)__builtin_bit_cast(_Float16, a.ks[head_base * a.cap + tt]);
                float vsc = (float)__builtin_bit_cast(_Float16, a.vs[head_base * a.cap + tt]);
                kv_ = (float)((const int8_t*)a.kc)[(head_base * a.cap + tt) * hd + d] * ksc;
                vv_ = (float)((const int8_t*)a.vc)[(head_base * hd + d) * a.cap + tt] * vsc;
            } else if (a.kv_fmt == KV_F16) {
                kv_ = (float)((const _Float16*)a.kc)[(head_base * a.cap + tt) * hd + d];
                vv_ = (float)((const _Float16*)a.vc)[(head_base * hd + d) * a.cap + tt];
            } else {
                kv_ = ((const float*)a.kc)[(head_base * a.cap + tt) * hd + d];
                vv_ = ((const float*)a.vc)[(head_base * hd + d) * a.cap + tt];
            }
            ks[t][d] = kv_;
            vs[t][d] = vv_;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < AT_MAXR / 4; j++) {
            const int r = wid + 4 * j;
            if (r >= R) break;
            const int s = (r0 + r) / G;
            const int limit = pos0 + s;  // causal: t <= (kv_len - S) + s
            float sc = -INFINITY;
            const int t = tb + lane;
            if (lane < nt && t <= limit) {
                float dot = 0.f;
                for (int d = 0; d < hd; d++) dot = fmaf(qs[r][d], ks[lane][d], dot);
                sc = dot * a.scale;
            }
            float bm = wave_max_f32(sc);
            float mnew = fmaxf(mrow[j], bm);
            float p = (sc == -INFINITY) ? 0.f : expf(sc - mnew);
            float alpha = (mrow[j] == -INFINITY) ? 0.f : expf(mrow[j] - mnew);
            float psum = wave_sum_f32(p);
            lrow[j] = lrow[j] * alpha + psum;
            mrow[j] = mnew;
            ps[r][lane] = p;
            o0[j] *= alpha;
            o1[j] *= alpha;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < AT_MAXR / 4; j++) {
            const int r = wid + 4 * j;
            if (r >= R) break;
            float a0 = 0.f, a1 = 0.f;
            for (int t = 0; t < nt; t++) {
                float p = ps[r][t];
                a0 = fmaf(p, vs[t][lane], a0);
                if (lane + 64 < hd) a1 = fmaf(p, vs[t][lane + 64], a1);
            }
            o0[j] += a0;
            o1[j] += a1;
        }
    }

    // ---- write partial (m, l, O) for this chunk ----
    const size_t grp = ((size_t)seq * a.n_kv + kvh) * a.ntiles + tile;
    const size_t rec = (size_t)hd + 2;
    float* part = a.part + (grp * a.nchunks + chunk) * (size_t)AT_MAXR * rec;
#pragma unroll
    for (int j = 0; j < AT_MAXR / 4; j++) {
        const int r = wid + 4 * j;
        if (r >= R) break;
        float* pr = part + (size_t)r * rec;
        if (lane < hd) st_coh(&pr[2 + lane], o0[j]);
        if (lane + 64 < hd) st_coh(&pr[2 + lane + 64], o1[j]);
        if (lane == 0) {
            st_coh(&pr[0], mrow[j]);
            st_coh(&pr[1], lrow[j]);
        }
    }
    if (!arrive_last(&a.counters[grp], (unsigned)a.nchunks, &s_last)) return;
    // merge chunks in order
    const float* gp = a.part + grp * a.nchunks * (size_t)AT_MAXR * rec;
    for (int r = wid; r < R; r += 4) {
        float M = -INFINITY;
        for (int c = 0; c < a.nchunks; c++) M = fmaxf(M, ld_coh(&gp[((size_t)c * AT_MAXR + r) * rec]));
        float L = 0.f, acc0 = 0.f, acc1 = 0.f;
        for (int c = 0; c < a.nchunks; c++) {
            const float* pr = gp + ((size_t)c * AT_MAXR + r) * rec;
            float mc = ld_coh(&pr[0]);
            float w = (mc == -INFINITY) ? 0.f : expf(mc - M);
            L += ld_coh(&pr[1]) * w;
            if (lane < hd) acc0 += ld_coh(&pr[2 + lane]) * w;
            if (lane + 64 < hd) acc1 += ld_coh(&pr[2 + lane + 64]) * w;
        }
        float inv = L > 0.f ? 1.0f / L : 0.f;
        const int rr = r0 + r;
        const int s = rr / G, g = rr % G;
        const int h = kvh + g * a.n_kv;
        float* out = a.out + (size_t)(seq * a.S + s) * QD + h * hd;
        if (lane < hd) out[lane] = acc0 * inv;
        if (lane + 64 < hd) out[lane + 64] = acc1 * inv;
    }
}

// ---------------------------------------------------------------------------
// MFMA flash-decode attention for INT8 (codes x fp16 per-token scale) and fp16
// caches.  Workgroup = 4 waves over (sequence, kv head, <=16 query rows,
// token chunk); wave w takes 32-token blocks w, w+4, ...  Per block:
//   S = Q K^T : A = Q rows as fp16 hi (rows 0-7) + lo (rows 8-15), B = K codes
//               converted exactly to fp16; hi+lo rows are summed afterwards.
//   online softmax on S * k_scale * 1/sqrt(hd) with the causal limit per row,
//   O += P V  : A = P * v_scale as fp16 hi + lo (via an LDS transpose),
//               B = V^T codes (V is stored transposed, 8 tokens per load).
// The 4 waves' (m, l, O) are merged in LDS, chunks by the last workgroup.
// ---------------------------------------------------------------------------
typedef _Float16 half2v_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half8_t i8x8_to_half8_perm(uint32_t d0, uint32_t d1) {
    // exact int8 -> fp16 via 0x6400 magic; emits element order [0,2,1,3,4,6,5,7]
    const half2v_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    d0 ^= 0x80808080u;
    d1 ^= 0x80808080u;
    half2v_t h0 = __builtin_bit_cast(half2v_t, (d0 & 0x00FF00FFu) | 0x64006400u) - off;
    half2v_t h1 = __builtin_bit_cast(half2v_t, ((d0 >> 8) & 0x00FF00FFu) | 0x64006400u) - off;
    half2v_t h2 = __builtin_bit_cast(half2v_t, (d1 & 0x00FF00FFu) | 0x64006400u) - off;
    half2v_t h3 = __builtin_bit_cast(half2v_t, ((d1 >> 8) & 0x00FF00FFu) | 0x64006400u) - off;
    half8_t r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

// slot of element k inside its 8-block so that an A operand matches the B order
template <int KVF>
__device__ __forceinline__ int kv_slot(int k) {
    if (KVF == KV_INT8) {
        const int w = k & 7;
        return (k & ~7) + ((w & 4) | ((w & 1) << 1) | ((w >> 1) & 1));
    }
    return k;
}

__device__ __forceinline__ void lds_wave_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

static constexpr int AM_RT = 2;     // row tiles of 8 real query rows
static constexpr int AM_ROWS = 16;  // real query rows per workgroup
static constexpr int AM_HD = 128;

template <int KVF>
__global__ void __launch_bounds__(256) attn_mfma_kernel(AttnArgs a) {
    __shared__ __align__(16) uint16_t qs[AM_RT][16][AM_HD + 8];
    __shared__ __align__(16) uint16_t pt[4][AM_RT][16][32 + 8];
    __shared__ float mg_m[4][AM_ROWS], mg_l[4][AM_ROWS];
    __shared__ float mg_o[4][AM_ROWS][AM_HD + 4];
    __shared__ unsigned s_last;

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4, rb = (lg & 1) * 4;
    const int hd = AM_HD, G = a.n_heads / a.n_kv;
    const int R_total = a.S * G;
    int bid = blockIdx.x;
    const int chunk = bid % a.nchunks;
    bid /= a.nchunks;
    const int tile = bid % a.ntiles;
    bid /= a.ntiles;
    const int kvh = bid % a.n_kv;
    const int seq = bid / a.n_kv;
    const int r0 = tile * a.rows_per_tile;
    const int R = min(a.rows_per_tile, R_total - r0);
    const int pos0 = a.pos0[seq];
    const int kv_len = pos0 + a.S;
    const int sl = a.slot[seq];
    const int QD = a.n_heads * hd;
    const size_t hb = (size_t)sl * a.n_kv + kvh;

    // ---- stage Q (hi / lo fp16, format-permuted) ----
    for (int idx = tid; idx < AM_ROWS * hd; idx += 256) {
        const int rr = idx / hd, d = idx % hd;
        float v = 0.f;
        if (rr < R) {
            const int real = r0 + rr, s = real / G, g = real % G;
            v = a.q[(size_t)(seq * a.S + s) * QD + (kvh + g * a.n_kv) * hd + d];
        }
        const _Float16 hi = (_Float16)v;
        const _Float16 lo = (_Float16)(v - (float)hi);
        const int rt = rr >> 3, r8 = rr & 7, sl2 = kv_slot<KVF>(d);
        qs[rt][r8][sl2] = __builtin_bit_cast(uint16_t, hi);
        qs[rt][8 + r8][sl2] = __builtin_bit_cast(uint16_t, lo);
    }
    __syncthreads();
    half8_t qa[AM_RT][4];
#pragma unroll
    for (int rt = 0; rt < AM_RT; rt++)
#pragma unroll
        for (int kk = 0; kk < 4; kk++) qa[rt][kk] = *(const half8_t*)&qs[rt][lr][32 * kk + 8 * lg];

    // causal limit of the real rows this lane tracks (rows rb+i of each row tile)
    int lim[AM_RT][4];
#pragma unroll
    for (int rt = 0; rt < AM_RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int rr = rt * 8 + rb + i;
            lim[rt][i] = rr < R ? pos0 + (r0 + rr) / G : -1;
        }
    float mrow[AM_RT][4], lrow[AM_RT][4];
    float4_t o[AM_RT][8];
#pragma unroll
    for (int rt = 0; rt < AM_RT; rt++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            mrow[rt][i] = -INFINITY;
            lrow[rt][i] = 0.f;
        }
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[rt][dt] = (float4_t){0.f, 0.f, 0.f, 0.f};
    }

    const int t_begin = chunk * a.chunk;
    const int t_end = min(kv_len, t_begin + a.chunk);
    const float qk_scale = a.scale;
    for (int tb = t_begin + 32 * wid; tb < t_end; tb += 128) {
        // ---- S = Q K^T for two 16-token sub-tiles ----
        float4_t sc[AM_RT][2];
        float ksc[2], vsc[2];
        int tokv[2];
#pragma unroll
        for (int ts = 0; ts < 2; ts++) {
            const int tok = tb + 16 * ts + lr;
            tokv[ts] = tok;
            const int tk = tok < t_end ? tok : t_end - 1;
            half8_t kb[4];
            if (KVF == KV_INT8) {
                const uint8_t* kr = (const uint8_t*)a.kc + (hb * a.cap + tk) * hd + 8 * lg;
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const uint2 w = *(const uint2*)(kr + 32 * kk);
                    kb[kk] = i8x8_to_half8_perm(w.x, w.y);
                }
                ksc[ts] = (float)__builtin_bit_cast(_Float16, a.ks[hb * a.cap + tk]);
                vsc[ts] = (float)__builtin_bit_cast(_Float16, a.vs[hb * a.cap + tk]);
            } else {
                const _Float16* kr = (const _Float16*)a.kc + (hb * a.cap + tk) * hd + 8 * lg;
#pragma unroll
                for (int kk = 0; kk < 4; kk++) kb[kk] = *(const half8_t*)(kr + 32 * kk);
                ksc[ts] = 1.0f;
                vsc[ts] = 1.0f;
            }
#pragma unroll
            for (int rt = 0; rt < AM_RT; rt++) {
                float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < 4; kk++) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[rt][kk], kb[kk], acc, 0, 0, 0);
                sc[rt][ts] = acc;
            }
        }
        // ---- online softmax (rows rb+i; hi+lo summed across the lane halves) ----
        float pv[AM_RT][2][4];
#pragma unroll
        for (int rt = 0; rt < AM_RT; rt++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float s0 = sc[rt][0][i] + __shfl_xor(sc[rt][0][i], 32, 64);
                float s1 = sc[rt][1][i] + __shfl_xor(sc[rt][1][i], 32, 64);
                s0 = (tokv[0] < t_end && tokv[0] <= lim[rt][i]) ? s0 * ksc[0] * qk_scale : -INFINITY;
                s1 = (tokv[1] < t_end && tokv[1] <= lim[rt][i]) ? s1 * ksc[1] * qk_scale : -INFINITY;
                float mx = fmaxf(s0, s1);
#pragma unroll
                for (int d = 1; d < 16; d <<= 1) mx = fmaxf(mx, __shfl_xor(mx, d, 64));
                const float mnew = fmaxf(mrow[rt][i], mx);
                const float alpha = (mrow[rt][i] == -INFINITY) ? (mnew == -INFINITY ? 1.f : 0.f)
                                                                : expf(mrow[rt][i] - mnew);
                const float p0 = s0 == -INFINITY ? 0.f : expf(s0 - mnew);
                const float p1 = s1 == -INFINITY ? 0.f : expf(s1 - mnew);
                float ps = p0 + p1;
#pragma unroll
                for (int d = 1; d < 16; d <<= 1) ps += __shfl_xor(ps, d, 64);
                lrow[rt][i] = lrow[rt][i] * alpha + ps;
                mrow[rt][i] = mnew;
                pv[rt][0][i] = p0 * vsc[0];
                pv[rt][1][i] = p1 * vsc[1];
#pragma unroll
                for (int dt = 0; dt < 8; dt++) o[rt][dt][i] *= alpha;
            }
        }
        // ---- P -> LDS (hi rows 0-7, lo rows 8-15, token order permuted like V) ----
        if (lg < 2) {
#pragma unroll
            for (int rt = 0; rt < AM_RT; rt++)
#pragma unroll
                for (int ts = 0; ts < 2; ts++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float p = pv[rt][ts][i];
                        const _Float16 hi = (_Float16)p;
                        const _Float16 lo = (_Float16)(p - (float)hi);
                        const int col = kv_slot<KVF>(16 * ts + lr);
                        pt[wid][rt][rb + i][col] = __builtin_bit_cast(uint16_t, hi);
                        pt[wid][rt][8 + rb + i][col] = __builtin_bit_cast(uint16_t, lo);
                    }
        }
        lds_wave_sync();
        half8_t pa[AM_RT];
#pragma unroll
        for (int rt = 0; rt < AM_RT; rt++) pa[rt] = *(const half8_t*)&pt[wid][rt][lr][8 * lg];
        lds_wave_sync();
        // ---- O += P V ----
        const int tv = min(tb + 8 * lg, a.cap - 8);
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            half8_t vb;
            if (KVF == KV_INT8) {
                const uint2 w = *(const uint2*)((const uint8_t*)a.vc + (hb * hd + 16 * dt + lr) * a.cap + tv);
                vb = i8x8_to_half8_perm(w.x, w.y);
            } else {
                vb = *(const half8_t*)((const _Float16*)a.vc + (hb * hd + 16 * dt + lr) * a.cap + tv);
            }
#pragma unroll
            for (int rt = 0; rt < AM_RT; rt++) o[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[rt], vb, o[rt][dt], 0, 0, 0);
        }
    }
    // ---- merge the 4 waves in LDS ----
#pragma unroll
    for (int rt = 0; rt < AM_RT; rt++) {
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = o[rt][dt][i] + __shfl_xor(o[rt][dt][i], 32, 64);
                if (lg < 2) mg_o[wid][rt * 8 + rb + i][16 * dt + lr] = v;
            }
        if (lg < 2 && lr == 0)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                mg_m[wid][rt * 8 + rb + i] = mrow[rt][i];
                mg_l[wid][rt * 8 + rb + i] = lrow[rt][i];
            }
    }
    __syncthreads();
    const size_t grp = ((size_t)seq * a.n_kv + kvh) * a.ntiles + tile;
    const size_t rec = (size_t)hd + 2;
    float* part = a.part + (grp * a.nchunks + chunk) * (size_t)32 * rec;
    for (int r = wid; r < R; r += 4) {
        float M = -INFINITY;
        for (int w = 0; w < 4; w++) M = fmaxf(M, mg_m[w][r]);
        float L = 0.f, acc0 = 0.f, acc1 = 0.f;
        for (int w = 0; w < 4; w++) {
            const float mw = mg_m[w][r];
            const float sc = mw == -INFINITY ? 0.f : expf(mw - M);
            L += mg_l[w][r] * sc;
            acc0 += mg_o[w][r][lane] * sc;
            acc1 += mg_o[w][r][64 + lane] * sc;
        }
        float* pr = part + (size_t)r * rec;
        st_coh(&pr[2 + lane], acc0);
        st_coh(&pr[2 + 64 + lane], acc1);
        if (lane == 0) {
            st_coh(&pr[0], M);
            st_coh(&pr[1], L);
        }
    }
    if (!arrive_last(&a.counters[grp], (unsigned)a.nchunks, &s_last)) return;
    const float* gp = a.part + grp * a.nchunks * (size_t)32 * rec;
    for (int r = wid; r < R; r += 4) {
        float M = -INFINITY;
        for (int c = 0; c < a.nchunks; c++) M = fmaxf(M, ld_coh(&gp[((size_t)c * 32 + r) * rec]));
        float L = 0.f, acc0 = 0.f, acc1 = 0.f;
        for (int c = 0; c < a.nchunks; c++) {
            const float* pr = gp + ((size_t)c * 32 + r) * rec;
            const float mc = ld_coh(&pr[0]);
            const float w = (mc == -INFINITY) ? 0.f : expf(mc - M);
            L += ld_coh(&pr[1]) * w;
            acc0 += ld_coh(&pr[2 + lane]) * w;
            acc1 += ld_coh(&pr[2 + 64 + lane]) * w;
        }
        const float inv = L > 0.f ? 1.0f / L : 0.f;
        const int rr = r0 + r;
        const int s = rr / G, g = rr % G;
        float* out = a.out + (size_t)(seq * a.S + s) * QD + (kvh + g * a.n_kv) * hd;
        out[lane] = acc0 * inv;
        out[64 + lane] = acc1 * inv;
    }
}

int launch_attention(const AttnArgs& a, hipStream_t stream) {
    const int grid = a.nseq * a.n_kv * a.ntiles * a.nchunks;
    (void)hipGetLastError();
    if ((a.kv_fmt == KV_INT8 || a.kv_fmt == KV_F16) && a.hd == AM_HD) {
        if (a.rows_per_tile > AM_ROWS || a.chunk % 128) return 3;
        if (a.kv_fmt == KV_INT8)
            hipLaunchKernelGGL(attn_mfma_kernel<KV_INT8>, dim3(grid), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL(attn_mfma_kernel<KV_F16>, dim3(grid), dim3(256), 0, stream, a);
        return note_error(hipGetLastError()) ? 4 : 0;
    }
    if (a.hd > AT_MAXHD || a.rows_per_tile > AT_MAXR || a.rows_per_tile <= 0) return 3;
    hipLaunchKernelGGL(attn_kernel, dim3(grid), dim3(AT_THREADS), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

bool attention_uses_mfma(int kv_fmt, int hd) { return (kv_fmt == KV_INT8 || kv_fmt == KV_F16) && hd == AM_HD; }

}  // namespace aarh
