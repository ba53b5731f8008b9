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
        if (lane < hd) pr[2 + lane] = o0[j];
        if (lane + 64 < hd) pr[2 + lane + 64] = o1[j];
        if (lane == 0) {
            pr[0] = mrow[j];
            pr[1] = lrow[j];
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = atomicAdd(&a.counters[grp], 1u);
        s_last = (prev == (unsigned)a.nchunks - 1u) ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (tid == 0) a.counters[grp] = 0u;
    // merge chunks in order
    const float* gp = a.part + grp * a.nchunks * (size_t)AT_MAXR * rec;
    for (int r = wid; r < R; r += 4) {
        float M = -INFINITY;
        for (int c = 0; c < a.nchunks; c++) M = fmaxf(M, gp[((size_t)c * AT_MAXR + r) * rec]);
        float L = 0.f, acc0 = 0.f, acc1 = 0.f;
        for (int c = 0; c < a.nchunks; c++) {
            const float* pr = gp + ((size_t)c * AT_MAXR + r) * rec;
            float mc = pr[0];
            float w = (mc == -INFINITY) ? 0.f : expf(mc - M);
            L += pr[1] * w;
            if (lane < hd) acc0 += pr[2 + lane] * w;
            if (lane + 64 < hd) acc1 += pr[2 + lane + 64] * w;
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

int launch_attention(const AttnArgs& a, hipStream_t stream) {
    if (a.hd > AT_MAXHD || a.rows_per_tile > AT_MAXR || a.rows_per_tile <= 0) return 3;
    const int grid = a.nseq * a.n_kv * a.ntiles * a.nchunks;
    (void)hipGetLastError();
    hipLaunchKernelGGL(attn_kernel, dim3(grid), dim3(AT_THREADS), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

}  // namespace aarh
