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
#include "frag.hpp"

namespace aarh {

static constexpr int AT_THREADS = 256;  // 4 waves
static constexpr int AT_TOK = 64;       // tokens per LDS sub-block
static constexpr int AT_MAXR = 32;      // query rows per workgroup
static constexpr int AT_MAXHD = 128;

// Append one new K / V row (position t of pos0 .. kv_len-1, post-RoPE f32 rows
// written by the QKV projection) to the cache of (slot, kv head); one wave.
// INT8: per token, per kv head absmax scale (1.0 when <= eps) kept as fp16,
// codes rounded from the f32 scale.
// The row's values for this lane (dims lane, lane + 64) are loaded by
// load_kv_token so that several tokens' loads share one round trip.
struct KvNew {
    float v[2][2];  // [K / V][dim lane, lane + 64]
};
__device__ __forceinline__ KvNew load_kv_token(const AttnArgs& a, int seq, int kvh, int pos0, int t) {
    const int lane = threadIdx.x & 63;
    const int hd = a.hd, KD = a.n_kv * hd;
    const size_t row = (size_t)seq * a.S + (t - pos0);
    KvNew r;
#pragma unroll
    for (int which = 0; which < 2; which++) {
        const float* src = a.knew + row * 2 * KD + (size_t)which * KD + (size_t)kvh * hd;
        r.v[which][0] = lane < hd ? src[lane] : 0.f;
        r.v[which][1] = lane + 64 < hd ? src[lane + 64] : 0.f;
    }
    return r;
}
__device__ __forceinline__ void store_kv_token(const AttnArgs& a, size_t hb, int t, const KvNew& nv) {
    const int lane = threadIdx.x & 63;
    const int hd = a.hd;
#pragma unroll
    for (int which = 0; which < 2; which++) {
        const float v0 = nv.v[which][0], v1 = nv.v[which][1];
        auto kdst = [&](int d) { return k_off(hb, t, d, a.cap, hd, a.kv_fmt); };
        auto vdst = [&](int d) { return vt_off(hb, d, t, a.cap, hd, a.kv_fmt); };  // V^T
        if (a.kv_fmt == KV_INT8) {
            const float amax = wave_max_f32(fmaxf(fabsf(v0), fabsf(v1)));
            const float sc = amax <= FLT_EPSILON ? 1.0f : amax / 127.0f;
            const int8_t q0 = (int8_t)fminf(fmaxf(roundf(v0 / sc), -127.0f), 127.0f);
            const int8_t q1 = (int8_t)fminf(fmaxf(roundf(v1 / sc), -127.0f), 127.0f);
            const uint16_t sh = __builtin_bit_cast(uint16_t, (_Float16)sc);
            if (which == 0) {
                int8_t* kc = (int8_t*)a.kc;
                if (lane < hd) kc[kdst(lane)] = q0;
                if (lane + 64 < hd) kc[kdst(lane + 64)] = q1;
                if (lane == 0) ((uint16_t*)a.ks)[hb * a.cap + t] = sh;
            } else {
                int8_t* vc = (int8_t*)a.vc;
                if (lane < hd) vc[vdst(lane)] = q0;
                if (lane + 64 < hd) vc[vdst(lane + 64)] = q1;
                if (lane == 0) ((uint16_t*)a.vs)[hb * a.cap + t] = sh;
            }
        } else if (a.kv_fmt == KV_F16) {
            _Float16* dst = (_Float16*)(which == 0 ? a.kc : a.vc);
            if (lane < hd) dst[which == 0 ? kdst(lane) : vdst(lane)] = (_Float16)v0;
            if (lane + 64 < hd) dst[which == 0 ? kdst(lane + 64) : vdst(lane + 64)] = (_Float16)v1;
        } else {
            float* dst = (float*)(which == 0 ? a.kc : a.vc);
            if (lane < hd) dst[which == 0 ? kdst(lane) : vdst(lane)] = v0;
            if (lane + 64 < hd) dst[which == 0 ? kdst(lane + 64) : vdst(lane + 64)] = v1;
        }
    }
}
__device__ __forceinline__ void append_kv_token(const AttnArgs& a, int seq, int kvh, size_t hb, int pos0, int t) {
    store_kv_token(a, hb, t, load_kv_token(a, seq, kvh, pos0, t));
}

// Append this launch's new positions that fall in [t_begin, t_end), spread over the
// workgroup's waves.  Every workgroup whose chunk covers a new position writes it
// (identical bytes) before it reads the chunk, so no other launch is needed.
// Returns with the writes visible to the workgroup.
__device__ void append_new_kv(const AttnArgs& a, int seq, int kvh, size_t hb, int pos0, int t_begin, int t_end) {
    const int lo = max(t_begin, pos0);
    if (lo >= t_end) return;  // uniform over the workgroup
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    for (int t = lo + wid; t < t_end; t += nw) append_kv_token(a, seq, kvh, hb, pos0, t);
    __threadfence_block();
    __syncthreads();
}

__global__ void __launch_bounds__(AT_THREADS) attn_kernel(AttnArgs a) {
    __shared__ float qs[AT_MAXR][AT_MAXHD];
    __shared__ float ks[AT_TOK][AT_MAXHD + 1];
    __shared__ float vs[AT_TOK][AT_MAXHD + 1];
    __shared__ float ps[AT_MAXR][AT_TOK];
    __shared__ unsigned s_last;

    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
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
    append_new_kv(a, seq, kvh, (size_t)sl * a.n_kv + kvh, pos0, t_begin, t_end);
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
                kv_ = (float)((const int8_t*)a.kc)[k_off(head_base, tt, d, a.cap, hd, KV_INT8)] * ksc;
                vv_ = (float)((const int8_t*)a.vc)[vt_off(head_base, d, tt, a.cap, hd, KV_INT8)] * vsc;
            } else if (a.kv_fmt == KV_F16) {
                kv_ = (float)((const _Float16*)a.kc)[k_off(head_base, tt, d, a.cap, hd, KV_F16)];
                vv_ = (float)((const _Float16*)a.vc)[vt_off(head_base, d, tt, a.cap, hd, KV_F16)];
            } else {
                kv_ = ((const float*)a.kc)[k_off(head_base, tt, d, a.cap, hd, KV_F32)];
                vv_ = ((const float*)a.vc)[vt_off(head_base, d, tt, a.cap, hd, KV_F32)];
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
                // one accumulation chain in dimension order; unrolled so the LDS reads of
                // later dimensions are in flight while earlier products accumulate
                float dot = 0.f;
#pragma unroll 16
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
#pragma unroll 8
            for (int t = 0; t < nt; t++) {
                float p = ps[r][t];
                a0 = fmaf(p, vs[t][lane], a0);
                if (lane + 64 < hd) a1 = fmaf(p, vs[t][lane + 64], a1);
            }
            o0[j] += a0;
            o1[j] += a1;
        }
    }

    if (a.nchunks == 1) {
        // one chunk: its (m, l, O) is the result (the merge below would weight it by exp(0) = 1)
#pragma unroll
        for (int j = 0; j < AT_MAXR / 4; j++) {
            const int r = wid + 4 * j;
            if (r >= R) break;
            const float inv = lrow[j] > 0.f ? 1.0f / lrow[j] : 0.f;
            const int rr = r0 + r;
            const int h = kvh + (rr % G) * a.n_kv;
            const int orow = seq * a.S + rr / G;
            float* out = a.out + (size_t)orow * QD + h * hd;
            if (lane < hd) out[lane] = o0[j] * inv;
            if (lane + 64 < hd) out[lane + 64] = o1[j] * inv;
            if (a.fo.buf) {
                if (lane < hd) frag_put(a.fo, orow, h * hd + lane, o0[j] * inv);
                if (lane + 64 < hd) frag_put(a.fo, orow, h * hd + lane + 64, o1[j] * inv);
            }
        }
        return;
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
        const int orow = seq * a.S + s;
        float* out = a.out + (size_t)orow * QD + h * hd;
        if (lane < hd) out[lane] = acc0 * inv;
        if (lane + 64 < hd) out[lane + 64] = acc1 * inv;
        if (a.fo.buf) {
            if (lane < hd) frag_put(a.fo, orow, h * hd + lane, acc0 * inv);
            if (lane + 64 < hd) frag_put(a.fo, orow, h * hd + lane + 64, acc1 * inv);
        }
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
    // v_perm_b32 places bytes (0, 2) or (1, 3) under 0x64 high bytes: fp16 1024 + (b ^ 0x80)
    const half2v_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    constexpr uint32_t HI = 0x64646464u, SEL_EVEN = 0x04020400u, SEL_ODD = 0x04030401u;
    d0 ^= 0x80808080u;
    d1 ^= 0x80808080u;
    half2v_t h0 = __builtin_bit_cast(half2v_t, __builtin_amdgcn_perm(HI, d0, SEL_EVEN)) - off;
    half2v_t h1 = __builtin_bit_cast(half2v_t, __builtin_amdgcn_perm(HI, d0, SEL_ODD)) - off;
    half2v_t h2 = __builtin_bit_cast(half2v_t, __builtin_amdgcn_perm(HI, d1, SEL_EVEN)) - off;
    half2v_t h3 = __builtin_bit_cast(half2v_t, __builtin_amdgcn_perm(HI, d1, SEL_ODD)) - off;
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

static constexpr int AM_ROWS = 16;          // query rows per workgroup (one MFMA column tile)
static constexpr int AM_HD = 128;
static constexpr int AM_WAVES = 8;          // 512 threads; wave w takes 32-token blocks w, w+8, ...
static constexpr int AM_TAIL = AM_WAVES - 1;  // INT8 path: the wave that appends and reads the new positions
static constexpr int AM_HAND = 2;             // old blocks the tail wave hands over beyond its tail blocks
static constexpr int AM_SOLO = 2;             // at most this many tail blocks go to the tail wave alone
static constexpr int AM_REC = AM_HD + 4;    // partial record: m, l, pad, pad, o[hd]
static constexpr int AM_MAXCH = 32;         // chunks one merge combines
static constexpr int AM_STAGE = 2 * 32 * AM_HD + 512;  // one INT8 block staged in LDS: K, V^T, scales
static constexpr float AM_LOG2E = 1.4426950408889634f;

// Raw K/V operands of one 32-token block for one lane (lane = (lr, lg)).
// K: token rows 8*(lr/4) + 4*ts + lr%4 of the block, dims 32*lg..+32.
// V^T: dim rows 16*dt + lr, tokens 8*lg..+8.  Scales: tokens 8*lg..+8.
// Vector-register types (not HIP's struct uint4) so a block stays in VGPRs.
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4v_t __attribute__((ext_vector_type(4)));
template <int KVF>
struct KvRaw;
template <>
struct KvRaw<KV_INT8> {
    u32x4v_t k[2][2];
    u32x4v_t ksc;
    u32x2_t v[8];
    u32x4v_t vsc;
};
template <>
struct KvRaw<KV_F16> {
    u32x4v_t k[2][4];
    u32x4v_t v[8];
};

// Loads are issued in the order they are consumed (K, K scales, V, V scales),
// so the scores of a block wait only for its K half.
template <int KVF>
__device__ __forceinline__ void load_kv_block(const AttnArgs& a, size_t hb, int tb, int lr, int lg, KvRaw<KVF>& r) {
    // K: chunk (ts, c) of every lane is one contiguous 1 KiB run of the block (k_off)
    const int lane = 16 * lg + lr;
    const uint8_t* kb = (const uint8_t*)a.kc + (hb * a.cap + tb) * AM_HD * (KVF == KV_INT8 ? 1 : 2);
#pragma unroll
    for (int ts = 0; ts < 2; ts++) {
        if constexpr (KVF == KV_INT8) {
#pragma unroll
            for (int c = 0; c < 2; c++) r.k[ts][c] = *(const u32x4v_t*)(kb + ((ts * 2 + c) * 64 + lane) * 16);
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) r.k[ts][c] = *(const u32x4v_t*)(kb + ((ts * 4 + c) * 64 + lane) * 16);
        }
    }
    if constexpr (KVF == KV_INT8) r.ksc = *(const u32x4v_t*)(a.ks + hb * a.cap + tb + 8 * lg);
#pragma unroll
    for (int dt = 0; dt < 8; dt++) {
        if constexpr (KVF == KV_INT8)
            r.v[dt] = *(const u32x2_t*)((const uint8_t*)a.vc + vt_off(hb, 16 * dt + lr, tb + 8 * lg, a.cap, AM_HD, KV_INT8));
        else
            r.v[dt] = *(const u32x4v_t*)((const _Float16*)a.vc + vt_off(hb, 16 * dt + lr, tb + 8 * lg, a.cap, AM_HD, KV_F16));
    }
    if constexpr (KVF == KV_INT8) r.vsc = *(const u32x4v_t*)(a.vs + hb * a.cap + tb + 8 * lg);
}

template <int KVF>
__device__ __forceinline__ half8_t k_operand(const KvRaw<KVF>& r, int ts, int kk) {
    if constexpr (KVF == KV_INT8) {
        const u32x4v_t w = r.k[ts][kk >> 1];
        return (kk & 1) ? i8x8_to_half8_perm(w.z, w.w) : i8x8_to_half8_perm(w.x, w.y);
    } else {
        return __builtin_bit_cast(half8_t, r.k[ts][kk]);
    }
}
template <int KVF>
__device__ __forceinline__ half8_t v_operand(const KvRaw<KVF>& r, int dt) {
    if constexpr (KVF == KV_INT8) return i8x8_to_half8_perm(r.v[dt].x, r.v[dt].y);
    else return __builtin_bit_cast(half8_t, r.v[dt]);
}
// fp16 scale of token 8*lg + idx (idx = 4*ts + i)
__device__ __forceinline__ float scale_at(u32x4v_t s, int idx) {
    const uint32_t w = idx < 2 ? s.x : idx < 4 ? s.y : idx < 6 ? s.z : s.w;
    return (float)__builtin_bit_cast(_Float16, (uint16_t)((idx & 1) ? (w >> 16) : (w & 0xFFFFu)));
}

// k-slot j of an 8-block holds element perm(j): the order i8x8_to_half8_perm emits
template <int KVF>
__device__ __forceinline__ constexpr int slot_elem(int j) {
    if constexpr (KVF == KV_INT8) return (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1);
    else return j;
}

// reductions over the four 16-lane rows of a wave (lanes lr, lr+16, lr+32, lr+48)
__device__ __forceinline__ float rows_max(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Output dims ocol .. ocol+3 of row orow held by lane q of a row's 32 lanes (ocol % 8 == 0 for
// even q): lanes q and q ^ 1 together form one 8-column fragment entry, written by the even lane.
__device__ __forceinline__ void frag_out_pair(const XFrag& fo, int orow, int ocol, float4_t o4, int q) {
    float4_t p;
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __shfl_xor(o4[i], 1, 64);
    if (q & 1) return;
    float v[8] = {o4[0], o4[1], o4[2], o4[3], p[0], p[1], p[2], p[3]};
    if (fo.norm_w)
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] *= fo.norm_w[ocol + e];
    frag_put8_w(fo, orow, ocol, v);
}

// Flash-decode attention on MFMA for head_dim 128 and fp16 / INT8 caches.
// Workgroup = (sequence, kv head, tile of <= 16 query rows, token chunk), 8 waves;
// wave w takes the chunk's 32-token blocks w, w+8, ... (INT8: the blocks before the
// new positions; the blocks holding new positions go to one wave, which appends
// them) with the next block's loads in flight while the current one computes.  Scores are computed
// transposed, S^T = K Q^T (A = K rows, B = Q^T as fp16 hi and lo halves), so the
// MFMA result layout (lane = query row, 8 tokens per lane) is directly the B
// operand of O^T = V^T P^T: no LDS round trip, and the row statistics live in
// the lane of their row.  Softmax runs in base 2 (v_exp_f32).  With one chunk
// the workgroup writes the output; otherwise chunk partials go out with
// coherent 16-byte stores and the last workgroup of the group merges them.
template <int KVF, int DEPTH, bool DMA>
__global__ void __launch_bounds__(512) attn_mfma_kernel(AttnArgs a) {
    // dynamic LDS: the DMA block stages during the token loop, then the wave merge
    extern __shared__ __attribute__((aligned(1024))) char am_lds[];
    float (*mg_o)[AM_ROWS][AM_REC] = reinterpret_cast<float (*)[AM_ROWS][AM_REC]>(am_lds);
    __shared__ float mg_m[AM_WAVES][AM_ROWS], mg_l[AM_WAVES][AM_ROWS];
    __shared__ unsigned s_last;

    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int G = a.n_heads / a.n_kv;
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
    const int QD = a.n_heads * AM_HD;
    const size_t hb = (size_t)sl * a.n_kv + kvh;
    const int t_begin = chunk * a.chunk;
    const int t_end = min(kv_len, t_begin + a.chunk);
    constexpr int STEP = 32 * AM_WAVES;
    int tb = t_begin + 32 * wid;
    const int t_chunk_last = (t_end - 1) & ~31;
    // register-ring path: the wave's own last block (re-reads hit L1), or the chunk's last one
    // for a wave without blocks
    const int t_last = tb <= t_chunk_last ? tb + (t_chunk_last - tb) / STEP * STEP : t_chunk_last;

    // INT8 blocks stream into two LDS stages per wave with direct loads (no VGPRs held
    // in flight, waits counted in the token loop): K 4 KiB, V^T 4 KiB, then 256 bytes
    // each of K and V scales (tokens 2l, 2l+1 in lane l < 16).
    constexpr int KVB = 32 * AM_HD;  // bytes of K (and of V) per block
    char* st0 = am_lds + wid * 2 * AM_STAGE;
    const __amdgpu_buffer_rsrc_t kr = coh_rsrc((const uint8_t*)a.kc + hb * a.cap * AM_HD);
    const __amdgpu_buffer_rsrc_t vr = coh_rsrc((const uint8_t*)a.vc + hb * a.cap * AM_HD);
    const __amdgpu_buffer_rsrc_t ksr = coh_rsrc(a.ks + hb * a.cap), vsr = coh_rsrc(a.vs + hb * a.cap);
    const int sc_voff = (lane & 15) * 4;
    auto issue = [&](char* st, int t) __attribute__((always_inline)) {
        t = __builtin_amdgcn_readfirstlane(t);  // wave-uniform: the loads take it as a scalar offset
#pragma unroll
        for (int p = 0; p < 4; p++) lds_dma16<true>(kr, st + p * 1024, lane * 16 + p * 1024, t * AM_HD);
#pragma unroll
        for (int p = 0; p < 4; p++) lds_dma16<true>(vr, st + KVB + p * 1024, lane * 16 + p * 1024, t * AM_HD);
        lds_dma4<true>(ksr, st + 2 * KVB, sc_voff, t * 2);
        lds_dma4<true>(vsr, st + 2 * KVB + 256, sc_voff, t * 2);
    };
    // DMA schedule: the blocks wholly before the new positions ("old" blocks) go round
    // robin to the eight waves; the blocks holding new positions ("tail" blocks) come
    // first in their wave's list, and that wave writes the new positions into its staged
    // copy of the block (patch_tail) and stores the block back whole, so no wave waits
    // for the cache append (a workgroup barrier after a byte-wise append held every wave
    // until the appending waves' loads and stores came back).  One or two tail blocks
    // (decode and verify) all go to wave AM_TAIL, which hands its last n_tail + AM_HAND
    // old blocks to wave 0 (the oldest wave of the workgroup, whose stream ends first:
    // issue arbitration favours it, and timestamps put its stream's end 9 us before the
    // others' at B = 32).  More tail blocks (prompt chunks) go round robin like the old
    // ones.  Wave wid's i-th block: tb_of(i); a wave issues no load past its last block.
    const int tail_start = pos0 < t_end ? max(t_begin, pos0 & ~31) : t_end;
    const int n_old = (tail_start - t_begin) >> 5, n_tail = (t_end - tail_start + 31) >> 5;
    auto own = [&](int n, int w) { return n > w ? (n - w + AM_WAVES - 1) / AM_WAVES : 0; };
    const bool solo = n_tail <= AM_SOLO;
    const int t_old = own(n_old, AM_TAIL), n_moved = solo && n_tail > 0 ? min(n_tail + AM_HAND, t_old) : 0;
    const int n_lead = solo ? (wid == AM_TAIL ? n_tail : 0) : own(n_tail, wid);  // tail blocks first
    const int n_first = solo && wid == AM_TAIL ? t_old - n_moved : own(n_old, wid);  // strided old blocks
    const int n_blk = n_lead + n_first + (wid == 0 ? n_moved : 0);
    auto tb_of = [&](int i) __attribute__((always_inline)) {
        i = min(i, n_blk - 1);
        if (i < n_lead) return tail_start + 32 * (solo ? i : wid + AM_WAVES * i);
        i -= n_lead;
        if (i < n_first) return t_begin + 32 * (wid + AM_WAVES * i);
        return t_begin + 32 * (AM_TAIL + AM_WAVES * (t_old - n_moved + i - n_first));  // handed over
    };
    // The cache append of tail block tb (positions max(tb, pos0) .. min(tb + 32, t_end) - 1,
    // the bytes append_kv_token writes), made in the block's landed stage; the patched
    // block then goes back to the cache whole, in the 16-byte runs the loads read.
    // The wave holding the first tail block loads the first four new rows before any
    // block (ahead of the block loads in the memory pipeline); other rows are loaded
    // when their block is patched.
    const int first_new = max(t_begin, pos0);
    const bool has_first = n_lead > 0 && (solo || wid == 0);
    KvNew pre[4];
    if (DMA && has_first)
#pragma unroll
        for (int j = 0; j < 4; j++) pre[j] = load_kv_token(a, seq, kvh, pos0, min(first_new + j, t_end - 1));
    auto patch_tail = [&](char* st, int tb) __attribute__((always_inline)) {
        const int lo = max(tb, pos0), hi = min(tb + 32, t_end);
        for (int t0 = lo; t0 < hi; t0 += 4) {
            KvNew nv[4];
            if (has_first && t0 == first_new) {
#pragma unroll
                for (int j = 0; j < 4; j++) nv[j] = pre[j];
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) nv[j] = load_kv_token(a, seq, kvh, pos0, min(t0 + j, hi - 1));
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (t0 + j >= hi) break;
                const int r = t0 + j - tb;
#pragma unroll
                for (int which = 0; which < 2; which++) {
                    const float v0 = nv[j].v[which][0], v1 = nv[j].v[which][1];
                    const float amax = wave_max_f32(fmaxf(fabsf(v0), fabsf(v1)));
                    const float sc = amax <= FLT_EPSILON ? 1.0f : amax / 127.0f;
                    const int8_t q0 = (int8_t)fminf(fmaxf(roundf(v0 / sc), -127.0f), 127.0f);
                    const int8_t q1 = (int8_t)fminf(fmaxf(roundf(v1 / sc), -127.0f), 127.0f);
                    const uint16_t sh = __builtin_bit_cast(uint16_t, (_Float16)sc);
                    if (which == 0) {
                        st[k_off(0, r, lane, a.cap, AM_HD, KV_INT8)] = q0;
                        st[k_off(0, r, lane + 64, a.cap, AM_HD, KV_INT8)] = q1;
                        if (lane == 0) *(uint16_t*)(st + 2 * KVB + 2 * r) = sh;
                    } else {
                        st[KVB + vt_off(0, lane, r, a.cap, AM_HD, KV_INT8)] = q0;
                        st[KVB + vt_off(0, lane + 64, r, a.cap, AM_HD, KV_INT8)] = q1;
                        if (lane == 0) *(uint16_t*)(st + 2 * KVB + 256 + 2 * r) = sh;
                    }
                }
            }
        }
        uint8_t* kb = (uint8_t*)a.kc + (hb * a.cap + tb) * AM_HD;
        uint8_t* vb = (uint8_t*)a.vc + (hb * a.cap + tb) * AM_HD;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            *(u32x4v_t*)(kb + p * 1024 + lane * 16) = *(const u32x4v_t*)(st + p * 1024 + lane * 16);
            *(u32x4v_t*)(vb + p * 1024 + lane * 16) = *(const u32x4v_t*)(st + KVB + p * 1024 + lane * 16);
        }
        if (lane < 16) {
            *(uint32_t*)((uint8_t*)((uint16_t*)a.ks + hb * a.cap + tb) + lane * 4) = *(const uint32_t*)(st + 2 * KVB + lane * 4);
            *(uint32_t*)((uint8_t*)((uint16_t*)a.vs + hb * a.cap + tb) + lane * 4) =
                *(const uint32_t*)(st + 2 * KVB + 256 + lane * 4);
        }
    };
    if constexpr (DMA) {
        if (n_blk > 0) {
            issue(st0, tb_of(0));
            if (n_blk > 1) issue(st0 + AM_STAGE, tb_of(1));
        }
    } else {
        if (t_end > pos0) append_new_kv(a, seq, kvh, hb, pos0, t_begin, t_end);
    }

    // ---- this lane's query row (lr): Q^T B operand, hi/lo, dims 32*lg + 8*kk + slot ----
    const bool row_ok = lr < R;
    int lim = -1;
    const float* qp = a.q;
    if (row_ok) {
        const int real = r0 + lr, s = real / G, g = real % G;
        lim = pos0 + s;
        qp = a.q + (size_t)(seq * a.S + s) * QD + (kvh + g * a.n_kv) * AM_HD + 32 * lg;
    }
    float4_t qv[8];
#pragma unroll
    for (int u = 0; u < 8; u++) qv[u] = row_ok ? *(const float4_t*)(qp + 4 * u) : (float4_t){0.f, 0.f, 0.f, 0.f};

    // Block ring of DEPTH + 1 register buffers, rotated by unrolling (no copies:
    // a register copy of a block still in flight would wait for every load).
    // Loads past the wave's last block re-read the chunk's last block (in
    // bounds, results unused), so inside a non-empty chunk every load is
    // unconditional; an empty chunk (past the sequence's length) loads nothing.
    KvRaw<KVF> ring[DEPTH + 1];
    if (!DMA && t_end > t_begin) {
#pragma unroll
        for (int d = 0; d < DEPTH; d++) load_kv_block<KVF>(a, hb, min(tb + d * STEP, t_last), lr, lg, ring[d]);
    }

    half8_t qh[4], ql[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int e = 8 * kk + slot_elem<KVF>(j);
            const float v = qv[e >> 2][e & 3];
            const _Float16 hi = (_Float16)v;
            qh[kk][j] = hi;
            ql[kk][j] = (_Float16)(v - (float)hi);
        }

    float m = -INFINITY, l = 0.f;
    float4_t o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o[dt] = (float4_t){0.f, 0.f, 0.f, 0.f};
    const float sc2 = a.scale * AM_LOG2E;

    auto block = [&](const KvRaw<KVF>& cur) __attribute__((always_inline)) {
        // ---- S^T = K Q^T: lane holds tokens 8*lg + 4*ts + i of row lr ----
        float4_t st[2];
#pragma unroll
        for (int ts = 0; ts < 2; ts++) {
            float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const half8_t ka = k_operand<KVF>(cur, ts, kk);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[kk], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[kk], acc, 0, 0, 0);
            }
            st[ts] = acc;
        }
        float s[8];
        float mx = -INFINITY;
        // a block wholly inside the chunk and before every row's own position needs no mask
        // (wave-uniform: tb is the wave's block)
        if (tb + 32 <= t_end && tb + 31 <= pos0) {
#pragma unroll
            for (int idx = 0; idx < 8; idx++) {
                float ksc = sc2;
                if constexpr (KVF == KV_INT8) ksc *= scale_at(cur.ksc, idx);
                s[idx] = st[idx >> 2][idx & 3] * ksc;
                mx = fmaxf(mx, s[idx]);
            }
        } else {
#pragma unroll
            for (int idx = 0; idx < 8; idx++) {
                const int tok = tb + 8 * lg + idx;
                float ksc = sc2;
                if constexpr (KVF == KV_INT8) ksc *= scale_at(cur.ksc, idx);
                const float v = st[idx >> 2][idx & 3] * ksc;
                s[idx] = (tok < t_end && tok <= lim) ? v : -INFINITY;
                mx = fmaxf(mx, s[idx]);
            }
        }
        mx = rows_max(mx);
        const float mnew = fmaxf(m, mx);
        const float alpha = mnew == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mnew);
        float p[8], ps = 0.f;
#pragma unroll
        for (int idx = 0; idx < 8; idx++) {
            p[idx] = s[idx] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s[idx] - mnew);
            ps += p[idx];
        }
        ps = rows_sum(ps);
        l = l * alpha + ps;
        m = mnew;
        // rescale only when some row's maximum moved (a factor of exactly 1 changes nothing)
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < 8; dt++) o[dt] *= alpha;
        }
        // ---- P^T B operand (hi / lo), slot j <-> token 8*lg + slot_elem(j) ----
        half8_t ph, pl;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int idx = slot_elem<KVF>(j);
            float pv = p[idx];
            if constexpr (KVF == KV_INT8) pv *= scale_at(cur.vsc, idx);
            const _Float16 hi = (_Float16)pv;
            ph[j] = hi;
            pl[j] = (_Float16)(pv - (float)hi);
        }
        // ---- O^T += V^T P^T ----
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const half8_t va = v_operand<KVF>(cur, dt);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[dt], 0, 0, 0);
        }
    };
    if constexpr (DMA) {
        static_assert(KVF == KV_INT8, "DMA staging is laid out for INT8 blocks");
        // A block is copied to registers as soon as it lands and its stage is refilled
        // at once, so both stages stay in flight while the block is computed.
        constexpr int NL = 10;  // DMA loads per block
        for (int i = 0; i < n_blk; i++) {
            tb = tb_of(i);
            char* cur_st = st0 + (i & 1) * AM_STAGE;
            // block i has landed; block i + 1 (the only loads issued after it) may still be in flight
            if (i + 1 < n_blk) wait_vmcnt<NL>();
            else wait_vmcnt<0>();
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (i < n_lead) patch_tail(cur_st, tb);
            KvRaw<KVF> cur;
#pragma unroll
            for (int ts = 0; ts < 2; ts++)
#pragma unroll
                for (int c = 0; c < 2; c++) cur.k[ts][c] = *(const u32x4v_t*)(cur_st + ((ts * 2 + c) * 64 + lane) * 16);
#pragma unroll
            for (int dt = 0; dt < 8; dt++) cur.v[dt] = *(const u32x2_t*)(cur_st + KVB + (16 * dt + lr) * 32 + 8 * lg);
            cur.ksc = *(const u32x4v_t*)(cur_st + 2 * KVB + 16 * lg);
            cur.vsc = *(const u32x4v_t*)(cur_st + 2 * KVB + 256 + 16 * lg);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the stage has been read
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (i + 2 < n_blk) issue(cur_st, tb_of(i + 2));
            block(cur);
        }
        wait_vmcnt<0>();
        __syncthreads();  // every wave's stages are idle before the merge reuses the LDS
    } else {
        for (; tb < t_end;) {
#pragma unroll
            for (int d = 0; d <= DEPTH; d++) {
                if (tb >= t_end) break;
                load_kv_block<KVF>(a, hb, min(tb + DEPTH * STEP, t_last), lr, lg, ring[(d + DEPTH) % (DEPTH + 1)]);
                __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the block's math
                block(ring[d]);
                tb += STEP;
            }
        }
    }
    // ---- merge the waves in LDS: lane holds O^T[16*dt + 4*lg + i][lr] ----
#pragma unroll
    for (int dt = 0; dt < 8; dt++) *(float4_t*)&mg_o[wid][lr][4 + 16 * dt + 4 * lg] = o[dt];
    if (lg == 0) {
        mg_m[wid][lr] = m;
        mg_l[wid][lr] = l;
    }
    __syncthreads();
    // thread -> (row r, 4 dims at 4*q); 16 rows x 32 quads = 512 threads
    const int r = tid >> 5, q = tid & 31;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < AM_WAVES; w++) M = fmaxf(M, mg_m[w][r]);
    float L = 0.f;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < AM_WAVES; w++) {
        const float mw = mg_m[w][r];
        const float sc = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        L += mg_l[w][r] * sc;
        acc += *(const float4_t*)&mg_o[w][r][4 + 4 * q] * sc;
    }
    const int rr = r0 + r;
    const int orow = seq * a.S + rr / G, ocol = (kvh + (rr % G) * a.n_kv) * AM_HD + 4 * q;
    float* out = a.out;
    if (r < R) out += (size_t)orow * QD + ocol;
    if (a.nchunks == 1) {
        if (r < R) {
            const float4_t o4 = acc * (L > 0.f ? 1.0f / L : 0.f);
            *(float4_t*)out = o4;
            if (a.fo.buf) frag_out_pair(a.fo, orow, ocol, o4, q);
        }
        return;
    }
    const size_t grp = ((size_t)seq * a.n_kv + kvh) * a.ntiles + tile;
    const __amdgpu_buffer_rsrc_t prs = coh_rsrc(a.part + grp * a.nchunks * (size_t)AM_ROWS * AM_REC);
    if (r < R) {
        const unsigned rec_off = (unsigned)((chunk * AM_ROWS + r) * AM_REC) * 4u;
        st4_coh(prs, rec_off + 16u + 16u * q, acc);
        if (q == 0) st4_coh(prs, rec_off, (float4_t){M, L, 0.f, 0.f});
    }
    if (!arrive_last(&a.counters[grp], (unsigned)a.nchunks, &s_last)) return;

    // ---- last workgroup: merge the chunks in chunk order.  Every chunk's (max, sum)
    //      header of the thread's row and every chunk's 4 dims of the thread are loaded
    //      at once (one round trip for up to AM_MAXCH chunks); then the row maximum over
    //      the chunks and the weighted sums, chunk by chunk. ----
    if (r >= R) return;
    const int C = a.nchunks;
    const unsigned rbase = (unsigned)(r * AM_REC) * 4u;
    constexpr unsigned CSTRIDE = (unsigned)(AM_ROWS * AM_REC) * 4u;
    float2_t hl[AM_MAXCH];
    float4_t ov[AM_MAXCH];
#pragma unroll
    for (int c = 0; c < AM_MAXCH; c++)
        if (c < C) {
            hl[c] = ld2_coh(prs, rbase + (unsigned)c * CSTRIDE);
            ov[c] = ld4_coh(prs, rbase + (unsigned)c * CSTRIDE + 16u + 16u * q);
        }
    float Mc = -INFINITY;
#pragma unroll
    for (int c = 0; c < AM_MAXCH; c++)
        if (c < C) Mc = fmaxf(Mc, hl[c][0]);
    float4_t tot = {0.f, 0.f, 0.f, 0.f};
    float Lc = 0.f;
#pragma unroll
    for (int c = 0; c < AM_MAXCH; c++)
        if (c < C) {
            const float w = hl[c][0] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(hl[c][0] - Mc);
            Lc += hl[c][1] * w;
            tot += ov[c] * w;
        }
    const float4_t o4 = tot * (Lc > 0.f ? 1.0f / Lc : 0.f);
    *(float4_t*)out = o4;
    if (a.fo.buf) frag_out_pair(a.fo, orow, ocol, o4, q);
}

int launch_attention(const AttnArgs& a, hipStream_t stream) {
    const int grid = a.nseq * a.n_kv * a.ntiles * a.nchunks;
    (void)hipGetLastError();
    if ((a.kv_fmt == KV_INT8 || a.kv_fmt == KV_F16) && a.hd == AM_HD) {
        if (a.rows_per_tile > AM_ROWS || a.chunk % (32 * AM_WAVES) || a.nchunks > AM_MAXCH || a.cap % 32) return 3;
        static bool attr = false;
        constexpr size_t merge_bytes = sizeof(float) * AM_WAVES * AM_ROWS * AM_REC;
        constexpr size_t dma_bytes = (size_t)AM_WAVES * 2 * AM_STAGE;
        constexpr size_t i8_bytes = dma_bytes > merge_bytes ? dma_bytes : merge_bytes;
        if (!attr) {
            if (note_error(hipFuncSetAttribute((const void*)attn_mfma_kernel<KV_INT8, 1, true>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)i8_bytes)) ||
                note_error(hipFuncSetAttribute((const void*)attn_mfma_kernel<KV_F16, 1, false>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)merge_bytes)))
                return 4;
            attr = true;
        }
        if (a.kv_fmt == KV_INT8)
            launch_timed(attn_mfma_kernel<KV_INT8, 1, true>, dim3(grid), dim3(512), (uint32_t)i8_bytes, stream, a);
        else
            launch_timed(attn_mfma_kernel<KV_F16, 1, false>, dim3(grid), dim3(512), (uint32_t)merge_bytes, stream, a);
        return note_error(hipGetLastError()) ? 4 : 0;
    }
    if (a.hd > AT_MAXHD || a.rows_per_tile > AT_MAXR || a.rows_per_tile <= 0) return 3;
    launch_timed(attn_kernel, dim3(grid), dim3(AT_THREADS), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

bool attention_uses_mfma(int kv_fmt, int hd) { return (kv_fmt == KV_INT8 || kv_fmt == KV_F16) && hd == AM_HD; }

}  // namespace aarh
