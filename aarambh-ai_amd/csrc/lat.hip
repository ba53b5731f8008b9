// Latent-attention (MLA) + fine-grained MoE decoder kernels for gfx950
// (benchmark config 5).
//
// MLA (nn/src/mla.rs:300-489): the cache holds c_kv = RMSNorm(kv_a_proj(x))
// and the shared rotary key k_rope per token.  Instead of reconstructing
// K_nope = up_k(c_kv) and V = up_v(c_kv) over the whole cache every step, as
// the reference does, the query is absorbed: q_lat_h = up_k_h^T q_nope_h, so
// score = q_lat_h . c_kv + q_rope_h . k_rope and o_h = up_v_h (sum_t p_t c_kv_t).
// All heads then read one latent row per token (multi-query attention over
// 576-wide keys and 512-wide values), on MFMA.
//
// MoE (nn/src/moe.rs:212-406): the router's top-k experts per row (softmax
// over the selected logits) and the shared experts become a list of
// (expert, row, weight) assignments; each expert's SwiGLU runs once over the
// rows routed to it (the reference runs every expert densely and multiplies
// the unselected ones by zero), and the outputs are combined per row in expert
// order, shared experts last.
#include "epilogue.hpp"

namespace aarh {

static constexpr float LAT_LOG2E = 1.4426950408889634f;
static constexpr int MOE_MAX_ROWS = 256;    // rows per routing launch
static constexpr int MOE_MAX_EXPERTS = 72;  // routed (<= 64) + shared experts

// Products of f32 values on MFMA: a = a_hi + a_lo and b = b_hi + b_lo in fp16,
// a.b ~= a_hi b_hi + a_hi b_lo + a_lo b_hi with f32 accumulation (about 22
// significant bits, like the f32 FMA chain it replaces).
__device__ __forceinline__ void split_f16x8(const float* v, half8_t& hi, half8_t& lo) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const _Float16 h = (_Float16)v[j];
        hi[j] = h;
        lo[j] = (_Float16)(v[j] - (float)h);
    }
}

__device__ __forceinline__ float4_t mfma3(const half8_t& ah, const half8_t& al, const half8_t& bh, const half8_t& bl,
                                         float4_t acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, acc, 0, 0, 0);
    return acc;
}

// ---------------------------------------------------------------------------
// q prep: rotate q_rope, absorb q_nope through up_k (q_lat = up_k_h^T q_nope_h)
// on MFMA.  Workgroup = 16 rows x 1 head x 64 latent columns, one 16x16 output
// tile per wave: A = q_nope rows (f32 split hi + lo), B = up_k^T hi + lo.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) mla_qprep_kernel(MlaArgs a) {
    const int M = a.nseq * a.S, h = blockIdx.y, mt = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, lr = lane & 15, lg = lane >> 4, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nope = a.nope, rd = a.rd, lat = a.lat, half = rd >> 1, KD = lat + rd;
    const int jt = blockIdx.z * 4 + wid;  // 16-column tile of q_lat
    if (jt * 16 < lat) {
        const int m = mt * 16 + lr;
        const float* arow = a.raw + (size_t)min(m, M - 1) * a.raw_ld + h * (nope + rd);
        const size_t boff = ((size_t)h * lat + jt * 16 + lr) * nope;
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < nope; k0 += 32) {
            float v[8];
            const float4 v0 = *(const float4*)(arow + k0 + 8 * lg), v1 = *(const float4*)(arow + k0 + 8 * lg + 4);
            v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w; v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
            if (m >= M)
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = 0.f;
            half8_t ah, al;
            split_f16x8(v, ah, al);
            const half8_t bh = *(const half8_t*)(a.upk_hi + boff + k0 + 8 * lg);
            const half8_t bl = *(const half8_t*)(a.upk_lo + boff + k0 + 8 * lg);
            acc = mfma3(ah, al, bh, bl, acc);
        }
        // D lane: rows 4 lg + i, column lr
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int mm = mt * 16 + 4 * lg + i;
            if (mm < M) a.q[((size_t)mm * a.nh + h) * KD + jt * 16 + lr] = acc[i];
        }
    }
    if (blockIdx.z != 0) return;
    const int m0 = mt * 16, nr = min(16, M - m0);
    for (int i = tid; i < nr * half; i += 256) {
        const int k = i / half, e = i - k * half, m = m0 + k;
        const int pos = a.pos0[m / a.S] + m % a.S;
        const float* src = a.raw + (size_t)m * a.raw_ld + h * (nope + rd) + nope;
        const float x1 = src[e], x2 = src[e + half];
        const float cs = a.rope_cos[(size_t)pos * half + e], sn = a.rope_sin[(size_t)pos * half + e];
        float* dst = a.q + ((size_t)m * a.nh + h) * KD + lat;
        {
#pragma clang fp contract(off)
            dst[e] = x1 * cs - x2 * sn;
            dst[e + half] = x1 * sn + x2 * cs;
        }
    }
}

// ---------------------------------------------------------------------------
// kv prep: c_kv = RMSNorm(kv_a) * w and rotated k_rope, appended (fp16) to the
// row-major [cap][lat + rd] cache and the transposed [lat][cap] value copy.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) mla_kvprep_kernel(MlaArgs a) {
    __shared__ float red[4];
    const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lat = a.lat, rd = a.rd, half = rd >> 1, KD = lat + rd;
    const int seq = m / a.S, pos = a.pos0[seq] + m % a.S, sl = a.slot[seq];
    const float* src = a.raw + (size_t)m * a.raw_ld + a.nh * (a.nope + rd);
    float ss = 0.f;
    for (int j = tid; j < lat; j += 256) ss += src[j] * src[j];
    ss = wave_sum_f32(ss);
    if (lane == 0) red[wid] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)lat + a.eps);
    _Float16* krow = a.kc + ((size_t)sl * a.cap + pos) * KD;
    for (int j = tid; j < lat; j += 256) {
        const _Float16 c = (_Float16)(src[j] * inv * a.kvn_w[j]);
        krow[j] = c;
        a.vt[(((size_t)sl * (a.cap >> 5) + (pos >> 5)) * lat + j) * 32 + (pos & 31)] = c;
    }
    if (tid < half) {
        const float x1 = src[lat + tid], x2 = src[lat + tid + half];
        const float c = a.rope_cos[(size_t)pos * half + tid], s = a.rope_sin[(size_t)pos * half + tid];
        float r1, r2;
        {
#pragma clang fp contract(off)
            r1 = x1 * c - x2 * s;
            r2 = x1 * s + x2 * c;
        }
        krow[lat + tid] = (_Float16)r1;
        krow[lat + tid + half] = (_Float16)r2;
    }
}

// reductions over the four 16-lane rows of a wave (lanes lr, lr+16, lr+32, lr+48)
__device__ __forceinline__ float lat_rows_max(float x) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float lat_rows_sum(float x) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Workgroup-wide barrier ordering only LDS traffic: global loads in flight stay
// in flight (a plain __syncthreads() would also wait for them).
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---------------------------------------------------------------------------
// Latent attention.  Workgroup = (sequence, group of up to three 16-row query
// tiles, token chunk) with NP waves per tile; the tile groups of one
// (sequence, chunk) are dispatched to the same XCD back to back, so a cache
// block comes from HBM once and from that XCD's L2 for the other groups.
// Query row r of a sequence is (token s = r / nh, head h = r % nh).  Each
// 32-token block of keys [c_kv | k_rope] and transposed latents is staged in
// LDS once for all waves (the next block's loads in flight in registers while
// the current one is computed).  Wave p of a tile: partial S^T = K Q^T over
// its k-steps (A = key rows from LDS, B = Q^T as fp16 hi + lo in registers);
// the NP partials are exchanged through LDS and added in wave order
// (identically in every wave); online softmax in base 2 with the causal
// limit; O^T += V^T P^T over the wave's share of the latent dims (A =
// transposed latent rows from LDS, B = P^T hi + lo).  The chunk's (m, l, O)
// rows go to scratch; mla_merge combines the chunks in order.
// ---------------------------------------------------------------------------
template <int NKK, int NDT>
struct MlaLds {
    static constexpr int KD = 32 * NKK, LAT = 16 * NDT;
    static constexpr int KROW = KD + 8;           // halves per staged key row (16-byte pad)
    static constexpr int VROW = 40;               // halves per staged latent row: 32 tokens + pad
    static constexpr int K_BYTES = 32 * KROW * 2;
    static constexpr int V_BYTES = LAT * VROW * 2;
    static constexpr int KCH = 32 * KD / 8;       // 16-byte chunks of a key block
    static constexpr int VCH = LAT * 4;           // 16-byte chunks of a latent block
};

template <int NKK, int NDT, int NP, int TW, int DEPTH>
__global__ void __launch_bounds__(64 * NP * TW) mla_attn_kernel(MlaArgs a) {
    typedef MlaLds<NKK, NDT> Lc;
    constexpr int KD = Lc::KD, LAT = Lc::LAT, KH = (NKK + NP - 1) / NP, DH = NDT / NP;
    constexpr int NT = 64 * NP * TW, NST = (Lc::KCH + Lc::VCH + NT - 1) / NT;
    static_assert(NDT % NP == 0, "latent tiles split evenly over the waves of a tile");
    extern __shared__ __attribute__((aligned(16))) char lds[];
    _Float16* ks = (_Float16*)lds;                                   // [32][KROW]
    _Float16* vs = (_Float16*)(lds + Lc::K_BYTES);                   // [LAT][VROW]
    float4_t* sx = (float4_t*)(lds + Lc::K_BYTES + Lc::V_BYTES);     // [2 parity][TW][NP][2][64]
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wt = wv / NP, p = wv % NP;
    const int ntg = (a.ntiles + TW - 1) / TW;
    // block b -> XCD b % 8; the ntg tile groups of work group gidx share an XCD
    const int xcd = blockIdx.x & 7, bi = blockIdx.x >> 3;
    const int gidx = xcd + 8 * (bi / ntg), tg = bi % ntg;
    if (gidx >= a.nseq * a.nchunks) return;
    const int seq = gidx / a.nchunks, chunk = gidx % a.nchunks;
    const int tile = tg * TW + wt;
    const bool tile_ok = tile < a.ntiles;
    const int R_total = a.S * a.nh;
    const int pos0 = a.pos0[seq], kv_len = pos0 + a.S, sl = a.slot[seq];
    const int t_begin = chunk * a.chunk, t_end = min(kv_len, t_begin + a.chunk);
    const int rr = tile * 16 + lr;
    const bool row_ok = tile_ok && rr < R_total;
    const int s_tok = row_ok ? rr / a.nh : 0, hh = row_ok ? rr % a.nh : 0;
    const int lim = row_ok ? pos0 + s_tok : -1;
    const int q0 = p * KH, q1 = min(NKK, q0 + KH);  // this wave's k-steps
    half8_t qh[KH], ql[KH];
    {
        const float* qv = a.q + ((size_t)(seq * a.S + s_tok) * a.nh + hh) * KD;
#pragma unroll
        for (int i = 0; i < KH; i++) {
            const int q = q0 + i;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float v = (row_ok && q < q1) ? qv[32 * q + 8 * lg + j] : 0.f;
                const _Float16 h = (_Float16)v;
                qh[i][j] = h;
                ql[i][j] = (_Float16)(v - (float)h);
            }
        }
    }
    float m = -INFINITY, l = 0.f;
    float4_t o[DH];
#pragma unroll
    for (int dt = 0; dt < DH; dt++) o[dt] = (float4_t){0.f, 0.f, 0.f, 0.f};
    const float sc2 = a.scale * LAT_LOG2E;
    const _Float16* kglob = a.kc + (size_t)sl * a.cap * KD;
    const _Float16* vglob = a.vt + (size_t)sl * LAT * a.cap;  // + (tb / 32) * LAT * 32: one contiguous block
    // staging: thread chunk idx < KCH is key row idx / (KD/8), 16-byte piece idx % (KD/8); the
    // rest are latent row (idx - KCH) / 4, token piece (idx - KCH) % 4
    u32x4_t sa[NST], sb[DEPTH == 2 ? NST : 1];
    constexpr int nthr = NT;
    auto fetch = [&](int tb, u32x4_t* stg) __attribute__((always_inline)) {
        if (tb >= t_end) return;
#pragma unroll
        for (int u = 0; u < NST; u++) {
            const int idx = tid + u * nthr;
            if (idx < Lc::KCH) {
                const int tok = idx / (KD / 8), pc = idx % (KD / 8);
                stg[u] = *(const u32x4_t*)(kglob + (size_t)(tb + tok) * KD + 8 * pc);
            } else if (idx < Lc::KCH + Lc::VCH) {
                stg[u] = *(const u32x4_t*)(vglob + (size_t)tb * LAT + 8 * (idx - Lc::KCH));
            }
        }
    };
    auto stage = [&](const u32x4_t* stg) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NST; u++) {
            const int idx = tid + u * nthr;
            if (idx < Lc::KCH) {
                const int tok = idx / (KD / 8), pc = idx % (KD / 8);
                *(u32x4_t*)(ks + tok * Lc::KROW + 8 * pc) = stg[u];
            } else if (idx < Lc::KCH + Lc::VCH) {
                const int d = (idx - Lc::KCH) >> 2, pc = (idx - Lc::KCH) & 3;
                *(u32x4_t*)(vs + d * Lc::VROW + 8 * pc) = stg[u];
            }
        }
    };
    // A row lr of S tile ts is token 8 (lr / 4) + 4 ts + lr % 4 of the block, so the result lane
    // (lr, lg) holds query row lr, tokens tb + 8 lg + (4 ts + i)
    const int trow0 = 8 * (lr >> 2) + (lr & 3);
    int par = 0;
    // one 32-token block: S, exchange, softmax, O (keys and latents of block tb in LDS)
    auto block = [&](int tb) __attribute__((always_inline)) {
            float4_t st[2];
#pragma unroll
            for (int ts = 0; ts < 2; ts++) {
                const _Float16* kp = ks + (trow0 + 4 * ts) * Lc::KROW + 8 * lg;
                float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < KH; i++) {
                    if (q0 + i < q1) {
                        const half8_t ka = *(const half8_t*)(kp + 32 * (q0 + i));
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[i], acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[i], acc, 0, 0, 0);
                    }
                }
                st[ts] = acc;
            }
            float4_t* grp = sx + (size_t)(par * TW + wt) * NP * 128;
            grp[p * 128 + lane] = st[0];
            grp[p * 128 + 64 + lane] = st[1];
            lds_barrier();
            float4_t t0 = grp[lane], t1 = grp[64 + lane];
#pragma unroll
            for (int pp = 1; pp < NP; pp++) {
                t0 += grp[pp * 128 + lane];
                t1 += grp[pp * 128 + 64 + lane];
            }
            float s[8], mx = -INFINITY;
#pragma unroll
            for (int idx = 0; idx < 8; idx++) {
                const int tok = tb + 8 * lg + idx;
                const float tot = idx < 4 ? t0[idx] : t1[idx - 4];
                s[idx] = (tok < t_end && tok <= lim) ? tot * sc2 : -INFINITY;
                mx = fmaxf(mx, s[idx]);
            }
            mx = lat_rows_max(mx);
            const float mnew = fmaxf(m, mx);
            const float alpha = mnew == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mnew);
            float pr[8], ps = 0.f;
#pragma unroll
            for (int idx = 0; idx < 8; idx++) {
                pr[idx] = s[idx] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s[idx] - mnew);
                ps += pr[idx];
            }
            ps = lat_rows_sum(ps);
            l = l * alpha + ps;
            m = mnew;
            half8_t ph, pl;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const _Float16 h = (_Float16)pr[j];
                ph[j] = h;
                pl[j] = (_Float16)(pr[j] - (float)h);
            }
            // ---- O^T += V^T P^T over this wave's latent tiles: A = dims 16 dt + lr, tokens 8 lg .. +8 ----
            const _Float16* vp = vs + (p * DH * 16 + lr) * Lc::VROW + 8 * lg;
#pragma unroll
            for (int dt = 0; dt < DH; dt++) {
                const half8_t va = *(const half8_t*)(vp + 16 * dt * Lc::VROW);
                o[dt] *= alpha;
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[dt], 0, 0, 0);
            }
        par ^= 1;
    };
    if (DEPTH == 2) {
        // two blocks in flight in registers (sa / sb alternate) while one is computed from LDS
        fetch(t_begin, sa);
        stage(sa);
        fetch(t_begin + 32, sb);
        fetch(t_begin + 64, sa);
        for (int tb = t_begin; tb < t_end; tb += 64) {
            lds_barrier();  // block tb staged
            block(tb);
            if (tb + 32 >= t_end) break;
            lds_barrier();  // every wave is done with block tb
            stage(sb);
            fetch(tb + 96, sb);
            lds_barrier();  // block tb + 32 staged
            block(tb + 32);
            if (tb + 64 >= t_end) break;
            lds_barrier();
            stage(sa);
            fetch(tb + 128, sa);
        }
    } else {
        // one block in flight in registers while one is computed from LDS
        fetch(t_begin, sa);
        stage(sa);
        fetch(t_begin + 32, sa);
        for (int tb = t_begin; tb < t_end; tb += 32) {
            lds_barrier();  // block tb staged
            block(tb);
            if (tb + 32 >= t_end) break;
            lds_barrier();  // every wave is done with block tb
            stage(sa);
            fetch(tb + 64, sa);
        }
    }
    if (!tile_ok) return;
    // ---- chunk partial: row lr, dims 16 (p DH + dt) + 4 lg + i ----
    float* rec = a.part + ((((size_t)seq * a.ntiles + tile) * a.nchunks + chunk) * 16 + lr) * (LAT + 4);
#pragma unroll
    for (int dt = 0; dt < DH; dt++) *(float4_t*)(rec + 4 + 16 * (p * DH + dt) + 4 * lg) = o[dt];
    if (p == 0 && lg == 0) {
        rec[0] = m;
        rec[1] = l;
    }
}

// ---------------------------------------------------------------------------
// Merge: one workgroup per (row, head) combines the chunk partials in chunk
// order into the latent output o_lat[m][h][lat]: wave 0 derives the weights
// exp2(m_c - max) / L (one lane per chunk), then every thread sums its latent
// dims over the chunks with independent loads.
// ---------------------------------------------------------------------------
static constexpr int MLA_MAXCH = 64;  // chunks one merge combines

__global__ void __launch_bounds__(256) mla_merge_kernel(MlaArgs a) {
    __shared__ float wsc[MLA_MAXCH];
    const int mrow = blockIdx.x / a.nh, h = blockIdx.x % a.nh, tid = threadIdx.x;
    const int lat = a.lat, REC = lat + 4, nch = a.nchunks;
    const int seq = mrow / a.S, s = mrow % a.S, r = s * a.nh + h;
    const size_t cstride = (size_t)16 * REC;
    const float* rec0 = a.part + (((size_t)seq * a.ntiles + (r >> 4)) * nch * 16 + (r & 15)) * REC;
    if (tid < 64) {
        const float mc = tid < nch ? rec0[tid * cstride] : -INFINITY;
        const float lc = tid < nch ? rec0[tid * cstride + 1] : 0.f;
        const float Mx = wave_max_f32(mc);
        const float w = mc == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc - Mx);
        const float L = wave_sum_f32(w * lc);
        if (tid < MLA_MAXCH) wsc[tid] = L > 0.f ? w / L : 0.f;
    }
    __syncthreads();
    float* dst = a.olat + ((size_t)mrow * a.nh + h) * lat;
    for (int j = tid; j < lat; j += 256) {
        const float* p = rec0 + 4 + j;
        float acc = 0.f;
        int c = 0;
        for (; c + 8 <= nch; c += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = p[(c + u) * cstride];
#pragma unroll
            for (int u = 0; u < 8; u++) acc = fmaf(v[u], wsc[c + u], acc);
        }
        for (; c < nch; c++) acc = fmaf(p[c * cstride], wsc[c], acc);
        dst[j] = acc;
    }
}

// ---------------------------------------------------------------------------
// up_v: o[m][h*vd + i] = sum_j up_v[h][i][j] o_lat[m][h][j] on MFMA.  Workgroup
// = 16 rows x 1 head x 64 output columns, one 16x16 tile per wave: A = o_lat
// rows (f32 split hi + lo), B = up_v hi + lo.  The o_proj input is written as
// fragments (and f32 rows when o_proj reads f32).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) mla_out_kernel(MlaArgs a) {
    const int M = a.nseq * a.S, h = blockIdx.y, mt = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, lr = lane & 15, lg = lane >> 4, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lat = a.lat, vd = a.vd;
    const int it = blockIdx.z * 4 + wid;
    if (it * 16 >= vd) return;
    const int m = mt * 16 + lr;
    const float* arow = a.olat + ((size_t)min(m, M - 1) * a.nh + h) * lat;
    const size_t boff = ((size_t)h * vd + it * 16 + lr) * lat;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < lat; k0 += 32) {
        float v[8];
        const float4 v0 = *(const float4*)(arow + k0 + 8 * lg), v1 = *(const float4*)(arow + k0 + 8 * lg + 4);
        v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w; v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
        if (m >= M)
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 0.f;
        half8_t ah, al;
        split_f16x8(v, ah, al);
        const half8_t bh = *(const half8_t*)(a.upv_hi + boff + k0 + 8 * lg);
        const half8_t bl = *(const half8_t*)(a.upv_lo + boff + k0 + 8 * lg);
        acc = mfma3(ah, al, bh, bl, acc);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int mm = mt * 16 + 4 * lg + i;
        if (mm >= M) continue;
        const int col = h * vd + it * 16 + lr;
        if (a.fo.buf) frag_put(a.fo, mm, col, acc[i]);
        if (a.out) a.out[(size_t)mm * a.nh * vd + col] = acc[i];
    }
}

// ---------------------------------------------------------------------------
// MoE routing (moe.rs:361-406): one wave per row ranks the E <= 64 logits
// (larger first, equal logits keep the lower index), softmax over the top k in
// rank order; then per-expert assignment lists (rows ascending), each row's
// assignment indices (routed experts in index order, then shared experts) and
// the list of 16-assignment chunks the expert projections run over.
// ---------------------------------------------------------------------------
static constexpr int MOE_RT_WAVES = 16;

// (v, i) comes before (w, j) in routing order: larger logit first, then lower index.
__device__ __forceinline__ bool route_before(float v, int i, float w, int j) { return v > w || (v == w && i < j); }

__device__ __forceinline__ unsigned long long wave_or_u64(unsigned long long x) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const unsigned lo = __shfl_xor((unsigned)x, d, 64), hi = __shfl_xor((unsigned)(x >> 32), d, 64);
        x |= ((unsigned long long)hi << 32) | lo;
    }
    return x;
}

__device__ __forceinline__ int lanes_below(unsigned long long bal) {
    return (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bal >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)bal, 0u));
}

// One wave per row: bitonic sort of (logit, expert) over the lanes into routing
// order, softmax over ranks 0..k-1 summed in rank order, the selected-expert
// mask, the dispatch weights and the k-th / (k+1)-th logit gap.
__global__ void __launch_bounds__(256) moe_rank_kernel(MoeArgs a) {
    const int lane = threadIdx.x & 63, m = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int E = a.E, K = a.K;
    if (m >= a.M) return;
    float v = lane < E ? a.logits[(size_t)m * a.lld + lane] : -INFINITY;
    int i = lane;
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const float pv = __shfl_xor(v, j, 64);
            const int pi = __shfl_xor(i, j, 64);
            const bool keep_first = ((lane & j) == 0) == ((lane & k) == 0);
            const bool take = keep_first ? route_before(pv, pi, v, i) : route_before(v, i, pv, pi);
            if (take) {
                v = pv;
                i = pi;
            }
        }
    }
    // lane r now holds the r-th expert in routing order
    const float mx = __shfl(v, 0, 64);
    const float ev = lane < K ? expf_rn(v - mx) : 0.f;
    float ssum = 0.f;
    for (int r = 0; r < K; r++) ssum += __shfl(ev, r, 64);
    if (lane < K) a.wsel[(size_t)m * 64 + i] = ev / ssum;
    const unsigned long long bm = wave_or_u64(lane < K ? (1ull << i) : 0ull);
    const float vk1 = __shfl(v, K - 1, 64), vk = __shfl(v, K < 64 ? K : 63, 64);
    if (lane == 0) {
        a.selm[m] = bm;
        if (a.gap && K < E) a.gap[m] = fminf(a.gap[m], vk1 - vk);
    }
}

// Single workgroup: per-expert counts, offsets and 16-assignment chunk list,
// then the assignment lists from the row masks.
__global__ void __launch_bounds__(1024) moe_route_kernel(MoeArgs a) {
    __shared__ unsigned long long selm[MOE_MAX_ROWS];
    __shared__ int offs[MOE_MAX_EXPERTS + 1];
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int E = a.E, K = a.K, NS = a.NS, M = a.M;
    for (int m = tid; m < M; m += 64 * MOE_RT_WAVES) selm[m] = a.selm[m];
    __syncthreads();
    // ---- rows per expert (shared experts take every row) ----
    __shared__ int cnt_s[2 * 64];
    for (int e = wid; e < 2 * 64; e += MOE_RT_WAVES) {
        int c = 0;
        if (e < E + NS)
            for (int m0 = 0; m0 < M; m0 += 64) {
                const int m = m0 + lane;
                const bool sel = m < M && (e >= E || ((selm[m] >> e) & 1ull));
                c += __popcll(__ballot(sel));
            }
        if (lane == 0) cnt_s[e] = c;
    }
    __syncthreads();
    // ---- offsets and the chunk list: wave 0 scans (lane l holds experts 2l, 2l + 1) ----
    if (wid == 0) {
        const int c0 = cnt_s[2 * lane], c1 = cnt_s[2 * lane + 1];
        const int k0 = (c0 + 15) >> 4, k1 = (c1 + 15) >> 4;
        const int o = wave_excl_scan_i32(c0 + c1), ko = wave_excl_scan_i32(k0 + k1);
        if (2 * lane <= MOE_MAX_EXPERTS) offs[2 * lane] = o;
        if (2 * lane + 1 <= MOE_MAX_EXPERTS) offs[2 * lane + 1] = o + c0;
        const int nc = __shfl(ko + k0 + k1, 63, 64);
        for (int r = 0; r < k0; r++)
            if (ko + r < a.cmax) {
                a.chunk_e[ko + r] = 2 * lane;
                a.chunk_r0[ko + r] = 16 * r;
            }
        for (int r = 0; r < k1; r++)
            if (ko + k0 + r < a.cmax) {
                a.chunk_e[ko + k0 + r] = 2 * lane + 1;
                a.chunk_r0[ko + k0 + r] = 16 * r;
            }
        if (lane == 0) *a.nchunk = min(nc, a.cmax);
        if (2 * lane < E + NS) a.cnt[2 * lane] = c0;
        if (2 * lane + 1 < E + NS) a.cnt[2 * lane + 1] = c1;
    }
    __syncthreads();
    if (tid <= E + NS) a.off[tid] = offs[tid];
    // ---- assignments: expert lists in ascending rows; a row's slots are its routed experts
    //      in index order, then the shared experts ----
    for (int e = wid; e < E + NS; e += MOE_RT_WAVES) {
        int k = offs[e];
        const unsigned long long below = e == 0 ? 0ull : (e >= 64 ? ~0ull : (~0ull >> (64 - e)));
        for (int m0 = 0; m0 < M; m0 += 64) {
            const int m = m0 + lane;
            const unsigned long long sm = m < M ? selm[m] : 0ull;
            const bool sel = m < M && (e >= E || ((sm >> e) & 1ull));
            const unsigned long long bal = __ballot(sel);
            if (sel) {
                const int pos = k + lanes_below(bal);
                a.arow[pos] = m;
                a.aw[pos] = e < E ? a.wsel[(size_t)m * 64 + e] : 1.0f;
                a.rowmap[(size_t)m * (K + NS) + (e < E ? __popcll(sm & below) : K + (e - E))] = pos;
            }
            k += __popcll(bal);
        }
    }
}

// ---------------------------------------------------------------------------
// Grouped expert projection over the routing's chunk list.  Workgroup = (chunk
// of up to 16 assignments of one expert, slice of its weight-tile steps); 8
// waves split the K groups (group g = wave + 8 gi); the chunk's rows are
// gathered once, split into fp16 (bf16) hi + lo MFMA operands held in
// registers, and the slice's tile steps (NTB tiles each) stream through with
// the next step's weights in flight; per step the 8 wave partials meet in LDS
// (double-buffered, one barrier) and the first NTB waves finish the tiles.
// PHASE 1: gate/up tiles (8 + 8 interleaved rows) -> SwiGLU -> h[assignment].
// PHASE 2: down tiles -> y[assignment] (unweighted).
// ---------------------------------------------------------------------------
template <int FMT>
struct MoeCfg {
    static constexpr int NTB = FMT == WF_INT4 ? 4 : (FMT == WF_INT8 ? 2 : 1);  // tiles per step
};

template <int FMT, int PHASE, int NGW>
__global__ void __launch_bounds__(512) moe_ffn_kernel(MoeArgs a) {
    typedef FmtTraits<FMT> T;
    constexpr int NW = 8, NTB = MoeCfg<FMT>::NTB, LW = T::LANE_WORDS;
    __shared__ float4_t part[2][NW][NTB][64];
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int ci = blockIdx.x / a.bpe, slice = blockIdx.x % a.bpe;
    if (ci >= *a.nchunk) return;
    const int e = a.chunk_e[ci], r0 = a.chunk_r0[ci];
    const int nr = min(16, a.cnt[e] - r0);
    const int base_a = a.off[e] + r0;
    const int Kin = PHASE == 1 ? a.H : a.D;
    const int Ne = PHASE == 1 ? 2 * a.D : a.H;
    const int G = Kin >> 7, ntiles = Ne >> 4, nsteps = (ntiles + NTB - 1) / NTB;
    if (slice >= nsteps) return;
    const uint8_t* W = PHASE == 1 ? a.gu : a.dn;
    const uint32_t* SZ = PHASE == 1 ? a.gu_sz : a.dn_sz;
    const float* RS = PHASE == 1 ? a.gu_rs : a.dn_rs;
    const size_t tile0 = (size_t)e * ntiles;

    // ---- weight words of one step (NTB tiles x this wave's groups), three steps in flight.
    //      Every load is unconditional: a step past the end re-reads the last step and a
    //      group past G re-reads group G - 1 (in bounds, results unused), so the compiler
    //      counts the loads in flight instead of waiting for all of them before each step.
    typedef uint32_t WStep[NTB][NGW][LW];
    typedef uint32_t ZStep[NTB][NGW];
    WStep w0, w1, w2;
    ZStep z0, z1, z2;
    auto load_step = [&](int st, WStep& wv, ZStep& zv) __attribute__((always_inline)) {
        const int stc = min(st, nsteps - 1);
#pragma unroll
        for (int j = 0; j < NTB; j++) {
            const int nt = min(stc * NTB + j, ntiles - 1);
#pragma unroll
            for (int gi = 0; gi < NGW; gi++) {
                const int g = min(wid + NW * gi, G - 1);
                const size_t tile = (tile0 + nt) * G + g;
#pragma unroll
                for (int q = 0; q < LW / 4; q++) {
                    const uint4 w4 = *(const uint4*)(W + tile * T::TILE_BYTES + tile_byte(lane, 16 * q));
                    wv[j][gi][4 * q] = w4.x;
                    wv[j][gi][4 * q + 1] = w4.y;
                    wv[j][gi][4 * q + 2] = w4.z;
                    wv[j][gi][4 * q + 3] = w4.w;
                }
                if (FMT == WF_INT4) zv[j][gi] = SZ[tile * 16 + lr];
            }
        }
    };
    // the chunk row's source index first, then the first two steps, then the activation
    // gather: the weights' round trip overlaps the gather
    const bool rv = lr < nr;
    const int ai = base_a + (rv ? lr : 0);
    const float* rowp = PHASE == 1 ? a.xn + (size_t)a.arow[ai] * a.H : a.h + (size_t)ai * a.D;
    const int B = a.bpe;
    load_step(slice, w0, z0);
    load_step(slice + B, w1, z1);

    // ---- activations of the chunk: A row lr = assignment base_a + lr ----
    half8_t ah[NGW][4], al[NGW][4];
    {
#pragma unroll
        for (int gi = 0; gi < NGW; gi++) {
            const int g = wid + NW * gi;
            const bool use = g < G && rv;
            const int gc = min(g, G - 1);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                // unconditional loads (clamped group, row 0 of the chunk for padding rows)
                const float4 v0 = *(const float4*)(rowp + gc * 128 + 32 * lg + 8 * t);
                const float4 v1 = *(const float4*)(rowp + gc * 128 + 32 * lg + 8 * t + 4);
                float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = use ? v[j] : 0.f;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float x = v[frag_elem(FMT, j)];
                    if (FMT == WF_BF16) {
                        const uint16_t hb = f32_to_bf16_rne(x);
                        ah[gi][t][j] = __builtin_bit_cast(_Float16, hb);
                        al[gi][t][j] = __builtin_bit_cast(_Float16, f32_to_bf16_rne(x - bf16_to_f32(hb)));
                    } else {
                        const _Float16 hx = (_Float16)x;
                        ah[gi][t][j] = hx;
                        al[gi][t][j] = (_Float16)(x - (float)hx);
                    }
                }
            }
        }
    }

    int buf = 0;
    auto compute_step = [&](int st, const WStep& wv, const ZStep& zv) {
#pragma unroll
        for (int j = 0; j < NTB; j++) {
            float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int gi = 0; gi < NGW; gi++) {
                const int g = wid + NW * gi;
                if (g >= G) continue;
                if (FMT == WF_INT4) {
                    const uint32_t szw = zv[j][gi];
                    const float sc = (float)__builtin_bit_cast(_Float16, (uint16_t)(szw & 0xFFFFu));
                    half2_t zl2, zh2;
                    int4_zero_operands(__builtin_bit_cast(_Float16, (uint16_t)(szw >> 16)), zl2, zh2);
                    float4_t ga = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const half8_t b = int4_b_operand(wv[j][gi][t], zl2, zh2);
                        ga = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[gi][t], b, ga, 0, 0, 0);
                        ga = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[gi][t], b, ga, 0, 0, 0);
                    }
                    acc += sc * ga;
                } else if (FMT == WF_INT8) {
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const half8_t b = int8_b_operand(wv[j][gi][2 * t], wv[j][gi][2 * t + 1]);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[gi][t], b, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[gi][t], b, acc, 0, 0, 0);
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const u32x4_t w4 = {wv[j][gi][4 * t], wv[j][gi][4 * t + 1], wv[j][gi][4 * t + 2],
                                            wv[j][gi][4 * t + 3]};
                        const bf16x8_t b = __builtin_bit_cast(bf16x8_t, w4);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ah[gi][t]), b, acc,
                                                                      0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, al[gi][t]), b, acc,
                                                                      0, 0, 0);
                    }
                }
            }
            part[buf][wid][j][lane] = acc;
        }
        lds_barrier();
        if (wid < NTB) {
            // wave j finishes tile j of the step: lane holds token rows 4 lg + i, weight row lr
            const int j = wid, nt = st * NTB + j;
            float4_t sum = part[buf][0][j][lane];
#pragma unroll
            for (int w = 1; w < NW; w++) sum += part[buf][w][j][lane];
            if (FMT == WF_INT8) sum *= RS[(tile0 + min(nt, ntiles - 1)) * 16 + lr];
            if (PHASE == 1) {
                // gate rows 0-7, up rows 8-15 of the tile: column nt * 8 + (lr & 7)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float u = __shfl_xor(sum[i], 8, 64);
                    const int r = 4 * lg + i;
                    if (lr < 8 && nt < ntiles && r < nr) {
                        const float g = sum[i];
                        a.h[(size_t)(base_a + r) * a.D + nt * 8 + lr] = g / (1.0f + expf(-g)) * u;
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * lg + i;
                    if (nt < ntiles && r < nr) a.y[(size_t)(base_a + r) * a.H + nt * 16 + lr] = sum[i];
                }
            }
        }
        buf ^= 1;
    };
    for (int st = slice; st < nsteps; st += 3 * B) {
        load_step(st + 2 * B, w2, z2);
        compute_step(st, w0, z0);
        if (st + B >= nsteps) break;
        load_step(st + 3 * B, w0, z0);
        compute_step(st + B, w1, z1);
        if (st + 2 * B >= nsteps) break;
        load_step(st + 4 * B, w1, z1);
        compute_step(st + 2 * B, w2, z2);
    }
}

// ---------------------------------------------------------------------------
// Combine (moe.rs:290-331): x += (sum_e w_e y_e over the routed experts in index
// order) + (sum of the shared experts in order); the new x as fragments and
// 16-column sums of squares for the next RMSNorm.  Thread per column (coalesced).
// ---------------------------------------------------------------------------
static constexpr int MOE_COMB_MAXK = 16;  // top-k + shared experts a combine handles

__global__ void __launch_bounds__(256) moe_combine_kernel(MoeArgs a) {
    const int m = blockIdx.x, c = blockIdx.y * 256 + threadIdx.x, H = a.H, K = a.K, NS = a.NS;
    const int* rmap = a.rowmap + (size_t)m * (K + NS);
    int ai[MOE_COMB_MAXK];
    float wt[MOE_COMB_MAXK];
#pragma unroll
    for (int j = 0; j < MOE_COMB_MAXK; j++) {
        ai[j] = j < K + NS ? rmap[j] : 0;
        wt[j] = j < K ? a.aw[ai[j]] : 0.f;
    }
    if (c >= H) return;
    float yv[MOE_COMB_MAXK];
#pragma unroll
    for (int j = 0; j < MOE_COMB_MAXK; j++) yv[j] = j < K + NS ? a.y[(size_t)ai[j] * H + c] : 0.f;
    // routed experts weighted in index order, then the shared experts summed in order
    float r = 0.f, sh = 0.f;
#pragma unroll
    for (int j = 0; j < MOE_COMB_MAXK; j++) {
        if (j < K) r += yv[j] * wt[j];
        else if (j == K) sh = yv[j];
        else if (j < K + NS) sh = sh + yv[j];
    }
    if (NS > 0) r += sh;
    const float xn = a.x[(size_t)m * H + c] + r;
    a.x[(size_t)m * H + c] = xn;
    if (a.fo.buf) frag_put(a.fo, m, c, xn);
    float ss = xn * xn;
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) ss += __shfl_xor(ss, d, 64);
    if (a.fo.ssq && (c & 15) == 0) a.fo.ssq[(size_t)m * a.fo.ssq_ld + (c >> 4)] = ss;
}

__global__ void split_hilo_kernel(const float* src, _Float16* hi, _Float16* lo, int N, int K, int tblk) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K) return;
    const int n = (int)(i / K), k = (int)(i % K);
    const size_t o = tblk > 0 ? ((size_t)(n / tblk) * K + k) * tblk + n % tblk : i;
    const float v = src[i];
    const _Float16 h = (_Float16)v;
    hi[o] = h;
    lo[o] = (_Float16)(v - (float)h);
}

int launch_split_hilo(const float* src, _Float16* hi, _Float16* lo, int N, int K, int tblk, hipStream_t stream) {
    if (tblk > 0 && N % tblk) return 2;
    const size_t n = (size_t)N * K;
    (void)hipGetLastError();
    hipLaunchKernelGGL(split_hilo_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, src, hi, lo, N, K,
                       tblk);
    return note_error(hipGetLastError()) ? 4 : 0;
}

__global__ void dequant_tiled_kernel(const uint8_t* tiled, const uint32_t* sz, const float* rscale, int fmt, int N,
                                     int K, float* out, int tblk) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K) return;
    const int n = (int)(i / K), k = (int)(i % K), G = K >> 7;
    const int nt = n >> 4, r = n & 15, g = k >> 7, kk = k & 127, j = kk >> 5, c = kk & 31;
    const size_t tile = (size_t)nt * G + g;
    float v;
    if (fmt == WF_INT4) {
        const uint8_t b = tiled[tile * 1024 + 16 * (j * 16 + r) + (c >> 1)];
        const uint32_t w = sz[tile * 16 + r];
        const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
        const float z = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
        v = ((float)((c & 1) ? (b >> 4) : (b & 15)) - z) * s;
    } else if (fmt == WF_INT8) {
        v = (float)(int8_t)tiled[tile * 2048 + tile_byte(j * 16 + r, c)] * rscale[n];
    } else if (fmt == WF_BF16) {
        v = bf16_to_f32(*(const uint16_t*)(tiled + tile * 4096 + tile_byte(j * 16 + r, 2 * c)));
    } else {
        v = ((const float*)tiled)[i];
    }
    const size_t o = tblk > 0 ? ((size_t)(n / tblk) * K + k) * tblk + n % tblk : i;
    out[o] = v;
}

int launch_dequant_tiled(const uint8_t* tiled, const uint32_t* sz, const float* rscale, int fmt, int N, int K,
                         float* out, int tblk, hipStream_t stream) {
    if (K % 128 || N % 16 || (tblk > 0 && N % tblk)) return 2;
    const size_t n = (size_t)N * K;
    (void)hipGetLastError();
    hipLaunchKernelGGL(dequant_tiled_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, tiled, sz,
                       rscale, fmt, N, K, out, tblk);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// Synthetic latent cache (same streams as the oracle): c_kv and k_rope ~ N(0, 1).
__global__ void lat_kv_fill_kernel(_Float16* kc, _Float16* vt, int slot, int lat, int rd, int cap, int len,
                                   unsigned long long seed, int layer) {
    const int t = blockIdx.x;
    if (t >= len) return;
    const int KD = lat + rd;
    for (int i = threadIdx.x; i < KD; i += blockDim.x) {
        float v;
        if (i < lat) {
            v = synth_normal(seed, 0x4C410000u + (uint32_t)(2 * layer), (uint64_t)t * lat + i);
            vt[(((size_t)slot * (cap >> 5) + (t >> 5)) * lat + i) * 32 + (t & 31)] = (_Float16)v;
        } else {
            v = synth_normal(seed, 0x4C410001u + (uint32_t)(2 * layer), (uint64_t)t * rd + (i - lat));
        }
        kc[((size_t)slot * cap + t) * KD + i] = (_Float16)v;
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
bool mla_supported(int lat, int rd, int vd, int nope) {
    const bool c5 = lat == 512 && rd == 64, small = lat == 128 && rd == 32;
    return (c5 || small) && vd > 0 && vd % 16 == 0 && nope > 0 && nope % 32 == 0;
}

// Raise a kernel's dynamic LDS limit to `bytes` once (first launch).
template <class K>
static bool lds_limit(K kernel, size_t bytes, bool& done) {
    if (done) return true;
    if (note_error(hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes)))
        return false;
    done = true;
    return true;
}

int launch_mla_qprep(const MlaArgs& a, hipStream_t stream) {
    const int M = a.nseq * a.S;
    if (a.nope % 32 || a.lat % 16) return 3;
    (void)hipGetLastError();
    hipLaunchKernelGGL(mla_qprep_kernel, dim3((M + 15) / 16, a.nh, (a.lat / 16 + 3) / 4), dim3(256), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

int launch_mla_kvprep(const MlaArgs& a, hipStream_t stream) {
    (void)hipGetLastError();
    hipLaunchKernelGGL(mla_kvprep_kernel, dim3(a.nseq * a.S), dim3(256), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

static constexpr int MLA_NP = 4;     // waves per 16-row query tile
static constexpr int MLA_TWMAX = 3;  // query tiles per workgroup

template <int NKK, int NDT, int TW>
static int launch_attn_tw(const MlaArgs& a, hipStream_t stream) {
    typedef MlaLds<NKK, NDT> Lc;
    static bool attr = false;
    const size_t lds = (size_t)Lc::K_BYTES + Lc::V_BYTES + (size_t)2 * TW * MLA_NP * 128 * 16;
    constexpr int DEPTH = TW == 3 ? 1 : 2;  // blocks in flight (3 tiles: register budget of 12 waves)
    if (!lds_limit(mla_attn_kernel<NKK, NDT, MLA_NP, TW, DEPTH>, lds, attr)) return 4;
    const int ntg = (a.ntiles + TW - 1) / TW;
    const int groups8 = (a.nseq * a.nchunks + 7) / 8 * 8;
    hipLaunchKernelGGL((mla_attn_kernel<NKK, NDT, MLA_NP, TW, DEPTH>), dim3(groups8 * ntg), dim3(64 * MLA_NP * TW), lds,
                       stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

template <int NKK, int NDT>
static int launch_attn_t(const MlaArgs& a, hipStream_t stream) {
    switch (a.tiles_per_wg) {
        case 1: return launch_attn_tw<NKK, NDT, 1>(a, stream);
        case 2: return launch_attn_tw<NKK, NDT, 2>(a, stream);
        case 3: return launch_attn_tw<NKK, NDT, 3>(a, stream);
    }
    return 2;
}

int mla_tiles_per_wg_max() { return MLA_TWMAX; }

int launch_mla_attn(const MlaArgs& a, hipStream_t stream) {
    if (a.chunk % 32 || a.cap % 32 || a.chunk <= 0 || a.nchunks <= 0) return 2;
    if (a.tiles_per_wg < 1 || a.tiles_per_wg > MLA_TWMAX || a.ntiles < 1) return 2;
    (void)hipGetLastError();
    if (a.lat == 512 && a.rd == 64) return launch_attn_t<18, 32>(a, stream);
    if (a.lat == 128 && a.rd == 32) return launch_attn_t<5, 8>(a, stream);
    return 3;
}

int launch_mla_out(const MlaArgs& a, hipStream_t stream) {
    const int M = a.nseq * a.S;
    if (a.lat % 32 || a.vd % 16 || a.nchunks > MLA_MAXCH || !a.olat) return 3;
    (void)hipGetLastError();
    hipLaunchKernelGGL(mla_merge_kernel, dim3(M * a.nh), dim3(256), 0, stream, a);
    if (note_error(hipGetLastError())) return 4;
    hipLaunchKernelGGL(mla_out_kernel, dim3((M + 15) / 16, a.nh, (a.vd / 16 + 3) / 4), dim3(256), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

int launch_moe_route(const MoeArgs& a, hipStream_t stream) {
    if (a.M > MOE_MAX_ROWS || a.E > 64 || a.E + a.NS > MOE_MAX_EXPERTS || a.K > a.E || a.K < 1) return 3;
    (void)hipGetLastError();
    hipLaunchKernelGGL(moe_rank_kernel, dim3((a.M + 3) / 4), dim3(256), 0, stream, a);
    if (note_error(hipGetLastError())) return 4;
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(64 * MOE_RT_WAVES), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

template <int FMT, int PHASE>
static int launch_ffn_phase(const MoeArgs& a, hipStream_t stream) {
    const int G = (PHASE == 1 ? a.H : a.D) >> 7;
    const dim3 grid(a.cmax * a.bpe), block(512);
    switch ((G + 7) / 8) {
        case 1: hipLaunchKernelGGL((moe_ffn_kernel<FMT, PHASE, 1>), grid, block, 0, stream, a); break;
        case 2: hipLaunchKernelGGL((moe_ffn_kernel<FMT, PHASE, 2>), grid, block, 0, stream, a); break;
        default: return 3;
    }
    return note_error(hipGetLastError()) ? 4 : 0;
}

int moe_tiles_per_step(int fmt) {
    return fmt == WF_INT4 ? MoeCfg<WF_INT4>::NTB : (fmt == WF_INT8 ? MoeCfg<WF_INT8>::NTB : MoeCfg<WF_BF16>::NTB);
}

int launch_moe_ffn(const MoeArgs& a, int phase, hipStream_t stream) {
    if (a.H % 128 || a.D % 128 || a.H / 128 > 16 || a.D / 128 > 16 || a.bpe < 1 || a.cmax < 1) return 3;
    (void)hipGetLastError();
    switch (a.fmt) {
        case WF_INT4: return phase == 1 ? launch_ffn_phase<WF_INT4, 1>(a, stream) : launch_ffn_phase<WF_INT4, 2>(a, stream);
        case WF_INT8: return phase == 1 ? launch_ffn_phase<WF_INT8, 1>(a, stream) : launch_ffn_phase<WF_INT8, 2>(a, stream);
        case WF_BF16: return phase == 1 ? launch_ffn_phase<WF_BF16, 1>(a, stream) : launch_ffn_phase<WF_BF16, 2>(a, stream);
    }
    return 3;
}

int launch_moe_combine(const MoeArgs& a, hipStream_t stream) {
    if (a.H % 16 || a.K + a.NS > MOE_COMB_MAXK) return 3;
    (void)hipGetLastError();
    hipLaunchKernelGGL(moe_combine_kernel, dim3(a.M, (a.H + 255) / 256), dim3(256), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

int launch_lat_kv_fill_synthetic(_Float16* kc, _Float16* vt, int slot, int lat, int rd, int cap, int len,
                                 unsigned long long seed, int layer, hipStream_t stream) {
    if (len <= 0) return 0;
    (void)hipGetLastError();
    hipLaunchKernelGGL(lat_kv_fill_kernel, dim3(len), dim3(256), 0, stream, kc, vt, slot, lat, rd, cap, len, seed,
                       layer);
    return note_error(hipGetLastError()) ? 4 : 0;
}

}  // namespace aarh
