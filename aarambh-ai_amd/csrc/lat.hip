// Latent-attention (MLA) + fine-grained MoE decoder kernels for gfx950
//
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

static constexpr int MLA_RB = 32;  // query rows per qprep / out workgroup

// ---------------------------------------------------------------------------
// q prep: rotate q_rope, absorb q_nope through up_k (q_lat = up_k_h^T q_nope_h).
// Workgroup = 32 rows x 1 head; q_nope staged in LDS as [nope][32].
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) mla_qprep_kernel(MlaArgs a) {
    extern __shared__ float4 qn4[];  // [nope][8] float4 = [nope][32 rows]
    float* qn = (float*)qn4;
    const int M = a.nseq * a.S, h = blockIdx.y, m0 = blockIdx.x * MLA_RB, tid = threadIdx.x;
    const int nope = a.nope, rd = a.rd, lat = a.lat, half = rd >> 1, KD = lat + rd;
    const int nr = min(MLA_RB, M - m0);
    for (int i = tid; i < MLA_RB * nope; i += 256) {
        const int k = i / nope, d = i - k * nope;
        qn[d * MLA_RB + k] = k < nr ? a.raw[(size_t)(m0 + k) * a.raw_ld + h * (nope + rd) + d] : 0.f;
    }
    __syncthreads();
    for (int j = tid; j < lat; j += 256) {
        float acc[MLA_RB];
#pragma unroll
        for (int k = 0; k < MLA_RB; k++) acc[k] = 0.f;
        const float* wp = a.upk + (size_t)h * nope * lat + j;
        for (int d = 0; d < nope; d++) {
            const float w = wp[(size_t)d * lat];
#pragma unroll
            for (int k4 = 0; k4 < MLA_RB / 4; k4++) {
                const float4 q = qn4[d * (MLA_RB / 4) + k4];
                acc[4 * k4] = fmaf(w, q.x, acc[4 * k4]);
                acc[4 * k4 + 1] = fmaf(w, q.y, acc[4 * k4 + 1]);
                acc[4 * k4 + 2] = fmaf(w, q.z, acc[4 * k4 + 2]);
                acc[4 * k4 + 3] = fmaf(w, q.w, acc[4 * k4 + 3]);
            }
        }
#pragma unroll
        for (int k = 0; k < MLA_RB; k++)
            if (k < nr) a.q[((size_t)(m0 + k) * a.nh + h) * KD + j] = acc[k];
    }
    for (int i = tid; i < nr * half; i += 256) {
        const int k = i / half, e = i - k * half, m = m0 + k;
        const int pos = a.pos0[m / a.S] + m % a.S;
        const float* src = a.raw + (size_t)m * a.raw_ld + h * (nope + rd) + nope;
        const float x1 = src[e], x2 = src[e + half];
        const float c = a.rope_cos[(size_t)pos * half + e], s = a.rope_sin[(size_t)pos * half + e];
        float* dst = a.q + ((size_t)m * a.nh + h) * KD + lat;
        {
#pragma clang fp contract(off)
            dst[e] = x1 * c - x2 * s;
            dst[e + half] = x1 * s + x2 * c;
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
        a.vt[((size_t)sl * lat + j) * a.cap + pos] = c;
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

// ---------------------------------------------------------------------------
// Latent attention.  Workgroup = (sequence, group of up to two 16-row query
// tiles, token chunk) with two waves per tile; the tile groups of one
// (sequence, chunk) are dispatched to the same XCD back to back, so a cache
// block comes from HBM once and from that XCD's L2 for the other groups.
// Query row r of a sequence is (token s = r / nh, head h = r % nh).  Per
// 32-token block, wave half p: partial S^T = K Q^T over its k-steps (A = key
// rows [c_kv | k_rope] from the cache, B = Q^T as fp16 hi + lo held in
// registers), the two halves exchange partials through LDS and add them
// (identically in both waves), online softmax in base 2 with the causal limit,
// then O^T += V^T P^T over the wave's half of the latent dims (A = transposed
// latent rows, B = P^T hi + lo).  The chunk's (m, l, O) rows go to scratch;
// mla_out merges the chunks in order.
// ---------------------------------------------------------------------------
template <int NKK, int NDT>
__global__ void __launch_bounds__(256) mla_attn_kernel(MlaArgs a) {
    constexpr int KD = 32 * NKK, LAT = 16 * NDT, KH = (NKK + 1) / 2, DH = NDT / 2;
    extern __shared__ float4_t sx[];  // [2 parity][tiles_per_wg][2 halves][2][64 lanes]
    const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wt = wv >> 1, p = wv & 1, TW = a.tiles_per_wg;
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
    const int q0 = p * KH, q1 = p == 0 ? KH : NKK;  // this wave's k-steps
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
    const _Float16* kbase = a.kc + (size_t)sl * a.cap * KD;
    const _Float16* vbase = a.vt + ((size_t)sl * LAT + p * DH * 16) * a.cap;
    int par = 0;
    for (int tb = t_begin; tb < t_end; tb += 32, par ^= 1) {
        // ---- partial S^T: A row lr of tile ts is token tb + 8 (lr / 4) + 4 ts + lr % 4, so the
        //      result lane (lr, lg) holds query row lr, tokens tb + 8 lg + (4 ts + i) ----
        float4_t st[2];
#pragma unroll
        for (int ts = 0; ts < 2; ts++) {
            const int tok = tb + 8 * (lr >> 2) + 4 * ts + (lr & 3);
            const _Float16* kp = kbase + (size_t)tok * KD + 8 * lg;
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
        float4_t* mine = sx + (((size_t)par * TW + wt) * 2 + p) * 128;
        float4_t* other = sx + (((size_t)par * TW + wt) * 2 + (p ^ 1)) * 128;
        mine[lane] = st[0];
        mine[64 + lane] = st[1];
        __syncthreads();
        const float4_t o0 = other[lane], o1 = other[64 + lane];
        float s[8], mx = -INFINITY;
#pragma unroll
        for (int idx = 0; idx < 8; idx++) {
            const int tok = tb + 8 * lg + idx;
            const float tot = idx < 4 ? st[0][idx] + o0[idx] : st[1][idx - 4] + o1[idx - 4];
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
        // ---- O^T += V^T P^T over this wave's latent tiles: A = dims 16 dt + lr, tokens tb + 8 lg .. +8 ----
#pragma unroll
        for (int dt = 0; dt < DH; dt++) {
            const half8_t va = *(const half8_t*)(vbase + (size_t)(16 * dt + lr) * a.cap + tb + 8 * lg);
            o[dt] *= alpha;
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[dt], 0, 0, 0);
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
// Output: merge the chunk partials of 32 rows of one head (chunk order), apply
// up_v, write the fragments of the o_proj input (column h * vd + i).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) mla_out_kernel(MlaArgs a) {
    extern __shared__ float4 ol4[];  // [lat][8] float4 = [lat][32 rows]
    float* ol = (float*)ol4;
    const int M = a.nseq * a.S, h = blockIdx.y, m0 = blockIdx.x * MLA_RB, tid = threadIdx.x;
    const int lat = a.lat, vd = a.vd, REC = lat + 4;
    const int nr = min(MLA_RB, M - m0);
    for (int k = 0; k < MLA_RB; k++) {
        if (k >= nr) {
            for (int j = tid; j < lat; j += 256) ol[j * MLA_RB + k] = 0.f;
            continue;
        }
        const int mrow = m0 + k, seq = mrow / a.S, s = mrow % a.S;
        const int r = s * a.nh + h, tile = r >> 4, rr = r & 15;
        const float* rec0 = a.part + (((size_t)seq * a.ntiles + tile) * a.nchunks * 16 + rr) * REC;
        const size_t cstride = (size_t)16 * REC;
        float Mx = -INFINITY;
        for (int c = 0; c < a.nchunks; c++) Mx = fmaxf(Mx, rec0[c * cstride]);
        float L = 0.f;
        for (int c = 0; c < a.nchunks; c++) {
            const float mc = rec0[c * cstride];
            L += mc == -INFINITY ? 0.f : rec0[c * cstride + 1] * __builtin_amdgcn_exp2f(mc - Mx);
        }
        const float invL = L > 0.f ? 1.0f / L : 0.f;
        for (int j = tid; j < lat; j += 256) {
            float acc = 0.f;
            for (int c = 0; c < a.nchunks; c++) {
                const float mc = rec0[c * cstride];
                if (mc != -INFINITY) acc += rec0[c * cstride + 4 + j] * __builtin_amdgcn_exp2f(mc - Mx);
            }
            ol[j * MLA_RB + k] = acc * invL;
        }
    }
    __syncthreads();
    const float* wp = a.upvT + (size_t)h * lat * vd;
    for (int idx = tid; idx < vd * (MLA_RB / 16); idx += 256) {
        const int i = idx % vd, rg = idx / vd;
        float acc[16];
#pragma unroll
        for (int k = 0; k < 16; k++) acc[k] = 0.f;
        for (int j = 0; j < lat; j++) {
            const float w = wp[(size_t)j * vd + i];
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++) {
                const float4 q = ol4[j * (MLA_RB / 4) + rg * 4 + k4];
                acc[4 * k4] = fmaf(w, q.x, acc[4 * k4]);
                acc[4 * k4 + 1] = fmaf(w, q.y, acc[4 * k4 + 1]);
                acc[4 * k4 + 2] = fmaf(w, q.z, acc[4 * k4 + 2]);
                acc[4 * k4 + 3] = fmaf(w, q.w, acc[4 * k4 + 3]);
            }
        }
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (rg * 16 + k >= nr) continue;
            const int m = m0 + rg * 16 + k;
            if (a.fo.buf) frag_put(a.fo, m, h * vd + i, acc[k]);
            if (a.out) a.out[(size_t)m * a.nh * vd + h * vd + i] = acc[k];
        }
    }
}

// ---------------------------------------------------------------------------
// MoE routing (moe.rs:361-406): one wave per row ranks the E <= 64 logits
// (larger first, equal logits keep the lower index), softmax over the top k in
// rank order; then per-expert assignment lists (rows ascending) and each row's
// assignment indices (routed experts in index order, then shared experts).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) moe_route_kernel(MoeArgs a) {
    extern __shared__ float wsel[];  // [M][64] dispatch weight of (row, expert)
    __shared__ unsigned long long selm[MOE_MAX_ROWS];
    __shared__ float tmp[4][64], rankv[4][64];
    __shared__ int offs[MOE_MAX_EXPERTS + 1];
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int E = a.E, K = a.K, NS = a.NS, M = a.M;
    for (int m = wid; m < M; m += 4) {
        const float v = lane < E ? a.logits[(size_t)m * a.lld + lane] : -INFINITY;
        int rank = 0;
        for (int e2 = 0; e2 < E; e2++) {
            const float v2 = __shfl(v, e2, 64);
            rank += (v2 > v || (v2 == v && e2 < lane)) ? 1 : 0;
        }
        const bool sel = lane < E && rank < K;
        const float mx = wave_max_f32(sel ? v : -INFINITY);
        const float ev = sel ? expf_rn(v - mx) : 0.f;
        if (sel) tmp[wid][rank] = ev;
        if (lane < E) rankv[wid][rank] = v;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // the wave's LDS writes are done
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        float ssum = 0.f;
        for (int r = 0; r < K; r++) ssum += tmp[wid][r];
        wsel[m * 64 + lane] = sel ? ev / ssum : 0.f;
        const unsigned long long bm = __ballot(sel);
        if (lane == 0) {
            selm[m] = bm;
            if (a.gap && K < E) a.gap[m] = fminf(a.gap[m], rankv[wid][K - 1] - rankv[wid][K]);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    __syncthreads();
    if (tid < E + NS) {
        int c = 0;
        if (tid < E) {
            for (int m = 0; m < M; m++) c += (int)((selm[m] >> tid) & 1ull);
        } else {
            c = M;
        }
        a.cnt[tid] = c;
        offs[tid + 1] = c;
    }
    __syncthreads();
    if (tid == 0) {
        offs[0] = 0;
        for (int e = 0; e < E + NS; e++) offs[e + 1] += offs[e];
        for (int e = 0; e <= E + NS; e++) a.off[e] = offs[e];
    }
    __syncthreads();
    if (tid < E) {
        int k = offs[tid];
        const unsigned long long below = tid == 0 ? 0ull : (~0ull >> (64 - tid));
        for (int m = 0; m < M; m++) {
            if (!((selm[m] >> tid) & 1ull)) continue;
            a.arow[k] = m;
            a.aw[k] = wsel[m * 64 + tid];
            a.rowmap[(size_t)m * (K + NS) + __popcll(selm[m] & below)] = k;
            k++;
        }
    } else if (tid < E + NS) {
        const int sidx = tid - E;
        for (int m = 0; m < M; m++) {
            const int k = offs[tid] + m;
            a.arow[k] = m;
            a.aw[k] = 1.0f;
            a.rowmap[(size_t)m * (K + NS) + K + sidx] = k;
        }
    }
}

// ---------------------------------------------------------------------------
// Grouped expert projection: block = (expert, 4 weight tiles), 8 waves split
// the K groups; the expert's assigned rows are taken 16 at a time, gathered
// from f32 rows and split into fp16 (bf16) hi + lo MFMA operands in registers.
// PHASE 1: gate/up tiles (8 + 8 interleaved rows) -> SwiGLU -> h[assignment].
// PHASE 2: down tiles -> y[assignment] (unweighted).
// ---------------------------------------------------------------------------
template <int FMT, int PHASE>
__global__ void __launch_bounds__(512) moe_ffn_kernel(MoeArgs a) {
    typedef FmtTraits<FMT> T;
    constexpr int NW = 8, NTB = 4, NGW = 4, LW = T::LANE_WORDS;
    __shared__ float4_t part[NW][NTB][64];
    __shared__ float yt[NTB][16][17];
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int Kin = PHASE == 1 ? a.H : a.D;
    const int Ne = PHASE == 1 ? 2 * a.D : a.H;
    const int G = Kin >> 7, ntiles = Ne >> 4, TB = (ntiles + NTB - 1) / NTB;
    const int e = blockIdx.x / TB, tg = blockIdx.x % TB;
    const int n_e = a.cnt[e];
    if (n_e == 0) return;
    const int base_a = a.off[e];
    const uint8_t* W = PHASE == 1 ? a.gu : a.dn;
    const uint32_t* SZ = PHASE == 1 ? a.gu_sz : a.dn_sz;
    const float* RS = PHASE == 1 ? a.gu_rs : a.dn_rs;

    for (int c0 = 0; c0 < n_e; c0 += 16) {
        const bool rv = c0 + lr < n_e;
        const int ai = base_a + min(c0 + lr, n_e - 1);
        const float* rowp = PHASE == 1 ? a.xn + (size_t)a.arow[ai] * a.H : a.h + (size_t)ai * a.D;
        half8_t ah[NGW][4], al[NGW][4];
#pragma unroll
        for (int gi = 0; gi < NGW; gi++) {
            const int g = wid + NW * gi;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                float v[8];
                if (g < G && rv) {
                    const float4 v0 = *(const float4*)(rowp + g * 128 + 32 * lg + 8 * t);
                    const float4 v1 = *(const float4*)(rowp + g * 128 + 32 * lg + 8 * t + 4);
                    v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
                    v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
                } else {
#pragma unroll
                    for (int j = 0; j < 8; j++) v[j] = 0.f;
                }
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float x = v[frag_elem(FMT, j)];
                    if (FMT == WF_BF16) {
                        const uint16_t hb = f32_to_bf16_rne(x);
                        ah[gi][t][j] = __builtin_bit_cast(_Float16, hb);
                        al[gi][t][j] = __builtin_bit_cast(_Float16, f32_to_bf16_rne(x - bf16_to_f32(hb)));
                    } else {
                        const _Float16 h = (_Float16)x;
                        ah[gi][t][j] = h;
                        al[gi][t][j] = (_Float16)(x - (float)h);
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NTB; j++) {
            const int nt = min(tg * NTB + j, ntiles - 1);
            float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int gi = 0; gi < NGW; gi++) {
                const int g = wid + NW * gi;
                if (g >= G) continue;
                const size_t tile = ((size_t)e * ntiles + nt) * G + g;
                uint32_t wv[LW];
#pragma unroll
                for (int q = 0; q < LW / 4; q++) {
                    const uint4 w4 = *(const uint4*)(W + tile * T::TILE_BYTES + (size_t)lane * LW * 4 + 16 * q);
                    wv[4 * q] = w4.x; wv[4 * q + 1] = w4.y; wv[4 * q + 2] = w4.z; wv[4 * q + 3] = w4.w;
                }
                if (FMT == WF_INT4) {
                    const uint32_t szw = SZ[tile * 16 + lr];
                    const float sc = (float)__builtin_bit_cast(_Float16, (uint16_t)(szw & 0xFFFFu));
                    half2_t zl2, zh2;
                    int4_zero_operands(__builtin_bit_cast(_Float16, (uint16_t)(szw >> 16)), zl2, zh2);
                    float4_t ga = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const half8_t b = int4_b_operand(wv[t], zl2, zh2);
                        ga = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[gi][t], b, ga, 0, 0, 0);
                        ga = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[gi][t], b, ga, 0, 0, 0);
                    }
                    acc += sc * ga;
                } else if (FMT == WF_INT8) {
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const half8_t b = int8_b_operand(wv[2 * t], wv[2 * t + 1]);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[gi][t], b, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[gi][t], b, acc, 0, 0, 0);
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const u32x4_t w4 = {wv[4 * t], wv[4 * t + 1], wv[4 * t + 2], wv[4 * t + 3]};
                        const bf16x8_t b = __builtin_bit_cast(bf16x8_t, w4);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ah[gi][t]), b, acc,
                                                                      0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, al[gi][t]), b, acc,
                                                                      0, 0, 0);
                    }
                }
            }
            part[wid][j][lane] = acc;
        }
        __syncthreads();
        if (tid < NTB * 64) {
            const int j = tid >> 6, ln = tid & 63;
            float4_t sum = part[0][j][ln];
#pragma unroll
            for (int w = 1; w < NW; w++) sum += part[w][j][ln];
            const int nt = min(tg * NTB + j, ntiles - 1);
            const float rs = FMT == WF_INT8 ? RS[((size_t)e * ntiles + nt) * 16 + (ln & 15)] : 1.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) yt[j][4 * (ln >> 4) + i][ln & 15] = sum[i] * rs;
        }
        __syncthreads();
        if (PHASE == 1) {
            for (int idx = tid; idx < NTB * 16 * 8; idx += NW * 64) {
                const int j = idx >> 7, r16 = (idx >> 3) & 15, q = idx & 7;
                const int nt = tg * NTB + j;
                if (nt < ntiles && c0 + r16 < n_e) {
                    const float g = yt[j][r16][q], u = yt[j][r16][8 + q];
                    const float silu = g / (1.0f + expf(-g));
                    a.h[(size_t)(base_a + c0 + r16) * a.D + nt * 8 + q] = silu * u;
                }
            }
        } else {
            for (int idx = tid; idx < NTB * 16 * 16; idx += NW * 64) {
                const int j = idx >> 8, r16 = (idx >> 4) & 15, n = idx & 15;
                const int nt = tg * NTB + j;
                if (nt < ntiles && c0 + r16 < n_e) a.y[(size_t)(base_a + c0 + r16) * a.H + nt * 16 + n] = yt[j][r16][n];
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Combine (moe.rs:290-331): x += (sum_e w_e y_e over the routed experts in index
// order) + (sum of the shared experts in order); the new x as fragments and
// 16-column sums of squares for the next RMSNorm.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(128) moe_combine_kernel(MoeArgs a) {
    const int m = blockIdx.x, H = a.H, KS = a.K + a.NS;
    const int* rmap = a.rowmap + (size_t)m * KS;
    for (int t = threadIdx.x; t < H / 16; t += blockDim.x) {
        float ss = 0.f;
        for (int n = 0; n < 16; n++) {
            const int c = t * 16 + n;
            float r = 0.f;
            for (int j = 0; j < a.K; j++) {
                const int ai = rmap[j];
                r += a.y[(size_t)ai * H + c] * a.aw[ai];
            }
            if (a.NS > 0) {
                float sh = a.y[(size_t)rmap[a.K] * H + c];
                for (int s = 1; s < a.NS; s++) sh = sh + a.y[(size_t)rmap[a.K + s] * H + c];
                r += sh;
            }
            const float xn = a.x[(size_t)m * H + c] + r;
            a.x[(size_t)m * H + c] = xn;
            if (a.fo.buf) frag_put(a.fo, m, c, xn);
            ss += xn * xn;
        }
        if (a.fo.ssq) a.fo.ssq[(size_t)m * a.fo.ssq_ld + t] = ss;
    }
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
        v = (float)(int8_t)tiled[tile * 2048 + 32 * (j * 16 + r) + c] * rscale[n];
    } else if (fmt == WF_BF16) {
        v = bf16_to_f32(((const uint16_t*)tiled)[tile * 2048 + 32 * (j * 16 + r) + c]);
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
            vt[((size_t)slot * lat + i) * cap + t] = (_Float16)v;
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
    return (c5 || small) && vd > 0 && nope > 0 && nope <= 1024;
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
    static bool attr = false;
    const int M = a.nseq * a.S;
    const size_t lds = (size_t)MLA_RB * a.nope * 4;
    if (a.nope > 1024) return 3;
    if (!lds_limit(mla_qprep_kernel, (size_t)MLA_RB * 1024 * 4, attr)) return 4;
    (void)hipGetLastError();
    hipLaunchKernelGGL(mla_qprep_kernel, dim3((M + MLA_RB - 1) / MLA_RB, a.nh), dim3(256), lds, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

int launch_mla_kvprep(const MlaArgs& a, hipStream_t stream) {
    (void)hipGetLastError();
    hipLaunchKernelGGL(mla_kvprep_kernel, dim3(a.nseq * a.S), dim3(256), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

template <int NKK, int NDT>
static int launch_attn_t(const MlaArgs& a, hipStream_t stream) {
    static bool attr = false;
    if (!lds_limit(mla_attn_kernel<NKK, NDT>, (size_t)2 * 2 * 2 * 128 * 16, attr)) return 4;
    const int ntg = (a.ntiles + a.tiles_per_wg - 1) / a.tiles_per_wg;
    const int groups8 = (a.nseq * a.nchunks + 7) / 8 * 8;
    const size_t lds = (size_t)2 * a.tiles_per_wg * 2 * 128 * 16;
    hipLaunchKernelGGL((mla_attn_kernel<NKK, NDT>), dim3(groups8 * ntg), dim3(128 * a.tiles_per_wg), lds, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

int launch_mla_attn(const MlaArgs& a, hipStream_t stream) {
    if (a.chunk % 32 || a.cap % 32 || a.chunk <= 0 || a.nchunks <= 0) return 2;
    if (a.tiles_per_wg < 1 || a.tiles_per_wg > 2 || a.ntiles < 1) return 2;
    (void)hipGetLastError();
    if (a.lat == 512 && a.rd == 64) return launch_attn_t<18, 32>(a, stream);
    if (a.lat == 128 && a.rd == 32) return launch_attn_t<5, 8>(a, stream);
    return 3;
}

int launch_mla_out(const MlaArgs& a, hipStream_t stream) {
    static bool attr = false;
    const int M = a.nseq * a.S;
    const size_t lds = (size_t)MLA_RB * a.lat * 4;
    if (a.lat > 512) return 3;
    if (!lds_limit(mla_out_kernel, (size_t)MLA_RB * 512 * 4, attr)) return 4;
    (void)hipGetLastError();
    hipLaunchKernelGGL(mla_out_kernel, dim3((M + MLA_RB - 1) / MLA_RB, a.nh), dim3(256), lds, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

int launch_moe_route(const MoeArgs& a, hipStream_t stream) {
    if (a.M > MOE_MAX_ROWS || a.E > 64 || a.E + a.NS > MOE_MAX_EXPERTS || a.K > a.E || a.K < 1) return 3;
    static bool attr = false;
    if (!lds_limit(moe_route_kernel, (size_t)MOE_MAX_ROWS * 64 * 4, attr)) return 4;
    (void)hipGetLastError();
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(256), (size_t)a.M * 64 * 4, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

template <int FMT>
static int launch_ffn_fmt(const MoeArgs& a, int phase, hipStream_t stream) {
    const int Ne = phase == 1 ? 2 * a.D : a.H;
    const int TB = (Ne / 16 + 3) / 4;
    const dim3 grid((a.E + a.NS) * TB);
    if (phase == 1) hipLaunchKernelGGL((moe_ffn_kernel<FMT, 1>), grid, dim3(512), 0, stream, a);
    else hipLaunchKernelGGL((moe_ffn_kernel<FMT, 2>), grid, dim3(512), 0, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

int launch_moe_ffn(const MoeArgs& a, int phase, hipStream_t stream) {
    if (a.H % 128 || a.D % 128 || a.H / 128 > 32 || a.D / 128 > 32) return 3;
    (void)hipGetLastError();
    switch (a.fmt) {
        case WF_INT4: return launch_ffn_fmt<WF_INT4>(a, phase, stream);
        case WF_INT8: return launch_ffn_fmt<WF_INT8>(a, phase, stream);
        case WF_BF16: return launch_ffn_fmt<WF_BF16>(a, phase, stream);
    }
    return 3;
}

int launch_moe_combine(const MoeArgs& a, hipStream_t stream) {
    if (a.H % 16) return 3;
    (void)hipGetLastError();
    hipLaunchKernelGGL(moe_combine_kernel, dim3(a.M), dim3(128), 0, stream, a);
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
