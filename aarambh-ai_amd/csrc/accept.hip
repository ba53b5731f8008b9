// Fused acceptance sampling for speculative verification on gfx950.
//
// Restates, per sequence, the host-side acceptance round of the reference:
//   probabilities     inference/src/sampler.rs:102-118, 226-312
//   accept_proposal   inference/src/speculative.rs:755-768
//   residual          inference/src/speculative.rs:770-793
//   sample            inference/src/sampler.rs:142-152, 314-347
// and the round structure of speculative.rs:343-501 (external draft, bonus
// sample) and mtp_speculative.rs:228-315 (MTP, no bonus).
//
// One workgroup per logits row computes the row's softmax max and the EXACT
// sequential f32 normaliser (seq_sum_wave), then the last workgroup of each
// sequence to finish resolves the proposals in order, draws ChaCha12 uniforms
// at the sequence's keystream offset, and on rejection builds the residual
// max(0, p - q) in LDS, normalises it with the exact sequential sum and walks
// the exact sequential CDF.  Logits are read once from HBM per row (the
// rejected position's two rows are read a second time).
#include <float.h>

#include "device_common.hpp"
#include "kernels.hpp"

namespace aarh {

static constexpr int ACC_THREADS = 512;
static constexpr int ACC_U = 8;  // logit loads a thread issues before consuming them

struct RowView {
    const float* p;
    float mx;
    float S;
};

// Probability of element j under row r: fl(expf(fl(l/T) - max) / S).
__device__ __forceinline__ float row_prob(const float* lg, int j, float invT_unused, float T, float mx, float S) {
    float m = lg[j] / T;
    if (!isfinite(m)) return 0.0f;
    return expf_rn(m - mx) / S;
}

__global__ void __launch_bounds__(ACC_THREADS) accept_kernel(AcceptArgs a) {
    extern __shared__ float lds[];
    __shared__ float red_f[ACC_THREADS / WAVE];
    __shared__ int red_k[ACC_THREADS / WAVE];
    __shared__ int red_i[ACC_THREADS / WAVE];
    __shared__ unsigned is_last;
    __shared__ float sh_bcast[4];
    __shared__ int sh_ibcast[8];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rows_per_seq = a.target_rows + a.K;
    const int b = blockIdx.x / rows_per_seq;
    const int r = blockIdx.x % rows_per_seq;
    const int V = a.V;
    int np = a.n_proposals ? a.n_proposals[b] : a.K;
    np = np < 0 ? 0 : (np > a.K ? a.K : np);

    // ---------------- stage 1: per-row statistics ----------------
    const bool is_target = r < a.target_rows;
    const int ridx = is_target ? r : r - a.target_rows;
    const bool needed = is_target ? (ridx < np || (a.bonus && ridx == np)) : (ridx < np);
    const size_t row_id = (size_t)b * rows_per_seq + r;
    const float* row = is_target ? a.target + ((size_t)b * a.target_rows + ridx) * V
                                 : a.draft + ((size_t)b * a.K + ridx) * V;
    if (needed) {
        if (a.greedy) {
            int bk = INT_MIN, bi = 0;
            // ACC_U loads in flight per thread, consumed in index order
            for (int j0 = tid; j0 < V; j0 += ACC_U * ACC_THREADS) {
                float vv[ACC_U];
#pragma unroll
                for (int u = 0; u < ACC_U; u++) {
                    const int j = j0 + u * ACC_THREADS;
                    vv[u] = j < V ? row[j] : 0.f;
                }
#pragma unroll
                for (int u = 0; u < ACC_U; u++) {
                    const int j = j0 + u * ACC_THREADS;
                    if (j < V) {
                        const int k = total_key(vv[u]);
                        if (k >= bk) { bk = k; bi = j; }
                    }
                }
            }
            for (int d = 32; d >= 1; d >>= 1) {
                int ok = __shfl_xor(bk, d, 64), oi = __shfl_xor(bi, d, 64);
                if (ok > bk || (ok == bk && oi > bi)) { bk = ok; bi = oi; }
            }
            if (lane == 0) { red_k[wid] = bk; red_i[wid] = bi; }
            __syncthreads();
            if (tid == 0) {
                int k0 = red_k[0], i0 = red_i[0];
                for (int w = 1; w < ACC_THREADS / WAVE; w++)
                    if (red_k[w] > k0 || (red_k[w] == k0 && red_i[w] > i0)) { k0 = red_k[w]; i0 = red_i[w]; }
                st_coh_i32(&a.row_argmax[row_id], i0);
            }
        } else {
            const float T = a.temperature;
            float mx = -INFINITY;
            for (int j0 = tid; j0 < V; j0 += ACC_U * ACC_THREADS) {
                float vv[ACC_U];
#pragma unroll
                for (int u = 0; u < ACC_U; u++) {
                    const int j = j0 + u * ACC_THREADS;
                    vv[u] = j < V ? row[j] : 0.f;
                }
#pragma unroll
                for (int u = 0; u < ACC_U; u++) {
                    const int j = j0 + u * ACC_THREADS;
                    if (j < V) {
                        const float m = vv[u] / T;
                        if (isfinite(m)) mx = fmaxf(mx, m);
                    }
                }
            }
            mx = wave_max_f32(mx);
            if (lane == 0) red_f[wid] = mx;
            __syncthreads();
            if (tid == 0) {
                float m0 = red_f[0];
                for (int w = 1; w < ACC_THREADS / WAVE; w++) m0 = fmaxf(m0, red_f[w]);
                sh_bcast[0] = m0;
            }
            __syncthreads();
            mx = sh_bcast[0];
            for (int j0 = tid; j0 < V; j0 += ACC_U * ACC_THREADS) {
                float vv[ACC_U];
#pragma unroll
                for (int u = 0; u < ACC_U; u++) {
                    const int j = j0 + u * ACC_THREADS;
                    vv[u] = j < V ? row[j] : 0.f;
                }
#pragma unroll
                for (int u = 0; u < ACC_U; u++) {
                    const int j = j0 + u * ACC_THREADS;
                    if (j < V) {
                        const float m = vv[u] / T;
                        lds[j] = isfinite(m) ? expf_rn(m - mx) : 0.0f;
                    }
                }
            }
            __syncthreads();
            if (wid == 0) {
                SeqSum ss = seq_sum_wave(lds, V, -1.0f);
                if (lane == 0) {
                    st_coh(&a.row_max[row_id], mx);
                    st_coh(&a.row_sum[row_id], ss.total);
                }
            }
        }
    }

    // ---------------- last workgroup of the sequence resolves ----------------
    if (!arrive_last(&a.counters[b], (unsigned)rows_per_seq, &is_last)) return;

    const size_t seq_row0 = (size_t)b * rows_per_seq;
    const float* trow0 = a.target + (size_t)b * a.target_rows * V;
    const float* drow0 = a.draft + (size_t)b * a.K * V;

    if (tid == 0) {
        uint32_t key[8];
        rng_key_from_seed(a.seeds ? a.seeds[b] : 0ull, key);
        uint64_t word = a.word_offsets ? a.word_offsets[b] : 0ull;
        int draws = 0, acc = 0, rej = -1;
        uint32_t flags = 0;
        for (int i = 0; i < np; i++) {
            if (a.greedy) {
                if (ld_coh_i32(&a.row_argmax[seq_row0 + a.target_rows + i]) == ld_coh_i32(&a.row_argmax[seq_row0 + i])) {
                    acc++;
                    continue;
                }
                rej = i;
                break;
            }
            const uint32_t x = a.draft_tokens[(size_t)b * a.K + i];
            const float* tl = trow0 + (size_t)i * V;
            const float* dl = drow0 + (size_t)i * V;
            float p = 0.0f, q = 0.0f;
            if ((int)x < V) {
                p = row_prob(tl, (int)x, 0.f, a.temperature, ld_coh(&a.row_max[seq_row0 + i]),
                             ld_coh(&a.row_sum[seq_row0 + i]));
                q = row_prob(dl, (int)x, 0.f, a.temperature, ld_coh(&a.row_max[seq_row0 + a.target_rows + i]),
                             ld_coh(&a.row_sum[seq_row0 + a.target_rows + i]));
            }
            if (!(q > 0.0f)) {
                rej = i;
                break;
            }
            float u = a.uniforms ? a.uniforms[(size_t)b * (a.K + 1) + draws] : rng_f32(key, word + draws);
            draws++;
            float ratio = p / q;
            float cl = ratio < 1.0f ? ratio : 1.0f;
            if (isnan(ratio)) cl = 1.0f;
            if (fabsf(cl - u) < 1e-5f) flags |= ACCEPT_FLAG_RATIO_NEAR;
            if (u < cl) {
                acc++;
                continue;
            }
            rej = i;
            break;
        }
        sh_ibcast[0] = acc;
        sh_ibcast[1] = rej;
        sh_ibcast[2] = draws;
        sh_ibcast[3] = (int)flags;
    }
    __syncthreads();
    const int acc = sh_ibcast[0], rej = sh_ibcast[1];
    int draws = sh_ibcast[2];
    uint32_t flags = (uint32_t)sh_ibcast[3];
    int token = -1, status = 0;

    if (a.greedy) {
        if (rej >= 0) token = ld_coh_i32(&a.row_argmax[seq_row0 + rej]);
        else if (a.bonus) token = ld_coh_i32(&a.row_argmax[seq_row0 + np]);
    } else if (rej >= 0 || a.bonus) {
        const float T = a.temperature;
        if (rej >= 0) {
            const float* tl = trow0 + (size_t)rej * V;
            const float* dl = drow0 + (size_t)rej * V;
            const float pmx = ld_coh(&a.row_max[seq_row0 + rej]), pS = ld_coh(&a.row_sum[seq_row0 + rej]);
            const float qmx = ld_coh(&a.row_max[seq_row0 + a.target_rows + rej]);
            const float qS = ld_coh(&a.row_sum[seq_row0 + a.target_rows + rej]);
            for (int j = tid; j < V; j += ACC_THREADS) {
                float d = row_prob(tl, j, 0.f, T, pmx, pS) - row_prob(dl, j, 0.f, T, qmx, qS);
                lds[j] = d > 0.0f ? d : 0.0f;
            }
            __syncthreads();
            if (wid == 0) {
                SeqSum ss = seq_sum_wave(lds, V, -1.0f);
                if (lane == 0) sh_bcast[1] = ss.total;
            }
            __syncthreads();
            const float R = sh_bcast[1];
            if (!isfinite(R) || R <= FLT_EPSILON) {
                status = 1;
            } else {
                for (int j = tid; j < V; j += ACC_THREADS) lds[j] = lds[j] / R;
            }
        } else {
            const float* tl = trow0 + (size_t)np * V;
            const float pmx = ld_coh(&a.row_max[seq_row0 + np]), pS = ld_coh(&a.row_sum[seq_row0 + np]);
            for (int j = tid; j < V; j += ACC_THREADS) lds[j] = row_prob(tl, j, 0.f, T, pmx, pS);
        }
        __syncthreads();
        if (status == 0 && wid == 0) {
            uint32_t key[8];
            float u;
            if (a.uniforms) {
                u = a.uniforms[(size_t)b * (a.K + 1) + draws];
            } else {
                rng_key_from_seed(a.seeds ? a.seeds[b] : 0ull, key);
                u = rng_f32(key, (a.word_offsets ? a.word_offsets[b] : 0ull) + draws);
            }
            SeqSum ss = seq_sum_wave(lds, V, u);
            if (lane == 0) {
                sh_ibcast[4] = ss.cross;
                sh_bcast[2] = fminf(fabsf(ss.s_at - u), fabsf(u - ss.s_before));
                sh_ibcast[5] = (!isfinite(ss.total) || fabsf(ss.total - 1.0f) > 1e-4f) ? 1 : 0;
            }
        }
        __syncthreads();
        if (status == 0) {
            token = sh_ibcast[4];
            status = sh_ibcast[5];
            if (sh_bcast[2] < 1e-6f) flags |= ACCEPT_FLAG_CDF_NEAR;
            draws++;
        }
    }
    if (tid == 0) {
        a.out_accept_len[b] = acc;
        a.out_token[b] = token;
        a.out_flags[b] = flags;
        a.out_draws[b] = draws;
        a.out_status[b] = status;
    }
}

int launch_accept(const AcceptArgs& a, hipStream_t stream) {
    const int rows = a.target_rows + a.K;
    const size_t lds = a.greedy ? 0 : (size_t)a.V * sizeof(float);
    if (lds > 160 * 1024) return 3;
    if (lds > MAX_DYN_LDS) return 3;
    static bool attr_set = false;
    if (!attr_set) {
        if (note_error(hipFuncSetAttribute((const void*)accept_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           MAX_DYN_LDS)))
            return 4;
        attr_set = true;
    }
    (void)hipGetLastError();
    hipLaunchKernelGGL(accept_kernel, dim3(a.B * rows), dim3(ACC_THREADS), lds, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// ---------------------------------------------------------------------------
// Sampler::top_candidates_from_probabilities (sampler.rs:188-208) of each row's
// distribution as the engines build it (Sampler::probabilities, sampler.rs:
// 102-118): a stable descending sort truncated to n, i.e. the n largest
// probabilities, equal probabilities in ascending token order.  Keys
// (probability bits << 32 | ~token) order both at once; each thread keeps its
// n best, wave 0 merges the 512 sorted lists.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(ACC_THREADS) candidates_kernel(CandArgs a) {
    extern __shared__ float lds[];
    __shared__ unsigned long long keys[ACC_THREADS][CAND_MAX];
    __shared__ float red_f[ACC_THREADS / WAVE];
    __shared__ int red_k[ACC_THREADS / WAVE], red_i[ACC_THREADS / WAVE];
    __shared__ float sh[2];
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int V = a.V, n = a.n;
    const float* row = a.logits + (size_t)blockIdx.x * a.ld;
    int am = -1;
    float S = 1.0f;
    if (a.greedy) {
        // argmax, last index on ties (sampler.rs:211-215 / argmax)
        int bk = INT_MIN, bi = 0;
        for (int j0 = tid; j0 < V; j0 += ACC_U * ACC_THREADS) {
            float vv[ACC_U];
#pragma unroll
            for (int u = 0; u < ACC_U; u++) {
                const int j = j0 + u * ACC_THREADS;
                vv[u] = j < V ? row[j] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < ACC_U; u++) {
                const int j = j0 + u * ACC_THREADS;
                if (j < V) {
                    const int k = total_key(vv[u]);
                    if (k >= bk) { bk = k; bi = j; }
                }
            }
        }
        for (int d = 32; d >= 1; d >>= 1) {
            const int ok = __shfl_xor(bk, d, 64), oi = __shfl_xor(bi, d, 64);
            if (ok > bk || (ok == bk && oi > bi)) { bk = ok; bi = oi; }
        }
        if (lane == 0) { red_k[wid] = bk; red_i[wid] = bi; }
        __syncthreads();
        if (tid == 0) {
            int k0 = red_k[0], i0 = red_i[0];
            for (int w = 1; w < ACC_THREADS / WAVE; w++)
                if (red_k[w] > k0 || (red_k[w] == k0 && red_i[w] > i0)) { k0 = red_k[w]; i0 = red_i[w]; }
            red_i[0] = i0;
        }
        __syncthreads();
        am = red_i[0];
    } else {
        const float T = a.temperature;
        float mx = -INFINITY;
        for (int j0 = tid; j0 < V; j0 += ACC_U * ACC_THREADS) {
            float vv[ACC_U];
#pragma unroll
            for (int u = 0; u < ACC_U; u++) {
                const int j = j0 + u * ACC_THREADS;
                vv[u] = j < V ? row[j] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < ACC_U; u++) {
                const int j = j0 + u * ACC_THREADS;
                if (j < V) {
                    const float m = vv[u] / T;
                    if (isfinite(m)) mx = fmaxf(mx, m);
                }
            }
        }
        mx = wave_max_f32(mx);
        if (lane == 0) red_f[wid] = mx;
        __syncthreads();
        if (tid == 0) {
            float m0 = red_f[0];
            for (int w = 1; w < ACC_THREADS / WAVE; w++) m0 = fmaxf(m0, red_f[w]);
            sh[0] = m0;
        }
        __syncthreads();
        mx = sh[0];
        for (int j0 = tid; j0 < V; j0 += ACC_U * ACC_THREADS) {
            float vv[ACC_U];
#pragma unroll
            for (int u = 0; u < ACC_U; u++) {
                const int j = j0 + u * ACC_THREADS;
                vv[u] = j < V ? row[j] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < ACC_U; u++) {
                const int j = j0 + u * ACC_THREADS;
                if (j < V) {
                    const float m = vv[u] / T;
                    lds[j] = isfinite(m) ? expf_rn(m - mx) : 0.0f;
                }
            }
        }
        __syncthreads();
        if (wid == 0) {
            const SeqSum ss = seq_sum_wave(lds, V, -1.0f);
            if (lane == 0) sh[1] = ss.total;
        }
        __syncthreads();
        S = sh[1];
    }
    // ---- this thread's n best keys, descending ----
    unsigned long long best[CAND_MAX];
#pragma unroll
    for (int i = 0; i < CAND_MAX; i++) best[i] = 0ull;
    for (int j = tid; j < V; j += ACC_THREADS) {
        const float p = a.greedy ? (j == am ? 1.0f : 0.0f) : lds[j] / S;
        unsigned long long k = ((unsigned long long)__float_as_uint(p) << 32) | (unsigned)(~(unsigned)j);
#pragma unroll
        for (int i = 0; i < CAND_MAX; i++) {
            if (i < n && k > best[i]) {
                const unsigned long long t = best[i];
                best[i] = k;
                k = t;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < CAND_MAX; i++) keys[tid][i] = best[i];
    __syncthreads();
    if (wid != 0) return;
    // ---- wave 0: lane l owns lists l + 64 q; n rounds of a wave-wide max over list heads ----
    int head[ACC_THREADS / 64];
#pragma unroll
    for (int q = 0; q < ACC_THREADS / 64; q++) head[q] = 0;
    for (int r = 0; r < n; r++) {
        unsigned long long mk = 0ull;
        int mq = -1;
#pragma unroll
        for (int q = 0; q < ACC_THREADS / 64; q++) {
            const unsigned long long k = head[q] < n ? keys[lane + 64 * q][head[q]] : 0ull;
            if (k > mk) { mk = k; mq = q; }
        }
        unsigned long long wk = mk;
        for (int d = 32; d >= 1; d >>= 1) {
            const unsigned lo = __shfl_xor((unsigned)wk, d, 64), hi = __shfl_xor((unsigned)(wk >> 32), d, 64);
            const unsigned long long o = ((unsigned long long)hi << 32) | lo;
            wk = o > wk ? o : wk;
        }
        if (mk == wk && mk != 0ull) {
#pragma unroll
            for (int q = 0; q < ACC_THREADS / 64; q++)
                if (q == mq) head[q]++;
        }
        if (lane == 0) {
            a.ids[(size_t)blockIdx.x * n + r] = wk ? ~(unsigned)(wk & 0xFFFFFFFFull) : 0xFFFFFFFFu;
            a.probs[(size_t)blockIdx.x * n + r] = __uint_as_float((unsigned)(wk >> 32));
        }
    }
}

int launch_candidates(const CandArgs& a, hipStream_t stream) {
    if (a.n < 1 || a.n > CAND_MAX || a.rows <= 0 || a.V <= 0) return 2;
    const size_t lds = a.greedy ? 0 : (size_t)a.V * sizeof(float);
    if (lds > MAX_DYN_LDS - sizeof(unsigned long long) * ACC_THREADS * CAND_MAX) return 3;
    static bool attr_set = false;
    if (!attr_set) {
        if (note_error(hipFuncSetAttribute((const void*)candidates_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)(MAX_DYN_LDS - sizeof(unsigned long long) * ACC_THREADS * CAND_MAX))))
            return 4;
        attr_set = true;
    }
    (void)hipGetLastError();
    hipLaunchKernelGGL(candidates_kernel, dim3(a.rows), dim3(ACC_THREADS), lds, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

}  // namespace aarh
