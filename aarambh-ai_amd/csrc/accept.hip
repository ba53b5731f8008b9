// Fused acceptance sampling for speculative verification on gfx950.
//
// Restates, per sequence, the host-side acceptance round of the reference:
//   probabilities     inference/src/sampler.rs:102-118, 226-312 (temperature,
//                     top-k, top-p, softmax, renormalise)
//   accept_proposal   inference/src/speculative.rs:755-768
//   residual          inference/src/speculative.rs:770-793
//   sample            inference/src/sampler.rs:142-152, 314-347
// and the round structure of speculative.rs:343-501 (external draft, bonus
// sample) and mtp_speculative.rs:228-315 (MTP, no bonus).
//
// Stage 1: one workgroup per logits row turns the row into the parameters of
// its sampling distribution (the temperature max, the EXACT sequential f32
// normaliser, the top-k and top-p cut keys and the top-p renormaliser), from
// which any probability is recomputed bit for bit as the reference computes it.
// Stage 2: the last workgroup of each sequence to finish resolves the proposals
// in order, draws ChaCha12 uniforms at the sequence's keystream offset, and on
// rejection walks the residual max(0, p - q): its exact sequential mass, then
// its exact sequential CDF.  Rows longer than one LDS chunk are scanned chunk by
// chunk with the running sum carried over, so the vocabulary size is unbounded.
#include <float.h>

#include <mutex>

#include "device_common.hpp"
#include "kernels.hpp"

namespace aarh {

static constexpr int ACC_THREADS = 512;
static constexpr int ACC_WAVES = ACC_THREADS / WAVE;
static constexpr int ACC_U = 8;              // logit loads a thread issues before consuming them
static constexpr int ACC_CHUNK = 8192;       // floats of a row per scan step; LDS holds two (64 KiB)
static constexpr int CAND_CHUNK = 8192;      // the same for the candidate kernel (its key lists use 20 KiB)
static constexpr int TOPP_PAGE = 4096;       // top-p candidates sorted per page (64-bit keys)
static constexpr int TOPP_LDS_FLOATS = TOPP_PAGE * 3;  // page keys (8 B) + their probabilities (4 B)
// A top-k filter keeping at most TOPK_FAST tokens takes the compact path: every
// probability outside the k survivors is exactly 0, and adding an exact 0 never
// changes an f32 running sum, so the sequential sums and CDFs of the reference
// (index order over the whole row) equal the same sums over the survivors in index
// order.  LDS: survivor keys (8 B), values (4 B) and top-p keys (8 B) per survivor.
static constexpr int TOPK_FAST = 1024;
static constexpr int TOPK_GATHER = 2048;  // candidate keys of the threshold selection (8 B each)
// The fast selection's candidate lists (value, index) follow: 1536 and 2048 entries.
static constexpr int TOPK_LIST0 = TOPK_FAST * 5 + TOPK_GATHER * 2, TOPK_LIST0_CAP = 1536;
static constexpr int TOPK_LIST1 = TOPK_LIST0 + 2 * TOPK_LIST0_CAP, TOPK_LIST1_CAP = 2048;
static constexpr int TOPK_LDS_FLOATS = TOPK_LIST1 + 2 * TOPK_LIST1_CAP;  // 64 KiB
__host__ __device__ __forceinline__ bool topk_compact(int top_k, int V) {
    return top_k > 0 && top_k < V && top_k <= TOPK_FAST;
}

// ---------------------------------------------------------------------------
// Sampling-distribution parameters of one row (filtered_probs, sampler.rs:226-278)
// ---------------------------------------------------------------------------
// Ranking keys: slice::sort_by(total_cmp) descending is stable, so equal values
// keep ascending index order; (value key << 32 | ~index) orders both at once and
// is unique per element.
__device__ __forceinline__ uint64_t logit_key(float l, int j) {
    return ((uint64_t)((uint32_t)total_key(l) ^ 0x80000000u) << 32) | (uint32_t)(~(uint32_t)j);
}
__device__ __forceinline__ uint64_t prob_key(float p, int j) {
    return ((uint64_t)__float_as_uint(p) << 32) | (uint32_t)(~(uint32_t)j);
}

struct RowFilt {
    float T;        // temperature
    float mx;       // max of the finite l / T among the top-k
    float S;        // sequential sum of exp(l / T - mx) (softmax normaliser)
    float R2;       // top-p renormaliser (sum of the kept probabilities)
    uint64_t kkey;  // top-k: logits with logit_key >= kkey are kept (0: all)
    uint64_t pkey;  // top-p: probabilities with prob_key >= pkey are kept (0: all)
    int topp;       // top-p applies
};

// exp(l / T - mx) of element j (0 when top-k drops it or l / T is not finite):
// softmax of the masked logits, sampler.rs:280-299 with temperature 1 after the
// division of :254-265.
__device__ __forceinline__ float filt_exp(const RowFilt& f, float l, int j) {
    if (logit_key(l, j) < f.kkey) return 0.0f;
    const float m = l / f.T;
    if (!isfinite(m)) return 0.0f;
    return expf_rn(m - f.mx);
}
// The probability filtered_probs returns for element j.
__device__ __forceinline__ float filt_prob(const RowFilt& f, float l, int j) {
    const float p0 = filt_exp(f, l, j) / f.S;
    if (!f.topp) return p0;
    if (!(p0 > 0.0f) || prob_key(p0, j) < f.pkey) return 0.0f;
    return p0 / f.R2;
}

// Row statistics handed from stage 1 to the resolving workgroup (ACC_RS_WORDS words per row).
enum { RS_MX = 0, RS_S = 1, RS_R2 = 2, RS_ARGMAX = 3, RS_KKEY = 4, RS_PKEY = 6, RS_FLAGS = 8, RS_STATUS = 9,
       RS_TOPP = 10 };

__device__ __forceinline__ void rs_put(uint32_t* w, int f, uint32_t v) {
    __hip_atomic_store(w + f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t rs_get(const uint32_t* w, int f) {
    return __hip_atomic_load(const_cast<uint32_t*>(w) + f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void rs_store(uint32_t* w, const RowFilt& f, uint32_t flags, int status) {
    rs_put(w, RS_MX, __float_as_uint(f.mx));
    rs_put(w, RS_S, __float_as_uint(f.S));
    rs_put(w, RS_R2, __float_as_uint(f.R2));
    rs_put(w, RS_KKEY, (uint32_t)f.kkey);
    rs_put(w, RS_KKEY + 1, (uint32_t)(f.kkey >> 32));
    rs_put(w, RS_PKEY, (uint32_t)f.pkey);
    rs_put(w, RS_PKEY + 1, (uint32_t)(f.pkey >> 32));
    rs_put(w, RS_FLAGS, flags);
    rs_put(w, RS_STATUS, (uint32_t)status);
    rs_put(w, RS_TOPP, (uint32_t)f.topp);
}
__device__ inline RowFilt rs_load(const uint32_t* w, float T) {
    RowFilt f;
    f.T = T;
    f.mx = __uint_as_float(rs_get(w, RS_MX));
    f.S = __uint_as_float(rs_get(w, RS_S));
    f.R2 = __uint_as_float(rs_get(w, RS_R2));
    f.kkey = (uint64_t)rs_get(w, RS_KKEY) | ((uint64_t)rs_get(w, RS_KKEY + 1) << 32);
    f.pkey = (uint64_t)rs_get(w, RS_PKEY) | ((uint64_t)rs_get(w, RS_PKEY + 1) << 32);
    f.topp = (int)rs_get(w, RS_TOPP);
    return f;
}

// ---------------------------------------------------------------------------
// Workgroup primitives
// ---------------------------------------------------------------------------
struct SelShared {
    unsigned hist[256];
    unsigned long long key;
    int digit, kk;
    unsigned cnt, total;
};

struct AccShared {
    SelShared sel;
    SeqScan scan;
    float red_f[ACC_WAVES], red_g[ACC_WAVES];
    int red_k[ACC_WAVES], red_i[ACC_WAVES];
    unsigned n;
    unsigned is_last;
    float fb[4];
    int ib[8];
};

// hist[d] += number of lanes holding digit d (d < 0: none).  Lanes with equal
// digits are grouped with 8 ballots so each digit costs one LDS atomic per wave.
__device__ __forceinline__ void wave_hist_add(unsigned* hist, int d) {
    const int lane = threadIdx.x & 63;
    const unsigned long long act = __ballot(d >= 0);
    if (act == 0ull) return;
    unsigned long long peers = act;
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const bool bit = (d >> b) & 1;
        const unsigned long long bb = __ballot(bit);
        peers &= bit ? bb : ~bb;
    }
    if (d >= 0 && (__ffsll((long long)peers) - 1) == lane) atomicAdd(&hist[d], (unsigned)__popcll(peers));
}

// Visits every element j of one or two rows [0, n) once: g(j, r0[j], r1[j], valid) is
// called by every thread the same number of times (valid marks real elements), so g
// may vote across the wave.  16-byte loads, ACC_U per row in flight per thread, when
// the rows are 16-byte aligned; 4-byte loads otherwise.
template <int NR, class G>
__device__ __forceinline__ void rows_foreach(const float* r0, const float* r1, int n, const G& g) {
    const int tid = threadIdx.x;
    const bool vec = ((reinterpret_cast<uintptr_t>(r0) | (NR == 2 ? reinterpret_cast<uintptr_t>(r1) : 0)) & 15) == 0;
    int done = 0;
    if (vec) {
        const int n4 = n >> 2;
        const float4_t* a4 = reinterpret_cast<const float4_t*>(r0);
        const float4_t* b4 = reinterpret_cast<const float4_t*>(r1);
        for (int q0 = 0; q0 < n4; q0 += ACC_U * ACC_THREADS) {
            float4_t va[ACC_U], vb[ACC_U];
#pragma unroll
            for (int q = 0; q < ACC_U; q++) {
                const int i4 = q0 + q * ACC_THREADS + tid;
                va[q] = i4 < n4 ? a4[i4] : (float4_t){0.f, 0.f, 0.f, 0.f};
                if (NR == 2) vb[q] = i4 < n4 ? b4[i4] : (float4_t){0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int q = 0; q < ACC_U; q++) {
                const int i4 = q0 + q * ACC_THREADS + tid;
#pragma unroll
                for (int e = 0; e < 4; e++) g(4 * i4 + e, va[q][e], NR == 2 ? vb[q][e] : 0.f, i4 < n4);
            }
        }
        done = n4 * 4;
    }
    for (int j0 = done; j0 < n; j0 += ACC_U * ACC_THREADS) {
        float va[ACC_U], vb[ACC_U];
#pragma unroll
        for (int q = 0; q < ACC_U; q++) {
            const int j = j0 + q * ACC_THREADS + tid;
            va[q] = j < n ? r0[j] : 0.f;
            vb[q] = (NR == 2 && j < n) ? r1[j] : 0.f;
        }
#pragma unroll
        for (int q = 0; q < ACC_U; q++) {
            const int j = j0 + q * ACC_THREADS + tid;
            g(j, va[q], vb[q], j < n);
        }
    }
}

// Block max of v (all threads get it).
__device__ inline float block_max(float v, AccShared* sh) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_max_f32(v);
    if (lane == 0) sh->red_f[wid] = v;
    __syncthreads();
    float m = sh->red_f[0];
    for (int w = 1; w < ACC_WAVES; w++) m = fmaxf(m, sh->red_f[w]);
    __syncthreads();
    return m;
}

// The k-th largest (k >= 1) of the keys kf(l_j, j, ok) with ok and key < U, over
// j in [0, V): an 8-bit MSD radix select (keys are unique, so it ends on one
// key).  Returns 0 when fewer than k keys qualify; *total gets their count.
template <class KF>
__device__ __forceinline__ uint64_t select_desc(const KF& kf, const float* row, int V, int k, uint64_t U, AccShared* sh,
                                unsigned* total) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    uint64_t prefix = 0, mask = 0;
    int kk = k;
    for (int pass = 0; pass < 8; pass++) {
        const int shift = 56 - 8 * pass;
        for (int i = tid; i < 256; i += ACC_THREADS) sh->sel.hist[i] = 0;
        __syncthreads();
        rows_foreach<1>(row, nullptr, V, [&](int j, float l, float, bool valid) {
            int d = -1;
            if (valid) {
                bool ok;
                const uint64_t key = kf(l, j, ok);
                if (ok && key < U && (key & mask) == prefix) d = (int)((key >> shift) & 255);
            }
            wave_hist_add(sh->sel.hist, d);
        });
        __syncthreads();
        if (wid == 0) {
            // lane l holds bins 255 - 4l .. 252 - 4l, so lanes run from the largest digit down
            unsigned c[4], sum = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                c[q] = sh->sel.hist[255 - 4 * lane - q];
                sum += c[q];
            }
            unsigned incl = sum;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const unsigned t = __shfl_up(incl, d, 64);
                if (lane >= d) incl += t;
            }
            const unsigned tot = __shfl(incl, 63, 64);
            const unsigned excl = incl - sum;
            if (lane == 0) {
                if (pass == 0) sh->sel.total = tot;
                if (tot < (unsigned)kk) sh->sel.digit = -1;
            }
            if (tot >= (unsigned)kk && excl < (unsigned)kk && (unsigned)kk <= incl) {
                unsigned run = excl;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    if (run < (unsigned)kk && run + c[q] >= (unsigned)kk) {
                        sh->sel.digit = 255 - 4 * lane - q;
                        sh->sel.kk = kk - (int)run;
                        sh->sel.cnt = c[q];
                    }
                    run += c[q];
                }
            }
        }
        __syncthreads();
        if (pass == 0) *total = sh->sel.total;
        const int d = sh->sel.digit;
        kk = sh->sel.kk;
        const unsigned cnt = sh->sel.cnt;
        __syncthreads();
        if (d < 0) return 0;
        prefix |= (uint64_t)d << shift;
        mask |= (uint64_t)255 << shift;
        if (cnt == 1 && pass < 7) {
            // one key carries this prefix: it is the k-th
            for (int j = tid; j < V; j += ACC_THREADS) {
                bool ok;
                const uint64_t key = kf(row[j], j, ok);
                if (ok && key < U && (key & mask) == prefix) sh->sel.key = key;
            }
            __syncthreads();
            const uint64_t r = sh->sel.key;
            __syncthreads();
            return r;
        }
    }
    return prefix;
}

// Exact sequential sum of f(a_j, b_j, j) >= 0 over j in [0, n) (a = r0[j], b = r1[j]
// for NR = 2), with the inverse-CDF crossing for u >= 0.  The row goes through LDS in
// chunks of `chunk` values, double buffered (buf holds 2 * chunk floats): every wave
// writes chunk 0, then wave 0 scans chunk c, carrying the running sum, while the
// other waves write chunk c + 1 into the other half.
template <int NR, class F>
__device__ __forceinline__ SeqScan block_seq_scan(const float* r0, const float* r1, int n, float u, const F& f, float* buf,
                                  int chunk, AccShared* sh) {
    const int tid = threadIdx.x, wid = tid >> 6;
    SeqScan st = seq_scan_init();
    rows_foreach<NR>(r0, NR == 2 ? r1 : nullptr, min(chunk, n), [&](int i, float a, float b, bool valid) {
        if (valid) buf[i] = f(a, b, i);
    });
    __syncthreads();
    for (int c0 = 0; c0 < n; c0 += chunk) {
        const int m = min(chunk, n - c0);
        float* cur = buf + ((c0 / chunk) & 1) * chunk;
        if (wid == 0) {
            seq_scan_wave(cur, m, u, c0, st);
        } else if (c0 + chunk < n) {
            const int c1 = c0 + chunk, m1 = min(chunk, n - c1);
            float* nxt = buf + (((c0 / chunk) + 1) & 1) * chunk;
            constexpr int NT = ACC_THREADS - 64, U = 4;
            for (int i0 = tid - 64; i0 < m1; i0 += U * NT) {
                float va[U], vb[U];
#pragma unroll
                for (int q = 0; q < U; q++) {
                    const int i = i0 + q * NT;
                    va[q] = i < m1 ? r0[c1 + i] : 0.f;
                    vb[q] = (NR == 2 && i < m1) ? r1[c1 + i] : 0.f;
                }
#pragma unroll
                for (int q = 0; q < U; q++) {
                    const int i = i0 + q * NT;
                    if (i < m1) nxt[i] = f(va[q], vb[q], c1 + i);
                }
            }
        }
        __syncthreads();
    }
    if (tid == 0) sh->scan = st;
    __syncthreads();
    const SeqScan r = sh->scan;
    __syncthreads();
    return r;
}

// Argmax with the last index on ties under total_cmp (sampler.rs:217-224).
__device__ inline int block_argmax(const float* row, int V, AccShared* sh) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    int bk = INT_MIN, bi = 0;
    rows_foreach<1>(row, nullptr, V, [&](int j, float l, float, bool valid) {
        if (valid) {
            const int k = total_key(l);
            if (k > bk || (k == bk && j > bi)) { bk = k; bi = j; }
        }
    });
    for (int d = 32; d >= 1; d >>= 1) {
        const int ok = __shfl_xor(bk, d, 64), oi = __shfl_xor(bi, d, 64);
        if (ok > bk || (ok == bk && oi > bi)) { bk = ok; bi = oi; }
    }
    if (lane == 0) { sh->red_k[wid] = bk; sh->red_i[wid] = bi; }
    __syncthreads();
    int k0 = sh->red_k[0], i0 = sh->red_i[0];
    for (int w = 1; w < ACC_WAVES; w++)
        if (sh->red_k[w] > k0 || (sh->red_k[w] == k0 && sh->red_i[w] > i0)) { k0 = sh->red_k[w]; i0 = sh->red_i[w]; }
    __syncthreads();
    return i0;
}

// Bitonic sort of keys[0..np2) into descending order (np2 a power of two).
__device__ inline void block_sort_desc(unsigned long long* keys, int np2) {
    for (int k = 2; k <= np2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < np2; i += ACC_THREADS) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const unsigned long long a = keys[i], b = keys[ixj];
                    const bool desc = (i & k) == 0;
                    if (desc ? a < b : a > b) {
                        keys[i] = b;
                        keys[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Appends make(j, l) for every element j of row[0..V) with take(l, j) to out[0..cap)
// in arbitrary order and returns the count (taken elements past cap are counted, not
// written).  Meant for rare takes: a thread tests 16 elements per step into a bit mask
// and the wave computes slots only in the steps where some lane took one.
template <class P, class M>
__device__ inline int gather_rare(const float* row, int V, const P& take, const M& make, unsigned long long* out,
                                  int cap, AccShared* sh) {
    if (threadIdx.x == 0) sh->n = 0;
    __syncthreads();
    // each taken element claims a slot with one LDS atomic (taken elements are rare, and the
    // callers rank the list by unique keys, so the slot order does not matter)
    rows_foreach<1>(row, nullptr, V, [&](int j, float l, float, bool valid) {
        if (valid && take(l, j)) {
            const unsigned slot = atomicAdd(&sh->n, 1u);
            if (slot < (unsigned)cap) out[slot] = make(l, j);
        }
    });
    __syncthreads();
    const int n = (int)sh->n;
    __syncthreads();
    return n;
}

// Sequential f32 sum of v[0..n) (index order) on wave 0 from registers, 64 values per
// load; returned to the whole workgroup.
__device__ inline float seq_sum_w0(const float* v, int n, AccShared* sh) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        float s = 0.0f;
        for (int c0 = 0; c0 < n; c0 += 64) {
            const int cnt = min(64, n - c0);
            const float x = lane < cnt ? v[c0 + lane] : 0.0f;
            for (int i = 0; i < cnt; i++) s += readlane_f32(x, i);
        }
        if (lane == 0) sh->fb[0] = s;
    }
    __syncthreads();
    const float s = sh->fb[0];
    __syncthreads();
    return s;
}

// Places the n unique keys in[0..n) into out[0..n) in descending order by rank (the
// number of keys above each), without a sorting network: O(n^2 / threads) LDS
// broadcast reads and two barriers.
__device__ inline void rank_sort_desc(const unsigned long long* in, unsigned long long* out, int n) {
    for (int i = threadIdx.x; i < n; i += ACC_THREADS) {
        const unsigned long long k = in[i];
        int r = 0;
        for (int j = 0; j < n; j++) r += in[j] > k;
        out[r] = k;
    }
    __syncthreads();
}

// The survivors of a top-k filter (logit keys >= kkey) of `row`, gathered in LDS and
// sorted by ascending index: keys[i] = (~index << 32 | logit bits).  Returns their
// count (<= TOPK_FAST; the keys are unique, so it is exactly k).
__device__ inline int topk_survivors(const float* row, int V, uint64_t kkey, unsigned long long* keys, AccShared* sh) {
    // the keys >= kkey: logits whose value key is above kkey's, or equal with index <= kkey's
    const uint32_t kv = (uint32_t)(kkey >> 32);
    const int kj = (int)~(uint32_t)kkey;
    const int n = min(gather_rare(
                          row, V,
                          [&](float l, int j) {
                              const uint32_t v = (uint32_t)total_key(l) ^ 0x80000000u;
                              return v > kv || (v == kv && j <= kj);
                          },
                          [](float l, int j) {
                              return ((unsigned long long)(~(uint32_t)j) << 32) | (unsigned long long)__float_as_uint(l);
                          },
                          keys + TOPK_FAST, TOPK_FAST, sh),
                      TOPK_FAST);
    // ranked descending by ~index: ascending index
    rank_sort_desc(keys + TOPK_FAST, keys, n);
    return n;
}
__device__ __forceinline__ int surv_index(unsigned long long k) { return (int)~(uint32_t)(k >> 32); }
__device__ __forceinline__ float surv_logit(unsigned long long k) { return __uint_as_float((uint32_t)k); }

// Inverse CDF of sample_from_probs (sampler.rs:337-347) over survivors in index order
// with values v[i] / div (div = 1: the values themselves), on thread 0: the first index
// with u <= cumulative, as seq_scan_wave reports it (u <= 0 stops at index 0 with the
// partial sums 0).
__device__ inline SeqScan block_cdf_small(const unsigned long long* keys, const float* v, int n, float div, float u,
                                          AccShared* sh) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        SeqScan st = seq_scan_init();
        if (u <= 0.0f) st.cross = 0;
        float s = 0.0f;
        for (int c0 = 0; c0 < n; c0 += 64) {
            const int cnt = min(64, n - c0);
            const float x = lane < cnt ? (div == 1.0f ? v[c0 + lane] : v[c0 + lane] / div) : 0.0f;
            for (int i = 0; i < cnt; i++) {
                const float before = s;
                s += readlane_f32(x, i);
                if (st.cross < 0 && u <= s) {
                    st.cross = surv_index(keys[c0 + i]);
                    st.s_at = s;
                    st.s_before = before;
                }
            }
        }
        st.s = s;
        if (lane == 0) sh->scan = st;
    }
    __syncthreads();
    const SeqScan r = sh->scan;
    __syncthreads();
    return r;
}

// Band of a finite logit l below the row max mx: q = (mx - l) / R (R = mx - mn, taken as
// (mx - l) * (1 / R)) in quarter octaves, b = 4 * (-exponent of q) - (top two fraction
// bits of q) - 1, clamped to [0, 63].  b is non-decreasing in l, so {b >= c} is an upper
// set of logit values; the top quarter of the range is b >= 8.
__device__ __forceinline__ int topk_band(float l, float mx, float rinv) {
    const float q = (mx - l) * rinv;
    if (!(q > 0.0f)) return 63;
    const uint32_t u = __float_as_uint(q);
    const int e = (int)((u >> 23) & 255u) - 127;
    return max(0, min(63, -4 * e - (int)((u >> 21) & 3u) - 1));
}

// Top-k selection for k <= TOPK_FAST without radix passes.  Bands: b(l) of topk_band
// relative to the row's finite max / min, non-decreasing in l; the top quarter of the
// range is b >= 8.  One pass takes the finite max / min; a second lists (value, index) of
// every logit above thr, a threshold below which b < 8 is certain (a cheap compare per
// logit; only the list gets banded), and the largest logit at or below thr.  From the list:
// a histogram of the top-quarter bands and the narrowest upper set of bands holding at
// least k logits (at most TOPK_GATHER); ranking those keys gives the k-th key, and
// ranking the k survivors by index puts them in keys[0..k) as topk_survivors leaves them.
// Rows with a few logits far above the rest (an MTP head scores the token it was fed far
// above every other) hold fewer than k logits in the top quarter: a third pass lists the
// logits in the top quarter of the range below those (up to the largest logit outside the
// top quarter), bands them relative to it, and completes k from its narrowest upper set.
// Both sets are upper sets in logit value, so their union holds the k largest keys.
// Returns false (the caller falls back to the radix select) on non-finite logits, a
// constant row, a range too narrow for the threshold's margin (R <= 0.01 |max|), a list
// past its capacity, or when no band set of at most TOPK_GATHER logits holds k.
__device__ inline bool topk_fast_select(const float* row, int V, int k, float* buf, AccShared* sh, uint64_t* kkey) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    unsigned long long* keys = (unsigned long long*)buf;
    unsigned long long* cand = (unsigned long long*)(buf + 5 * TOPK_FAST);
    unsigned long long* tmp = (unsigned long long*)(buf + 3 * TOPK_FAST);  // k <= TOPK_FAST entries
    unsigned long long* list0 = (unsigned long long*)(buf + TOPK_LIST0);
    unsigned long long* list1 = (unsigned long long*)(buf + TOPK_LIST1);
    float mx = -INFINITY, mn = INFINITY;
    int nonfin = 0;
    rows_foreach<1>(row, nullptr, V, [&](int j, float l, float, bool valid) {
        if (valid) {
            if (isfinite(l)) {
                mx = fmaxf(mx, l);
                mn = fminf(mn, l);
            } else {
                nonfin = 1;
            }
        }
    });
    mx = wave_max_f32(mx);
    mn = -wave_max_f32(-mn);
    nonfin = __any(nonfin) ? 1 : 0;
    if (lane == 0) {
        sh->red_f[wid] = mx;
        sh->red_i[wid] = nonfin;
        sh->red_k[wid] = __float_as_int(mn);
    }
    __syncthreads();
    for (int w = 0; w < ACC_WAVES; w++) {
        mx = fmaxf(mx, sh->red_f[w]);
        mn = fminf(mn, __int_as_float(sh->red_k[w]));
        nonfin |= sh->red_i[w];
    }
    __syncthreads();
    // A logit at or below top - 0.2501 range lies in band < 8 (relative to top) whatever the
    // rounding of (top - l) / range: the 0.0001 range margin exceeds the rounding of top - l
    // whenever range > 0.01 |top|.  -INFINITY: no such threshold.
    auto skip_below = [](float top, float range) {
        return range > 0.01f * fabsf(top) ? top - 0.2501f * range : -INFINITY;
    };
    const float R = mx - mn;
    if (nonfin || !(R > 0.0f) || !isfinite(R)) return false;
    const float rinv = 1.0f / R, thr = skip_below(mx, R);
    if (thr == -INFINITY) return false;
    // (value, index) of every logit with lo < l <= hi into out (cap entries); the largest
    // logit at or below lo goes to *below_lo (-INFINITY for none); returns the count
    auto list_pass = [&](float lo, float hi, unsigned long long* out, int cap, float* below_lo) {
        if (tid == 0) sh->n = 0;
        __syncthreads();
        float bl = -INFINITY;
        rows_foreach<1>(row, nullptr, V, [&](int j, float l, float, bool valid) {
            if (valid && l > lo && l <= hi) {
                const unsigned slot = atomicAdd(&sh->n, 1u);
                if (slot < (unsigned)cap)
                    out[slot] = ((unsigned long long)__float_as_uint(l) << 32) | (unsigned long long)(uint32_t)j;
            } else if (valid && l <= lo) {
                bl = fmaxf(bl, l);
            }
        });
        bl = wave_max_f32(bl);
        if (lane == 0) sh->red_g[wid] = bl;
        __syncthreads();
        bl = -INFINITY;
        for (int w = 0; w < ACC_WAVES; w++) bl = fmaxf(bl, sh->red_g[w]);
        *below_lo = bl;
        const int n = (int)sh->n;
        __syncthreads();
        return n;
    };
    auto ent_l = [](unsigned long long e) { return __uint_as_float((uint32_t)(e >> 32)); };
    auto ent_j = [](unsigned long long e) { return (int)(uint32_t)e; };
    // histogram of bands >= 8 of the listed logits (relative to top / tinv); returns through
    // sh->red_g the largest listed logit in a band < 8
    auto band_hist = [&](const unsigned long long* lst, int n, float top, float tinv) {
        if (tid < 64) sh->sel.hist[tid] = 0u;
        __syncthreads();
        float bl = -INFINITY;
        for (int i = tid; i < n; i += ACC_THREADS) {
            const float l = ent_l(lst[i]);
            const int b = topk_band(l, top, tinv);
            if (b >= 8) atomicAdd(&sh->sel.hist[b], 1u);
            else bl = fmaxf(bl, l);
        }
        bl = wave_max_f32(bl);
        if (lane == 0) sh->red_g[wid] = bl;
        __syncthreads();
    };
    // pick: the lowest band of the narrowest upper set holding `need` logits; -1 when the
    // counted bands hold fewer (their total in sel.total), -2 when that set exceeds `room`
    auto pick_band = [&](unsigned need, unsigned room) {
        unsigned acc = 0;
        for (int b = 63; b >= 8; b--) {
            acc += sh->sel.hist[b];
            if (acc >= need) {
                sh->sel.digit = acc <= room ? b : -2;
                return;
            }
        }
        sh->sel.digit = -1;
        sh->sel.total = acc;
    };

    float below_lo;
    const int n0 = list_pass(thr, INFINITY, list0, TOPK_LIST0_CAP, &below_lo);
    if (n0 > TOPK_LIST0_CAP) return false;
    band_hist(list0, n0, mx, rinv);
    float below = below_lo;  // largest logit outside the top quarter
    for (int w = 0; w < ACC_WAVES; w++) below = fmaxf(below, sh->red_g[w]);
    if (tid == 0) pick_band((unsigned)k, (unsigned)TOPK_GATHER);
    __syncthreads();
    const int band = sh->sel.digit;
    const unsigned top = sh->sel.total;
    __syncthreads();
    if (band == -2) return false;
    int c = 0;
    if (band >= 8) {
        // candidates: the listed logits in bands >= band
        if (tid == 0) sh->n = 0;
        __syncthreads();
        for (int i = tid; i < n0; i += ACC_THREADS) {
            const unsigned long long e = list0[i];
            if (topk_band(ent_l(e), mx, rinv) >= band) cand[atomicAdd(&sh->n, 1u)] = logit_key(ent_l(e), ent_j(e));
        }
        __syncthreads();
        c = (int)sh->n;
        __syncthreads();
    } else {
        // second level below the top quarter: bands relative to its largest logit mx1
        const float mx1 = below, R1 = mx1 - mn;
        if (!(R1 > 0.0f) || !isfinite(R1)) return false;
        const float rinv1 = 1.0f / R1, thr1 = skip_below(mx1, R1);
        if (thr1 == -INFINITY) return false;
        float unused;
        const int n1 = list_pass(thr1, mx1, list1, TOPK_LIST1_CAP, &unused);
        if (n1 > TOPK_LIST1_CAP) return false;
        band_hist(list1, n1, mx1, rinv1);
        if (tid == 0) pick_band((unsigned)k - top, (unsigned)TOPK_GATHER - top);
        __syncthreads();
        const int band1 = sh->sel.digit;
        __syncthreads();
        if (band1 < 0) return false;
        // candidates: the top quarter (the logits above mx1) and the second-level set
        if (tid == 0) sh->n = 0;
        __syncthreads();
        for (int i = tid; i < n0; i += ACC_THREADS) {
            const unsigned long long e = list0[i];
            if (ent_l(e) > mx1) cand[atomicAdd(&sh->n, 1u)] = logit_key(ent_l(e), ent_j(e));
        }
        for (int i = tid; i < n1; i += ACC_THREADS) {
            const unsigned long long e = list1[i];
            if (topk_band(ent_l(e), mx1, rinv1) >= band1) cand[atomicAdd(&sh->n, 1u)] = logit_key(ent_l(e), ent_j(e));
        }
        __syncthreads();
        c = (int)sh->n;
        __syncthreads();
    }
    // the k largest candidate keys, by rank; the k-th is the top-k cut
    for (int i = tid; i < c; i += ACC_THREADS) {
        const unsigned long long key = cand[i];
        int r = 0;
        for (int j = 0; j < c; j++) r += cand[j] > key;
        if (r < k) {
            const int jj = (int)~(uint32_t)key;
            tmp[r] = ((unsigned long long)(~(uint32_t)jj) << 32) | (unsigned long long)__float_as_uint(row[jj]);
            if (r == k - 1) sh->sel.key = key;
        }
    }
    __syncthreads();
    *kkey = sh->sel.key;
    // survivors (~index << 32 | logit bits): descending order is ascending index
    rank_sort_desc(tmp, keys, k);
    return true;
}

// filtered_probs (sampler.rs:226-278) for a top-k row on the compact path; f.kkey is set.
// The k survivors are in buf (keys[0..n), sorted by index, as topk_survivors leaves them).
__device__ inline void row_filter_topk(float top_p, int n, float* buf, AccShared* sh, RowFilt& f, uint32_t& flags,
                                       int& status) {
    const int tid = threadIdx.x;
    unsigned long long* keys = (unsigned long long*)buf;
    float* vals = buf + 2 * TOPK_FAST;
    unsigned long long* pk = (unsigned long long*)(buf + 3 * TOPK_FAST);
    float mx = -INFINITY;
    for (int i = tid; i < n; i += ACC_THREADS) {
        const float m = surv_logit(keys[i]) / f.T;
        if (isfinite(m)) mx = fmaxf(mx, m);
    }
    mx = block_max(mx, sh);
    if (!(mx > -INFINITY)) {  // "all logits are non-finite" (sampler.rs:286-288)
        status = 1;
        return;
    }
    f.mx = mx;
    const RowFilt fe = f;
    for (int i = tid; i < n; i += ACC_THREADS) vals[i] = filt_exp(fe, surv_logit(keys[i]), surv_index(keys[i]));
    __syncthreads();
    f.S = seq_sum_w0(vals, n, sh);
    if (!(f.S > 0.0f) || !isfinite(f.S)) {
        status = 1;
        return;
    }
    if (!f.topp) return;
    // top-p: probabilities in descending (stable) order, cumulative until it reaches top_p
    // probability keys (0 for p = 0), ranked descending: the positive keys are unique and
    // take ranks 0 .. P-1; every zero key has rank P and writes the 0 that ends the walk
    unsigned long long* pk_in = (unsigned long long*)(buf + 5 * TOPK_FAST);
    for (int i = tid; i < n; i += ACC_THREADS) {
        const float p = vals[i] / f.S;
        vals[i] = p;
        pk_in[i] = p > 0.0f ? prob_key(p, surv_index(keys[i])) : 0ull;
    }
    __syncthreads();
    for (int i = tid; i < n; i += ACC_THREADS) {
        const unsigned long long k = pk_in[i];
        int r = 0;
        for (int j = 0; j < n; j++) r += pk_in[j] > k;
        pk[r] = k;
    }
    __syncthreads();
    if (tid < 64) {
        // cumulative in descending probability order until it reaches top_p (wave 0, registers)
        const int lane = tid;
        float cum = 0.0f;
        unsigned long long pkey = 0ull;
        bool done = false;
        for (int c0 = 0; c0 < n && !done; c0 += 64) {
            const int cnt = min(64, n - c0);
            const unsigned long long k = lane < cnt ? pk[c0 + lane] : 0ull;
            const float p = __uint_as_float((uint32_t)(k >> 32));
            for (int i = 0; i < cnt; i++) {
                const float pi = readlane_f32(p, i);
                if (!(pi > 0.0f)) {  // the zero keys: every positive probability taken
                    done = true;
                    break;
                }
                const float before = cum;
                cum += pi;
                if (top_p <= cum) {
                    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, i);
                    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), i);
                    pkey = ((unsigned long long)hi << 32) | lo;
                    if (fminf(cum - top_p, top_p - before) < 1e-6f && lane == 0) sh->ib[7] = (int)ACCEPT_FLAG_TOPP_NEAR;
                    done = true;
                    break;
                }
            }
        }
        if (lane == 0) sh->sel.key = pkey;
    }
    __syncthreads();
    f.pkey = sh->sel.key;
    // renormalise over the kept probabilities, sequential in index order
    float* kept = (float*)(buf + 5 * TOPK_FAST);  // pk_in is dead after the ranking
    for (int i = tid; i < n; i += ACC_THREADS) {
        const float p0 = vals[i];
        kept[i] = (p0 > 0.0f && prob_key(p0, surv_index(keys[i])) >= f.pkey) ? p0 : 0.0f;
    }
    __syncthreads();
    f.R2 = seq_sum_w0(kept, n, sh);
    flags |= (uint32_t)sh->ib[7];
    __syncthreads();
    if (!(f.R2 > 0.0f) || !isfinite(f.R2)) status = 1;
}

// Distribution parameters of a sampled row (TopKTopP at T > EPSILON):
// filtered_probs (sampler.rs:226-278).  status 1: no finite logit survives or a
// normaliser is not positive (the reference returns Err).  flags: the top-p
// cumulative sum crossed top_p within 1e-6 (its decision may flip with an ulp).
__device__ __forceinline__ void row_filter(const float* row, int V, float T, int top_k, float top_p, float* buf, int chunk,
                           AccShared* sh, RowFilt& f, uint32_t& flags, int& status) {
    const int tid = threadIdx.x, wid = tid >> 6;
    f.T = T;
    f.kkey = 0;
    f.pkey = 0;
    f.R2 = 1.0f;
    f.S = 1.0f;
    f.mx = 0.0f;
    f.topp = (top_p > 0.0f && top_p < 1.0f) ? 1 : 0;
    flags = 0;
    status = 0;
    // ---- top-k: the k-th largest logit key under the stable total_cmp ranking ----
    if (top_k > 0 && top_k < V) {
        auto kf = [](float l, int j, bool& ok) {
            ok = true;
            return logit_key(l, j);
        };
        if (topk_compact(top_k, V)) {
            if (tid == 0) sh->ib[7] = 0;
            __syncthreads();
            int n = top_k;
            if (!topk_fast_select(row, V, top_k, buf, sh, &f.kkey)) {
                unsigned tot;
                f.kkey = select_desc(kf, row, V, top_k, ~0ull, sh, &tot);
                n = topk_survivors(row, V, f.kkey, (unsigned long long*)buf, sh);
            }
            // survivors stay in buf[0 .. 2 n) (keys sorted by index) for a resolver in this workgroup
            if (threadIdx.x == 0) sh->ib[6] = n;
            row_filter_topk(top_p, n, buf, sh, f, flags, status);
            return;
        }
        unsigned tot;
        f.kkey = select_desc(kf, row, V, top_k, ~0ull, sh, &tot);
    }
    // ---- max of the finite masked logits ----
    float mx = -INFINITY;
    const uint64_t kk = f.kkey;
    rows_foreach<1>(row, nullptr, V, [&](int j, float l, float, bool valid) {
        if (valid && logit_key(l, j) >= kk) {
            const float m = l / T;
            if (isfinite(m)) mx = fmaxf(mx, m);
        }
    });
    mx = block_max(mx, sh);
    if (!(mx > -INFINITY)) {  // "all logits are non-finite" (sampler.rs:286-288)
        status = 1;
        return;
    }
    f.mx = mx;
    // ---- softmax normaliser: exact sequential sum in index order ----
    const RowFilt fe = f;
    const SeqScan s1 = block_seq_scan<1>(
        row, nullptr, V, -1.0f, [&](float a, float, int j) { return filt_exp(fe, a, j); }, buf, chunk, sh);
    f.S = s1.s;
    if (!(f.S > 0.0f) || !isfinite(f.S)) {
        status = 1;
        return;
    }
    if (!f.topp) return;
    // ---- top-p: walk the probabilities in descending (stable) order, a page of the
    // TOPP_PAGE next-largest keys at a time, with the exact sequential cumulative ----
    const RowFilt fp = f;
    auto pkf = [&](float l, int j, bool& ok) {
        const float p = filt_exp(fp, l, j) / fp.S;
        ok = p > 0.0f;
        return prob_key(p, j);
    };
    unsigned long long* keys = (unsigned long long*)buf;
    float* vals = buf + 2 * TOPP_PAGE;
    uint64_t U = ~0ull;
    float carry = 0.0f;
    uint64_t pkey = 0;
    for (;;) {
        unsigned remain = 0;
        const uint64_t L = select_desc(pkf, row, V, TOPP_PAGE, U, sh, &remain);  // 0: fewer than a page left
        if (remain == 0) break;  // every positive probability taken without reaching top_p: keep all
        if (tid == 0) sh->n = 0;
        __syncthreads();
        rows_foreach<1>(row, nullptr, V, [&](int j, float l, float, bool valid) {
            bool ok = false;
            uint64_t key = 0;
            if (valid) key = pkf(l, j, ok);
            const bool take = ok && key < U && key >= L;
            const unsigned long long m = __ballot(take);
            unsigned base = 0;
            if ((threadIdx.x & 63) == 0 && m) base = atomicAdd(&sh->n, (unsigned)__popcll(m));
            base = __shfl(base, 0, 64);
            const unsigned slot = base + (unsigned)__popcll(m & ((1ull << (threadIdx.x & 63)) - 1ull));
            if (take && slot < (unsigned)TOPP_PAGE) keys[slot] = key;
        });
        __syncthreads();
        const int n = min((int)sh->n, TOPP_PAGE);
        int np2 = 1;
        while (np2 < n) np2 <<= 1;
        for (int i = n + tid; i < np2; i += ACC_THREADS) keys[i] = 0ull;
        __syncthreads();
        block_sort_desc(keys, np2);
        for (int i = tid; i < n; i += ACC_THREADS) vals[i] = __uint_as_float((uint32_t)(keys[i] >> 32));
        __syncthreads();
        if (wid == 0) {
            SeqScan st = seq_scan_init();
            st.s = carry;
            seq_scan_wave(vals, n, top_p, 0, st);
            if (tid == 0) sh->scan = st;
        }
        __syncthreads();
        const SeqScan st = sh->scan;
        carry = st.s;
        if (st.cross >= 0) {
            pkey = keys[st.cross];
            if (fminf(st.s_at - top_p, top_p - st.s_before) < 1e-6f) flags |= ACCEPT_FLAG_TOPP_NEAR;
            __syncthreads();
            break;
        }
        __syncthreads();
        if (L == 0) break;  // that was the last (partial) page: keep all
        U = L;
    }
    f.pkey = pkey;
    // ---- renormalise over the kept probabilities (sequential sum in index order) ----
    const RowFilt fr = f;
    const SeqScan s2 = block_seq_scan<1>(
        row, nullptr, V, -1.0f,
        [&](float a, float, int j) {
            const float p0 = filt_exp(fr, a, j) / fr.S;
            return (p0 > 0.0f && prob_key(p0, j) >= fr.pkey) ? p0 : 0.0f;
        },
        buf, chunk, sh);
    f.R2 = s2.s;
    if (!(f.R2 > 0.0f) || !isfinite(f.R2)) status = 1;
}

__device__ __forceinline__ int acc_chunk_floats(int V) { return V < ACC_CHUNK ? V : ACC_CHUNK; }

// Row statistics with every field read once into scalar registers (they are uniform).
__device__ __forceinline__ RowFilt rs_load_uniform(const uint32_t* w, float T) {
    RowFilt f = rs_load(w, T);
    f.mx = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(f.mx)));
    f.S = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(f.S)));
    f.R2 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(f.R2)));
    f.kkey = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)f.kkey) |
             ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(f.kkey >> 32)) << 32);
    f.pkey = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)f.pkey) |
             ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(f.pkey >> 32)) << 32);
    f.topp = __builtin_amdgcn_readfirstlane(f.topp);
    return f;
}

// The resolver's draw on the compact top-k path.  wd == nullptr: the bonus draw from
// the target row's distribution.  Otherwise the residual max(0, p - q), which is 0
// outside the target row's top-k survivors: its exact mass, then its exact CDF.
// have >= 0: the survivors of the target row are already in lds (this workgroup filtered it).
__device__ __noinline__ void resolve_compact(const uint32_t* wt, const uint32_t* wd, const float* tl, const float* dl,
                                             int V, float T, float u, float* lds, AccShared* sh, SeqScan* cdf,
                                             int* status, int have) {
    const int tid = threadIdx.x;
    unsigned long long* ckeys = (unsigned long long*)lds;
    float* cvals = lds + 2 * TOPK_FAST;
    const RowFilt ft = rs_load_uniform(wt, T);
    const int n = have >= 0 ? have : topk_survivors(tl, V, ft.kkey, ckeys, sh);
    if (wd) {
        const RowFilt fd = rs_load_uniform(wd, T);
        for (int i = tid; i < n; i += ACC_THREADS) {
            const int j = surv_index(ckeys[i]);
            const float d = filt_prob(ft, surv_logit(ckeys[i]), j) - filt_prob(fd, dl[j], j);
            cvals[i] = d > 0.0f ? d : 0.0f;
        }
        __syncthreads();
        const float R = seq_sum_w0(cvals, n, sh);
        if (!isfinite(R) || R <= FLT_EPSILON)
            *status = 1;
        else
            *cdf = block_cdf_small(ckeys, cvals, n, R, u, sh);
    } else {
        for (int i = tid; i < n; i += ACC_THREADS) cvals[i] = filt_prob(ft, surv_logit(ckeys[i]), surv_index(ckeys[i]));
        __syncthreads();
        *cdf = block_cdf_small(ckeys, cvals, n, 1.0f, u, sh);
    }
}

// ---------------------------------------------------------------------------
// Acceptance kernel: grid = B * (target_rows + K) workgroups.
// ---------------------------------------------------------------------------
// Four waves per SIMD (at most 128 VGPRs, the rest spilled): two 8-wave workgroups
// per CU, so C2's 288 rows run in one dispatch round (measured faster than one
// workgroup per CU with no spills, also on the top-k / top-p path).
__global__ void __launch_bounds__(ACC_THREADS) __attribute__((amdgpu_waves_per_eu(4, 4))) accept_kernel(AcceptArgs a) {
    extern __shared__ float lds[];
    __shared__ AccShared sh;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rows_per_seq = a.target_rows + a.K;
    const int b = blockIdx.x / rows_per_seq;
    const int r = blockIdx.x % rows_per_seq;
    const int V = a.V;
    const int chunk = a.chunk;
    int np = a.n_proposals ? a.n_proposals[b] : a.K;
    np = np < 0 ? 0 : (np > a.K ? a.K : np);

    // ---------------- stage 1: per-row distribution parameters ----------------
    const bool is_target = r < a.target_rows;
    const int ridx = is_target ? r : r - a.target_rows;
    const bool needed = is_target ? (ridx < np || (a.bonus && ridx == np)) : (ridx < np);
    const size_t row_id = (size_t)b * rows_per_seq + r;
    const float* row = is_target ? a.target + ((size_t)b * a.target_rows + ridx) * V
                                 : a.draft + ((size_t)b * a.K + ridx) * V;
    if (needed) {
        uint32_t* w = a.rstat + row_id * ACC_RS_WORDS;
        if (a.greedy) {
            const int am = block_argmax(row, V, &sh);
            if (tid == 0) rs_put(w, RS_ARGMAX, (uint32_t)am);
        } else {
            RowFilt f;
            uint32_t fl;
            int stt;
            row_filter(row, V, a.temperature, a.top_k, a.top_p, lds, chunk, &sh, f, fl, stt);
            if (tid == 0) rs_store(w, f, fl, stt);
        }
    }

    // ---------------- last workgroup of the sequence resolves ----------------
    if (!arrive_last(&a.counters[b], (unsigned)rows_per_seq, &sh.is_last)) return;

    const uint32_t* rs0 = a.rstat + (size_t)b * rows_per_seq * ACC_RS_WORDS;
    const uint32_t* rsd0 = rs0 + (size_t)a.target_rows * ACC_RS_WORDS;
    const float* trow0 = a.target + (size_t)b * a.target_rows * V;
    const float* drow0 = a.draft + (size_t)b * a.K * V;
    const float T = a.temperature;

    // The resolution draws at most np + 1 uniforms (one per acceptance test, one resample),
    // keystream words word .. word + np: lane d of wave 0 computes draw d (one ChaCha block
    // each, in parallel) instead of thread 0 computing them one after another.
    __shared__ float u_s[64];
    const bool par_u = !a.greedy && np + 1 <= 64;
    if (par_u && tid <= np) {
        if (a.uniforms) {
            u_s[tid] = a.uniforms[(size_t)b * (a.K + 1) + tid];
        } else {
            uint32_t key[8];
            rng_key_from_seed(a.seeds ? a.seeds[b] : 0ull, key);
            u_s[tid] = rng_f32(key, (a.word_offsets ? a.word_offsets[b] : 0ull) + tid);
        }
    }
    __syncthreads();

    if (tid == 0) {
        uint32_t key[8];
        if (!par_u) rng_key_from_seed(a.seeds ? a.seeds[b] : 0ull, key);
        const uint64_t word = a.word_offsets ? a.word_offsets[b] : 0ull;
        int draws = 0, acc = 0, rej = -1, status = 0;
        uint32_t flags = 0;
        for (int i = 0; i < np; i++) {
            if (a.greedy) {
                if (rs_get(rsd0 + i * ACC_RS_WORDS, RS_ARGMAX) == rs_get(rs0 + i * ACC_RS_WORDS, RS_ARGMAX)) {
                    acc++;
                    continue;
                }
                rej = i;
                break;
            }
            const uint32_t* wt = rs0 + i * ACC_RS_WORDS;
            const uint32_t* wd = rsd0 + i * ACC_RS_WORDS;
            flags |= rs_get(wt, RS_FLAGS) | rs_get(wd, RS_FLAGS);
            if (rs_get(wt, RS_STATUS) | rs_get(wd, RS_STATUS)) {
                status = 1;
                rej = i;
                break;
            }
            const uint32_t x = a.draft_tokens[(size_t)b * a.K + i];
            float p = 0.0f, q = 0.0f;
            if ((int)x < V) {
                p = filt_prob(rs_load(wt, T), trow0[(size_t)i * V + x], (int)x);
                q = filt_prob(rs_load(wd, T), drow0[(size_t)i * V + x], (int)x);
            }
            if (!(q > 0.0f)) {
                rej = i;
                break;
            }
            const float u = par_u       ? u_s[draws]
                            : a.uniforms ? a.uniforms[(size_t)b * (a.K + 1) + draws]
                                         : rng_f32(key, word + draws);
            draws++;
            const float ratio = p / q;
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
        if (!a.greedy && rej < 0 && a.bonus) {
            const uint32_t* wt = rs0 + np * ACC_RS_WORDS;
            flags |= rs_get(wt, RS_FLAGS);
            if (rs_get(wt, RS_STATUS)) status = 1;
        }
        sh.ib[0] = acc;
        sh.ib[1] = rej;
        sh.ib[2] = draws;
        sh.ib[3] = (int)flags;
        sh.ib[4] = status;
    }
    __syncthreads();
    const int acc = sh.ib[0], rej = sh.ib[1];
    int draws = sh.ib[2];
    uint32_t flags = (uint32_t)sh.ib[3];
    int status = sh.ib[4];
    int token = -1;
    __syncthreads();

    if (a.greedy) {
        if (rej >= 0) token = (int)rs_get(rs0 + rej * ACC_RS_WORDS, RS_ARGMAX);
        else if (a.bonus) token = (int)rs_get(rs0 + np * ACC_RS_WORDS, RS_ARGMAX);
    } else if (status == 0 && (rej >= 0 || a.bonus)) {
        float u;
        if (par_u) {
            u = u_s[draws];
        } else {
            uint32_t key[8];
            if (a.uniforms) {
                u = a.uniforms[(size_t)b * (a.K + 1) + draws];
            } else {
                rng_key_from_seed(a.seeds ? a.seeds[b] : 0ull, key);
                u = rng_f32(key, (a.word_offsets ? a.word_offsets[b] : 0ull) + draws);
            }
        }
        SeqScan cdf = seq_scan_init();
        if (topk_compact(a.top_k, V)) {
            const int row = rej >= 0 ? rej : np;
            // a one-row launch (a proposal draw) filtered that row in this workgroup
            const int have = (rows_per_seq == 1 && rej < 0 && needed) ? sh.ib[6] : -1;
            resolve_compact(rs0 + row * ACC_RS_WORDS, rej >= 0 ? rsd0 + rej * ACC_RS_WORDS : nullptr,
                            trow0 + (size_t)row * V, rej >= 0 ? drow0 + (size_t)rej * V : nullptr, V, T, u, lds, &sh,
                            &cdf, &status, have);
        } else if (rej >= 0) {
            // residual max(0, p - q): exact mass, then the exact CDF of r / mass
            const RowFilt ft = rs_load(rs0 + rej * ACC_RS_WORDS, T);
            const RowFilt fd = rs_load(rsd0 + rej * ACC_RS_WORDS, T);
            const float* tl = trow0 + (size_t)rej * V;
            const float* dl = drow0 + (size_t)rej * V;
            auto resid = [&](float lt, float ld, int j) {
                const float d = filt_prob(ft, lt, j) - filt_prob(fd, ld, j);
                return d > 0.0f ? d : 0.0f;
            };
            const SeqScan m = block_seq_scan<2>(tl, dl, V, -1.0f, resid, lds, chunk, &sh);
            const float R = m.s;
            if (!isfinite(R) || R <= FLT_EPSILON) {
                status = 1;
            } else {
                cdf = block_seq_scan<2>(
                    tl, dl, V, u, [&](float lt, float ld, int j) { return resid(lt, ld, j) / R; }, lds, chunk, &sh);
            }
        } else {
            const RowFilt ft = rs_load(rs0 + np * ACC_RS_WORDS, T);
            cdf = block_seq_scan<1>(
                trow0 + (size_t)np * V, nullptr, V, u, [&](float lt, float, int j) { return filt_prob(ft, lt, j); },
                lds, chunk, &sh);
        }
        if (status == 0) {
            if (cdf.cross < 0) {  // no partial sum reaches the draw: the last index (sampler.rs:346)
                cdf.cross = V - 1;
                cdf.s_at = cdf.s;
                cdf.s_before = cdf.s;
            }
            token = cdf.cross;
            // validate_probabilities (sampler.rs:314-335): the sampled distribution sums to 1
            if (!isfinite(cdf.s) || fabsf(cdf.s - 1.0f) > 1e-4f) status = 1;
            if (fminf(fabsf(cdf.s_at - u), fabsf(u - cdf.s_before)) < 1e-6f) flags |= ACCEPT_FLAG_CDF_NEAR;
            draws++;
        }
    }
    (void)lane;
    (void)wid;
    if (tid == 0) {
        a.out_accept_len[b] = acc;
        a.out_token[b] = status ? -1 : token;
        a.out_flags[b] = flags;
        a.out_draws[b] = draws;
        a.out_status[b] = status;
    }
}

static size_t accept_lds_bytes(int V, int greedy, int top_p_active, int top_k) {
    if (greedy) return 0;
    size_t f = 2 * (size_t)(V < ACC_CHUNK ? V : ACC_CHUNK);
    if (top_p_active && f < (size_t)TOPP_LDS_FLOATS) f = TOPP_LDS_FLOATS;
    if (topk_compact(top_k, V) && f < (size_t)TOPK_LDS_FLOATS) f = TOPK_LDS_FLOATS;
    return f * sizeof(float);
}

int launch_accept(const AcceptArgs& a_in, hipStream_t stream) {
    AcceptArgs a = a_in;
    const int rows = a.target_rows + a.K;
    const bool topp = a.top_p > 0.0f && a.top_p < 1.0f;
    const size_t lds = accept_lds_bytes(a.V, a.greedy, topp, a.top_k);
    if (lds > MAX_DYN_LDS) return 3;
    a.chunk = a.V < ACC_CHUNK ? a.V : ACC_CHUNK;
    if (a.chunk < 1) a.chunk = 1;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)accept_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)MAX_DYN_LDS);
    });
    if (note_error(attr)) return 4;
    (void)hipGetLastError();
    launch_timed(accept_kernel, dim3(a.B * rows), dim3(ACC_THREADS), (uint32_t)lds, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

// ---------------------------------------------------------------------------
// Statically allocated scratch for aarh_accept_sample_static: the row statistics
// and arrival counters of one call, in device memory owned by the library from
// load to process exit (one copy per GPU).  Host code never uses the symbol's
// name as an address; accept_static_scratch() returns the device address that
// hipGetSymbolAddress reported for the current device at set-up.
// ---------------------------------------------------------------------------
static constexpr size_t ACC_STATIC_WORDS = (size_t)ACC_STATIC_ROWS * ACC_RS_WORDS + ACC_STATIC_SEQS;
static __device__ __align__(256) uint32_t scratch[ACC_STATIC_WORDS];

static constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static uint32_t* g_scratch_ptr[MAX_DEVICES];

__global__ void zero_u32_kernel(uint32_t* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

int accept_static_init(int device, hipStream_t stream) {
    if (device < 0 || device >= MAX_DEVICES) return 3;
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (g_scratch_ptr[device]) return 0;
    void* p = nullptr;
    if (note_error(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)))) return 4;
    if (!p) return 4;
    // counters start at zero (the kernel re-arms them after every call)
    uint32_t* cnt = (uint32_t*)p + (size_t)ACC_STATIC_ROWS * ACC_RS_WORDS;
    (void)hipGetLastError();
    hipLaunchKernelGGL(zero_u32_kernel, dim3((ACC_STATIC_SEQS + 255) / 256), dim3(256), 0, stream, cnt,
                       ACC_STATIC_SEQS);
    if (note_error(hipGetLastError())) return 4;
    if (note_error(hipStreamSynchronize(stream))) return 4;
    g_scratch_ptr[device] = (uint32_t*)p;
    return 0;
}

int accept_static_scratch(int device, uint32_t** rstat, unsigned** counters) {
    if (device < 0 || device >= MAX_DEVICES) return 3;
    std::lock_guard<std::mutex> g(g_scratch_mu);
    uint32_t* p = g_scratch_ptr[device];
    if (!p) return 4;
    *rstat = p;
    *counters = p + (size_t)ACC_STATIC_ROWS * ACC_RS_WORDS;
    return 0;
}

int launch_zero_u32(uint32_t* p, int n, hipStream_t stream) {
    if (n <= 0) return 0;
    (void)hipGetLastError();
    hipLaunchKernelGGL(zero_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, p, n);
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
    __shared__ AccShared sh;
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int V = a.V, n = a.n;
    const float* row = a.logits + (size_t)blockIdx.x * a.ld;
    int am = -1;
    RowFilt f{};
    int status = 0;
    if (a.greedy) {
        am = block_argmax(row, V, &sh);  // one-hot at the argmax (sampler.rs:211-215)
        // The stable descending order of a one-hot vector is the argmax (1.0), then the
        // zeros in ascending index order: the n - 1 smallest indices other than am.
        if (tid < n) {
            const int id = tid == 0 ? am : (tid - 1 < am ? tid - 1 : tid);
            a.ids[(size_t)blockIdx.x * n + tid] = id < V ? (uint32_t)id : 0xFFFFFFFFu;
            a.probs[(size_t)blockIdx.x * n + tid] = tid == 0 ? 1.0f : 0.0f;
        }
        return;
    } else {
        uint32_t fl;
        row_filter(row, V, a.temperature, a.top_k, a.top_p, lds, a.chunk, &sh, f, fl, status);
    }
    // ---- this thread's n best keys, descending ----
    unsigned long long best[CAND_MAX];
#pragma unroll
    for (int i = 0; i < CAND_MAX; i++) best[i] = 0ull;
    auto offer = [&](int j, float p) {
        unsigned long long k = prob_key(p, j);
#pragma unroll
        for (int i = 0; i < CAND_MAX; i++) {
            if (i < n && k > best[i]) {
                const unsigned long long t = best[i];
                best[i] = k;
                k = t;
            }
        }
    };
    if (status == 0 && a.greedy) {
        for (int j = tid; j < V; j += ACC_THREADS) offer(j, j == am ? 1.0f : 0.0f);
    } else if (status == 0) {
        rows_foreach<1>(row, nullptr, V, [&](int j, float l, float, bool valid) {
            if (valid) offer(j, filt_prob(f, l, j));
        });
    }
#pragma unroll
    for (int i = 0; i < CAND_MAX; i++) keys[tid][i] = best[i];
    __syncthreads();
    if (wid != 0) return;
    if (status != 0) {
        // the distribution is invalid (the reference returns Err): no candidates
        if (lane < n) {
            a.ids[(size_t)blockIdx.x * n + lane] = 0xFFFFFFFFu;
            a.probs[(size_t)blockIdx.x * n + lane] = __uint_as_float(0x7FC00000u);
        }
        return;
    }
    // ---- wave 0: lane l owns lists l + 64 q; n rounds of a wave-wide max over list heads ----
    int head[ACC_WAVES];
#pragma unroll
    for (int q = 0; q < ACC_WAVES; q++) head[q] = 0;
    for (int r = 0; r < n; r++) {
        unsigned long long mk = 0ull;
        int mq = -1;
#pragma unroll
        for (int q = 0; q < ACC_WAVES; q++) {
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
            for (int q = 0; q < ACC_WAVES; q++)
                if (q == mq) head[q]++;
        }
        if (lane == 0) {
            a.ids[(size_t)blockIdx.x * n + r] = wk ? ~(unsigned)(wk & 0xFFFFFFFFull) : 0xFFFFFFFFu;
            a.probs[(size_t)blockIdx.x * n + r] = __uint_as_float((unsigned)(wk >> 32));
        }
    }
}

int launch_candidates(const CandArgs& a_in, hipStream_t stream) {
    CandArgs a = a_in;
    if (a.n < 1 || a.n > CAND_MAX || a.rows <= 0 || a.V <= 0) return 2;
    const bool topp = a.top_p > 0.0f && a.top_p < 1.0f;
    size_t fl = a.greedy ? 0 : 2 * (size_t)(a.V < CAND_CHUNK ? a.V : CAND_CHUNK);
    if (!a.greedy && topp && fl < (size_t)TOPP_LDS_FLOATS) fl = TOPP_LDS_FLOATS;
    if (!a.greedy && topk_compact(a.top_k, a.V) && fl < (size_t)TOPK_LDS_FLOATS) fl = TOPK_LDS_FLOATS;
    const size_t lds = fl * sizeof(float);
    const size_t cap = MAX_DYN_LDS - sizeof(unsigned long long) * ACC_THREADS * CAND_MAX;
    if (lds > cap) return 3;
    a.chunk = a.V < CAND_CHUNK ? a.V : CAND_CHUNK;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [cap] {
        attr = hipFuncSetAttribute((const void*)candidates_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)cap);
    });
    if (note_error(attr)) return 4;
    (void)hipGetLastError();
    launch_timed(candidates_kernel, dim3(a.rows), dim3(ACC_THREADS), (uint32_t)lds, stream, a);
    return note_error(hipGetLastError()) ? 4 : 0;
}

}  // namespace aarh
