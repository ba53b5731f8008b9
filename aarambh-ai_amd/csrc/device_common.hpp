// Device-side helpers shared by the gfx950 kernels of libaarambh_hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));

#define WAVE 64

// Build-defined synthetic generator (same formula as the test oracle):
// splitmix64 counter hash -> Box-Muller in f64.
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__device__ __forceinline__ float synth_normal(uint64_t seed, uint32_t stream, uint64_t index) {
    uint64_t base = splitmix64(seed ^ ((uint64_t)stream * 0xD1B54A32D192ED03ull));
    uint64_t h = splitmix64(base + index);
    double u1 = ((double)(h >> 40) + 1.0) * (1.0 / 16777216.0);
    double u2 = (double)((h >> 16) & 0xFFFFFFull) * (1.0 / 16777216.0);
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

// f32::total_cmp ordering key: larger key == larger value, NaN above +inf.
__device__ __forceinline__ int32_t total_key(float f) {
    int32_t i = __float_as_int(f);
    return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

// exp rounded to nearest f32: evaluate in f64 and round once.  This matches a
// correctly rounded libm expf except in the rare cases where the host libm
// itself misrounds; those show up as flagged near-ties, never silently.
__device__ __forceinline__ float expf_rn(float x) { return (float)exp((double)x); }

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

// ---------------------------------------------------------------------------
// rand 0.8 StdRng (ChaCha12, rand_chacha 0.3.1) seeded by seed_from_u64
// (rand_core 0.6.4): keystream word n of sequence seed, evaluated on device.
// ---------------------------------------------------------------------------
// Byte offset, inside one 16-row x 128-column weight tile, of byte b of lane l's
// share (TILE_BYTES / 64 bytes: row l % 16, columns 32 * (l / 16) .. +32 of the
// group).  The share is cut into 16-byte chunks and chunk q of every lane sits in
// the q-th KiB of the tile, lanes in order: a 16-byte load per lane reads one
// contiguous KiB.  INT4 shares are a single chunk.
__host__ __device__ __forceinline__ int tile_byte(int lane, int b) { return ((b >> 4) << 10) + lane * 16 + (b & 15); }

__device__ __forceinline__ uint32_t rotl32(uint32_t v, int n) { return (v << n) | (v >> (32 - n)); }

__device__ inline void rng_key_from_seed(uint64_t state, uint32_t key[8]) {
    const uint64_t mul = 6364136223846793005ull, inc = 11634580027462260723ull;
    for (int i = 0; i < 8; i++) {
        state = state * mul + inc;
        uint32_t xs = (uint32_t)(((state >> 18) ^ state) >> 27);
        uint32_t rot = (uint32_t)(state >> 59);
        key[i] = (xs >> rot) | (xs << ((32 - rot) & 31));
    }
}

#define CHACHA_QR(a, b, c, d)                                                                      \
    a += b; d ^= a; d = rotl32(d, 16);                                                             \
    c += d; b ^= c; b = rotl32(b, 12);                                                             \
    a += b; d ^= a; d = rotl32(d, 8);                                                              \
    c += d; b ^= c; b = rotl32(b, 7);

__device__ inline uint32_t rng_word(const uint32_t key[8], uint64_t word) {
    uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                       key[0], key[1], key[2], key[3], key[4], key[5], key[6], key[7],
                       (uint32_t)(word >> 4), (uint32_t)(word >> 36), 0u, 0u};
    uint32_t x[16];
#pragma unroll
    for (int i = 0; i < 16; i++) x[i] = in[i];
    for (int r = 0; r < 12; r += 2) {
        CHACHA_QR(x[0], x[4], x[8], x[12]);
        CHACHA_QR(x[1], x[5], x[9], x[13]);
        CHACHA_QR(x[2], x[6], x[10], x[14]);
        CHACHA_QR(x[3], x[7], x[11], x[15]);
        CHACHA_QR(x[0], x[5], x[10], x[15]);
        CHACHA_QR(x[1], x[6], x[11], x[12]);
        CHACHA_QR(x[2], x[7], x[8], x[13]);
        CHACHA_QR(x[3], x[4], x[9], x[14]);
    }
    uint32_t idx = (uint32_t)(word & 15);
    uint32_t out = 0;
#pragma unroll
    for (int i = 0; i < 16; i++)
        if ((uint32_t)i == idx) out = x[i] + in[i];
    return out;
}

// rand 0.8 Standard f32: (next_u32 >> 8) * 2^-24.
__device__ inline float rng_f32(const uint32_t key[8], uint64_t word) {
    return (float)(rng_word(key, word) >> 8) * (1.0f / 16777216.0f);
}

// ---------------------------------------------------------------------------
// Cross-workgroup hand-off without L2 flushes.
//
// A device-scope fence on gfx950 writes back the whole XCD L2 (buffer_wbl2),
// which costs microseconds per workgroup.  Data that one workgroup hands to
// another inside a kernel (split-K partials, row statistics) is instead written
// and read with agent-scope relaxed atomics, which compile to sc1 (coherent,
// L2-bypassing) stores/loads; the writer waits for its stores to complete
// (s_waitcnt vmcnt(0)) before it signals arrival on the counter.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void st_coh(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh_i32(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_coh_i32(const int32_t* p) {
    return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// All of this thread's memory operations have completed.
// 16-byte agent-coherent global access through a raw buffer resource (cache policy
// sc1: the access is performed at device scope, past the per-XCD L2 state), for
// partial results handed between workgroups of one launch.  Offsets in bytes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coh_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ float4_t ld4_coh(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
    return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 16));
}
__device__ __forceinline__ float2_t ld2_coh(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
    return __builtin_bit_cast(float2_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)byte_off, 0, 16));
}
__device__ __forceinline__ void st4_coh(__amdgpu_buffer_rsrc_t r, unsigned byte_off, float4_t v) {
    typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, (int)byte_off, 0, 16);
}
__device__ __forceinline__ void wait_mem() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Called by every thread of the workgroup after its coherent stores; returns
// true in the workgroup that arrives last (which also re-arms the counter).
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned expected, unsigned* s_flag) {
    wait_mem();
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool last = prev == expected - 1u;
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = last ? 1u : 0u;
    }
    __syncthreads();
    bool last = *s_flag != 0u;
    wait_mem();
    return last;
}

// ---------------------------------------------------------------------------
// Wave-level primitives
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wave_excl_scan_i32(int v) {
    const int lane = threadIdx.x & 63;
    int incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        int t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
    }
    return incl - v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

// ---------------------------------------------------------------------------
// Exact sequential f32 summation on one wave.
//
// Continues s_k = fl(s_{k-1} + v[k]) over v[0..n) for v[k] >= 0 from the running
// sum st.s, bit-identical to a scalar left-to-right f32 loop (the reference's
// iter().sum::<f32>() and the running cumulative of sample_from_probs), so a long
// vector can be summed in pieces.  With u >= 0 it also records the first k with
// u <= s_k (inverse CDF, `draw <= cumulative`), as gbase + k.
//
// Method: while s stays inside one binade [2^e, 2^(e+1)), every partial sum
// is an integer multiple of ulp(s), and fl(s + x) = s + ulp * RNE(x / ulp)
// unless x / ulp has fraction exactly 1/2 (a tie, decided by parity).  So the
// wave turns 512 elements at a time into integer increments, scans them, and
// stops at the first element that leaves the binade or ties; that element is
// added with a real f32 add and the scan restarts after it.
// ---------------------------------------------------------------------------
struct SeqScan {
    float s;         // running sum
    int cross;       // first global index k with u <= s_k; -1 while none
    float s_at;      // s_cross
    float s_before;  // s_{cross-1} (0 before the first element)
};

__device__ __forceinline__ SeqScan seq_scan_init() {
    SeqScan st;
    st.s = 0.0f;
    st.cross = -1;
    st.s_at = 0.0f;
    st.s_before = 0.0f;
    return st;
}

// Inclusive prefix sum over the 64 lanes with DPP row shifts and row broadcasts
// (register-to-register, no LDS round trip per step).
__device__ __forceinline__ int wave_incl_scan_dpp(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
    return v;
}
__device__ __forceinline__ float readlane_f32(float x, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

// Elements added one at a time after the sum first becomes non-zero (see below).
constexpr int SCAN_SCALAR = 64;
__device__ __forceinline__ void seq_scan_wave(const float* v, int n, float u, int gbase, SeqScan& st) {
    constexpr int E = 8;  // consecutive elements per lane in the binade fast path (512 per step)
    const int lane = threadIdx.x & 63;
    float s = st.s;
    int pos = 0;
    int cross = st.cross;
    float s_at = st.s_at, s_before = st.s_before;
    const bool want = u >= 0.0f;
    int scal = 0;  // elements still to add one at a time
    while (pos < n) {
        if (scal > 0) {
            // Plain f32 adds in element order (64 loaded per round trip, four added per
            // crossing check).  Used for the first SCAN_SCALAR elements after the sum
            // becomes non-zero, where the sum still doubles every few elements and the
            // binade windows would restart at almost every element.
            const int cnt = min(64, min(scal, n - pos));
            const float xv = lane < cnt ? v[pos + lane] : 0.0f;  // lanes past cnt add 0: no change
            for (int i = 0; i < cnt; i += 4) {
                const float x0 = readlane_f32(xv, i), x1 = readlane_f32(xv, i + 1);
                const float x2 = readlane_f32(xv, i + 2), x3 = readlane_f32(xv, i + 3);
                const float s0 = s + x0, s1 = s0 + x1, s2 = s1 + x2, s3 = s2 + x3;
                if (want && cross < 0 && (u <= s0 || u <= s1 || u <= s2 || u <= s3)) {
                    // the first of the four partial sums to reach u (a padding lane repeats
                    // the last real sum, so the first one found is a real element)
                    const int k = u <= s0 ? 0 : u <= s1 ? 1 : u <= s2 ? 2 : 3;
                    cross = gbase + pos + i + k;
                    s_at = k == 0 ? s0 : k == 1 ? s1 : k == 2 ? s2 : s3;
                    s_before = k == 0 ? s : k == 1 ? s0 : k == 2 ? s1 : s2;
                }
                s = s3;
            }
            pos += cnt;
            scal -= cnt;
            continue;
        }
        if (s == 0.0f) {
            // Zeros keep s at 0 (0 + 0 = 0); the first non-zero element x gives s = x.
            const int base = pos + 4 * lane;
            float x[4];
#pragma unroll
            for (int k = 0; k < 4; k++) x[k] = (base + k < n) ? v[base + k] : 0.0f;
            int fnz = 4;
#pragma unroll
            for (int k = 3; k >= 0; k--)
                if (base + k < n && x[k] != 0.0f) fnz = k;
            unsigned long long m = __ballot(fnz < 4);
            if (want && cross < 0 && u <= 0.0f) {
                cross = gbase + pos;
                s_at = 0.0f;
                s_before = 0.0f;
            }
            if (m == 0ull) {
                pos += 256;
                continue;
            }
            const int bl = __ffsll((long long)m) - 1;
            const int t = pos + 4 * bl + __builtin_amdgcn_readlane(fnz, bl);
            s = v[t];
            if (want && cross < 0 && u <= s) {
                cross = gbase + t;
                s_at = s;
                s_before = 0.0f;
            }
            pos = t + 1;
            scal = SCAN_SCALAR;
            continue;
        }
        const uint32_t bits = __float_as_uint(s);
        const int eb = (int)((bits >> 23) & 0xFF);
        if (eb == 0) {
            // subnormal running sum: one scalar step
            const float xt = v[pos];
            const float sp = s;
            s = s + xt;
            if (want && cross < 0 && u <= s) {
                cross = gbase + pos;
                s_at = s;
                s_before = sp;
            }
            pos++;
            continue;
        }
        const int sh = 150 - eb;                               // x / ulp(s) == ldexp(x, sh)
        const int ns = (int)((bits & 0x7FFFFFu) | 0x800000u);  // s / ulp(s)
        // window [w0, w0 + 64 E) aligned to 4 elements; elements below pos count as 0
        const int w0 = pos & ~3;
        const int base = w0 + E * lane;
        float x[E];
        if (base + E <= n && base >= pos) {
#pragma unroll
            for (int c = 0; c < E / 4; c++) {
                const float4_t q = *(const float4_t*)(v + base + 4 * c);
                x[4 * c] = q[0];
                x[4 * c + 1] = q[1];
                x[4 * c + 2] = q[2];
                x[4 * c + 3] = q[3];
            }
        } else {
#pragma unroll
            for (int k = 0; k < E; k++) {
                const int i = base + k;
                x[k] = (i >= pos && i < n) ? v[i] : 0.0f;
            }
        }
        // r = RNE(c) for c = x / ulp.  An element is special when c is not a finite value
        // in [0, 2^24) (its bit pattern, read as unsigned, is at or above that of 2^24:
        // also negative values and NaN) or is a tie (|c - RNE(c)| == 1/2).  The lane
        // tests both once over its E elements with vector max operations, and only a
        // flagged lane marks its elements one by one (special elements become 2^24).
        int r[E];
        bool special = false;
        int lsum = 0;
        float dmax = 0.0f;
        uint32_t bmax = 0u;
#pragma unroll
        for (int k = 0; k < E; k++) {
            const float c = ldexpf(x[k], sh);
            const float rr = __builtin_rintf(c);
            dmax = fmaxf(dmax, fabsf(c - rr));
            bmax = max(bmax, __float_as_uint(c));
            r[k] = (int)rr;
            lsum += r[k];
        }
        if (bmax >= 0x4B800000u || dmax == 0.5f) {
            special = true;
            lsum = 0;
#pragma unroll
            for (int k = 0; k < E; k++) {
                const float c = ldexpf(x[k], sh);
                const float rr = __builtin_rintf(c);
                const bool sp = !(__float_as_uint(c) < 0x4B800000u) || (fabsf(c - rr) == 0.5f);
                r[k] = sp ? 16777216 : (int)rr;
                lsum += r[k];
            }
        }
        if (special || lsum > 16777217) lsum = 16777217;  // past the binade anyway; keeps the scan in range
        const int incl = wave_incl_scan_dpp(lsum);
        // Fast path: no element is special and the window ends inside the binade, and no
        // partial sum of the window reaches u (sums only grow, so each lane's end value
        // decides): the window advances without walking its elements.
        {
            const int lane_end = ns + incl;
            const bool lane_bad = special || lane_end >= 16777216;
            const bool lane_cross = want && cross < 0 && u <= ldexpf((float)lane_end, -sh);
            if (__ballot(lane_bad || lane_cross) == 0ull) {
                s = ldexpf((float)(ns + __builtin_amdgcn_readlane(incl, 63)), -sh);
                pos = w0 + 64 * E;
                continue;
            }
        }
        int run = ns + incl - lsum;
        int first_bad = E, first_cross = E, run_bad = 0;
        float cs_at = 0.0f, cs_before = 0.0f;
        // walk the lane's elements with predication only (no early exit), so the loop
        // unrolls and r[] stays in registers
#pragma unroll
        for (int k = 0; k < E; k++) {
            const int rk = run + r[k];
            const bool live = first_bad == E;
            if (live && (r[k] >= 16777216 || rk >= 16777216)) {
                first_bad = k;
                run_bad = run;
            }
            if (want && first_bad == E && first_cross == E && r[k] > 0) {
                const float sk = ldexpf((float)rk, -sh);
                if (u <= sk) {
                    first_cross = k;
                    cs_at = sk;
                    cs_before = ldexpf((float)run, -sh);
                }
            }
            if (first_bad == E) run = rk;
        }
        const unsigned long long badm = __ballot(first_bad < E);
        const int bad_lane = badm ? (__ffsll((long long)badm) - 1) : 64;
        const unsigned long long lanes_ok = bad_lane >= 64 ? ~0ull : ((1ull << bad_lane) | ((1ull << bad_lane) - 1ull));
        const unsigned long long cm = __ballot(first_cross < E) & lanes_ok;
        if (want && cross < 0 && cm) {
            const int cl = __ffsll((long long)cm) - 1;
            cross = gbase + w0 + E * cl + __builtin_amdgcn_readlane(first_cross, cl);
            s_at = readlane_f32(cs_at, cl);
            s_before = readlane_f32(cs_before, cl);
        }
        if (bad_lane == 64) {
            s = ldexpf((float)(ns + __builtin_amdgcn_readlane(incl, 63)), -sh);
            pos = w0 + 64 * E;
        } else {
            const int t = w0 + E * bad_lane + __builtin_amdgcn_readlane(first_bad, bad_lane);
            const float sp = ldexpf((float)__builtin_amdgcn_readlane(run_bad, bad_lane), -sh);
            const float xt = v[t];
            s = sp + xt;
            if (want && cross < 0 && u <= s) {
                cross = gbase + t;
                s_at = s;
                s_before = sp;
            }
            pos = t + 1;
        }
    }
    st.s = s;
    st.cross = cross;
    st.s_at = s_at;
    st.s_before = s_before;
}

// One-shot form over v[0..n): total, and the crossing (n - 1 with s_at = total when
// no partial sum reaches u, as sample_from_probs falls back to the last index).
struct SeqSum {
    float total;
    int cross;      // first k with u <= s_k (n-1 if none); -1 when u < 0
    float s_at;     // s_cross
    float s_before; // s_{cross-1} (0 for cross == 0)
};

__device__ inline SeqSum seq_sum_wave(const float* v, int n, float u) {
    SeqScan st = seq_scan_init();
    seq_scan_wave(v, n, u, 0, st);
    SeqSum res;
    res.total = st.s;
    res.cross = st.cross;
    res.s_at = st.s_at;
    res.s_before = st.s_before;
    if (u >= 0.0f && st.cross < 0) {
        res.cross = n - 1;
        res.s_at = st.s;
        res.s_before = st.s;
    }
    return res;
}

// One 1 KiB wave load straight into LDS: lane l's 16 bytes at rsrc + voff +
// soff land at LDS address lds_base + 16 l (buffer_load_dwordx4 ... lds, base in
// M0).  Written as inline asm so the compiler does not see an LDS write it would
// guard with a conservative vmcnt(0) before every LDS read: the kernel counts
// these loads itself.  M0 is restored before the statement ends.  NT marks the load
// non-temporal (data read once: a stream of weights or cache blocks).
template <bool NT = false>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, const void* lds_dst, int voff, int soff) {
    const unsigned base = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_dst);
    int saved;
    if constexpr (NT)
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "buffer_load_dwordx4 %2, %3, %4 offen nt lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(base), "v"(voff), "s"(r), "s"(soff)
            : "memory");
    else
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(base), "v"(voff), "s"(r), "s"(soff)
            : "memory");
}

// One 256-byte wave load into LDS: lane l's 4 bytes land at lds_dst + 4 l.
template <bool NT = false>
__device__ __forceinline__ void lds_dma4(__amdgpu_buffer_rsrc_t r, const void* lds_dst, int voff, int soff) {
    const unsigned base = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_dst);
    int saved;
    if constexpr (NT)
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "buffer_load_dword %2, %3, %4 offen nt lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(base), "v"(voff), "s"(r), "s"(soff)
            : "memory");
    else
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "buffer_load_dword %2, %3, %4 offen lds\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(base), "v"(voff), "s"(r), "s"(soff)
            : "memory");
}

// s_waitcnt vmcnt(n) (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14), other counters unconstrained.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
