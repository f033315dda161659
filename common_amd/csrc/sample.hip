// Token sampling on the device: temperature softmax, nucleus (top-p) filtering and the
// categorical draw of AutoregressiveModel.sampleToken (engine/ml/.../AutoregressiveModel.java:323-386),
// and the sample function AutoregressiveModel.of installs (:413-425: logits / temperature, the
// DistributionFeatures.softmax of compute/stats/.../DistributionFeatures.java:129-141, then
// sampleToken(probabilities, V, 1.0, 1.0, random)), with java.util.Random's generator
// (48-bit LCG, nextDouble = ((next(26) << 27) + next(27)) * 2^-53) kept per sequence on the device.
//
// Everything after the fp32 logits is double, the reference's precision.  A row of V values is cut
// into kBlocks chunks; each pass is one grid of (kBlocks, rows) 1024-thread blocks whose per-block
// maxima / sums go to the workspace and are combined by the next kernel in a fixed order (a
// wavefront butterfly over the 64 chunk values), so every result is deterministic.
//
// Nucleus filtering does not sort.  The reference keeps the shortest prefix of the probabilities
// sorted in descending order (ties in index order: Arrays.sort is stable) whose running sum
// reaches top_p.  With p* the smallest kept value, that is every value > p* plus the first c
// (by index) of the values == p*; p* is the largest key t with sum(p >= t) >= top_p.  It is found
// by a radix descent over the 64-bit patterns of the probabilities (non-negative doubles order as
// their bit patterns): 8 passes of 8-bit digits.  Each pass is one kernel: every chunk builds its
// histogram of (count, sum) in LDS and adds it into the row's histogram with device-scope integer
// atomics; the last chunk to finish (an arrival counter) picks the digit and clears the row's
// histogram and counter for the next pass.  Bucket sums are 2^-60 fixed point in u64, so the
// atomics are exact and associative (the result does not depend on arrival order); the kept set
// agrees with the reference's sequential double sums except when top_p lies within ~1e-13 of a
// partial sum.
//
// The draw mirrors the reference's loop `cumulative += probs[i]; if (r < cumulative) return i`:
// chunk masses locate the chunk whose interval holds r, then per-thread sums of contiguous index
// ranges and a walk of the crossing thread's elements locate the index.  Partial sums group
// differently from the reference's single running sum (rounding ~1e-16), so a draw within that
// distance of a boundary may pick the neighbour.
#include "ar_hip_internal.h"

namespace {

constexpr int kBlocks = 64;   // chunks per row (one wavefront of partials)
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr double kFix = 1152921504606846976.0;     // 2^60
constexpr double kEps64 = 2.220446049250313e-16;   // FP64 machine epsilon (Precision.java:110-121)

struct Ws {
    double* buf;                // [rows][V] exp values
    double* pmax;               // [rows][kBlocks]
    double* psum;
    double* pemax;
    double* psum2;
    double* pmass;
    unsigned* hcnt;             // [rows][kBlocks][256] per-chunk counts of the last pass
    unsigned* gcnt;             // [rows][256] row histogram of the current pass (zero between passes)
    unsigned long long* gsum;   // [rows][256]
    unsigned* arrived;          // [rows] chunks done with the current pass (zero between passes)
    unsigned long long* sel;    // [rows][8]: prefix, above, done, take
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// The zero-initialised part (gcnt, gsum, arrived) comes first so that it can be cleared once.
Ws carve(void* base, int rows, int V, size_t* total, size_t* zero_bytes) {
    Ws w{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const uintptr_t p = reinterpret_cast<uintptr_t>(base) + off;
        off += align256(bytes);
        return reinterpret_cast<void*>(p);
    };
    w.gcnt = (unsigned*)take((size_t)rows * 256 * 4);
    w.gsum = (unsigned long long*)take((size_t)rows * 256 * 8);
    w.arrived = (unsigned*)take((size_t)rows * 4);
    if (zero_bytes) *zero_bytes = off;
    w.buf = (double*)take((size_t)rows * V * 8);
    w.pmax = (double*)take((size_t)rows * kBlocks * 8);
    w.psum = (double*)take((size_t)rows * kBlocks * 8);
    w.pemax = (double*)take((size_t)rows * kBlocks * 8);
    w.psum2 = (double*)take((size_t)rows * kBlocks * 8);
    w.pmass = (double*)take((size_t)rows * kBlocks * 8);
    w.hcnt = (unsigned*)take((size_t)rows * kBlocks * 256 * 4);
    w.sel = (unsigned long long*)take((size_t)rows * 8 * 8);
    if (total) *total = off;
    return w;
}

struct Args {
    const float* logits;
    int ls, V, mode;
    double T;
    bool topp;
    Ws w;
    unsigned long long* rng;
    const int* state;
    unsigned long long* keys;
    int keys_stride;
    int* out;
};

__device__ inline double wave_max_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ inline double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
// inclusive prefix over the lanes of a wavefront (Hillis-Steele; a fixed order of additions)
template <typename T>
__device__ inline T wave_incl_scan(T v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
    }
    return v;
}
// block reductions: butterfly per wavefront, then the wavefront values in order
__device__ inline double block_max_d(double v, double* red) {
    v = wave_max_d(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = red[0];
    for (int w = 1; w < kWaves; w++) r = fmax(r, red[w]);
    __syncthreads();
    return r;
}
__device__ inline double block_sum_d(double v, double* red) {
    v = wave_sum_d(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = red[0];
    for (int w = 1; w < kWaves; w++) r += red[w];
    __syncthreads();
    return r;
}
// inclusive prefix over the block's threads in thread order (wavefront scans + the wavefront
// totals in order)
template <typename T>
__device__ inline T block_incl_scan(T v, T* red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    v = wave_incl_scan(v);
    if (lane == 63) red[w] = v;
    __syncthreads();
    T base = 0;
    for (int k = 0; k < w; k++) base += red[k];
    __syncthreads();
    return base + v;
}
// combine one row's 64 chunk partials (every thread gets the value; same order in every block)
__device__ inline double row_max(const double* p) { return wave_max_d(p[threadIdx.x & 63]); }
__device__ inline double row_sum(const double* p) { return wave_sum_d(p[threadIdx.x & 63]); }

__device__ inline void chunk_of(int V, int blk, int* c0, int* c1) {
    const int per = (V + kBlocks - 1) / kBlocks;
    *c0 = min(V, blk * per);
    *c1 = min(V, *c0 + per);
}

__device__ inline double scaled(const Args& a, int b, int i) { return (double)a.logits[(size_t)b * a.ls + i] / a.T; }

// 1. maximum of logits / temperature per chunk
__global__ __launch_bounds__(kThreads) void smp_max_kernel(Args a) {
    __shared__ double red[kWaves];
    const int blk = blockIdx.x, b = blockIdx.y;
    int c0, c1;
    chunk_of(a.V, blk, &c0, &c1);
    double m = -INFINITY;
    for (int i = c0 + threadIdx.x; i < c1; i += kThreads) m = fmax(m, scaled(a, b, i));
    m = block_max_d(m, red);
    if (threadIdx.x == 0) a.w.pmax[b * kBlocks + blk] = m;
}

// 2. exponentials: sampleToken's exp(x - max), or the softmax-ignoring-zero of the model's sample
//    function (a value equal to 0 stays 0; the maximum itself gets exp(epsilon))
__global__ __launch_bounds__(kThreads) void smp_exp_kernel(Args a) {
    __shared__ double red[kWaves];
    const int blk = blockIdx.x, b = blockIdx.y;
    int c0, c1;
    chunk_of(a.V, blk, &c0, &c1);
    const double M = row_max(a.w.pmax + b * kBlocks);
    double s = 0.0, emax = 0.0;
    double* buf = a.w.buf + (size_t)b * a.V;
    for (int i = c0 + threadIdx.x; i < c1; i += kThreads) {
        const double y = scaled(a, b, i);
        double e;
        if (a.mode == AR_SAMPLE_TOKEN) {
            e = exp(y - M);
        } else {
            const double d = (y == 0.0) ? 0.0 : ((y == M) ? kEps64 : y - M);
            e = (d == 0.0) ? 0.0 : exp(d);
        }
        buf[i] = e;
        s += e;
        emax = fmax(emax, e);
    }
    s = block_sum_d(s, red);
    emax = block_max_d(emax, red);
    if (threadIdx.x == 0) {
        a.w.psum[b * kBlocks + blk] = s;
        a.w.pemax[b * kBlocks + blk] = emax;
    }
}

// 3. (model sample function) sampleToken's own softmax of the probabilities p = e / S1 at
//    temperature 1: f = exp(p - max p); max p = fl(max e / S1), division being monotone
__global__ __launch_bounds__(kThreads) void smp_exp2_kernel(Args a) {
    __shared__ double red[kWaves];
    const int blk = blockIdx.x, b = blockIdx.y;
    int c0, c1;
    chunk_of(a.V, blk, &c0, &c1);
    const double S1 = row_sum(a.w.psum + b * kBlocks);
    const double m2 = row_max(a.w.pemax + b * kBlocks) / S1;
    double* buf = a.w.buf + (size_t)b * a.V;
    double s = 0.0;
    for (int i = c0 + threadIdx.x; i < c1; i += kThreads) {
        const double f = exp(buf[i] / S1 - m2);
        buf[i] = f;
        s += f;
    }
    s = block_sum_d(s, red);
    if (threadIdx.x == 0) a.w.psum2[b * kBlocks + blk] = s;
}

__device__ inline double denom(const Args& a, int b) {
    return row_sum((a.mode == AR_SAMPLE_TOKEN ? a.w.psum : a.w.psum2) + b * kBlocks);
}

// The digit choice of one pass (wavefront 0 of the last chunk): the highest non-empty bucket d
// with above + sum(buckets >= d) >= target, scanning buckets in descending order, 4 per lane.
__device__ void select_digit(const Args& a, int b, int level, unsigned long long target, const unsigned* cnt,
                             const unsigned long long* sm) {
    const int lane = threadIdx.x & 63;
    unsigned long long* sel = a.w.sel + b * 8;
    // state left by the previous pass (nothing before the first)
    const unsigned long long prefix0 = level ? sel[0] : 0ull;
    const unsigned long long above = level ? sel[1] : 0ull;
    unsigned long long lsum = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) lsum += sm[255 - 4 * lane - k];
    const unsigned long long before = wave_incl_scan(lsum) - lsum;  // buckets above this lane's four
    unsigned long long acc = above + before;
    int hit = -1;
    unsigned long long acc_hit = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int d = 255 - 4 * lane - k;
        if (hit < 0 && cnt[d] && acc + sm[d] >= target) {
            hit = d;
            acc_hit = acc;
        }
        acc += sm[d];
    }
    const unsigned long long hits = __ballot(hit >= 0);
    if (!hits) {  // the whole row sums to less than top_p: the reference keeps every value
        if (lane == 0) sel[2] = 1;
        return;
    }
    if (lane != __builtin_ctzll(hits)) return;
    const int shift = 56 - 8 * level;
    const unsigned long long prefix = prefix0 | ((unsigned long long)hit << shift);
    sel[0] = prefix;  // prefix
    sel[1] = acc_hit; // fixed-point sum of the values above the prefix range
    unsigned long long done = 0, take = 0;  // done: 0 searching, 1 keep everything, 2 cut found
    if (level == 7) {
        const double pstar = __longlong_as_double((long long)prefix);
        const unsigned long long pf = (unsigned long long)(pstar * kFix);
        const unsigned long long ties = cnt[hit];
        take = 1;
        if (target > acc_hit) take = pf ? (target - acc_hit + pf - 1) / pf : ties;
        take = take < 1 ? 1 : (take > ties ? ties : take);
        done = 2;
    }
    sel[2] = done;
    sel[3] = take;  // values == p* kept
}

// 4. nucleus search, pass `level`: histogram of digit (key >> shift) & 255 over the keys that match
//    the prefix chosen so far; the last chunk to arrive picks the digit
__global__ __launch_bounds__(kThreads) void smp_hist_kernel(Args a, int level, unsigned long long target) {
    __shared__ unsigned cnt[256];
    __shared__ unsigned long long sm[256];
    __shared__ int last_s;
    const int blk = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    if (t < 256) {
        cnt[t] = 0;
        sm[t] = 0;
    }
    __syncthreads();
    int c0, c1;
    chunk_of(a.V, blk, &c0, &c1);
    const double D = denom(a, b);
    const int shift = 56 - 8 * level;
    const int hs = level ? shift + 8 : 0;  // bits above the current digit (none at level 0)
    const unsigned long long want = level ? a.w.sel[b * 8 + 0] >> hs : 0ull;
    const bool searching = level == 0 || a.w.sel[b * 8 + 2] == 0;
    const double* buf = a.w.buf + (size_t)b * a.V;
    if (searching) {
        for (int i = c0 + t; i < c1; i += kThreads) {
            const double p = buf[i] / D;
            const unsigned long long key = (unsigned long long)__double_as_longlong(p);
            if (level == 0 || (key >> hs) == want) {
                const int d = (int)((key >> shift) & 255);
                atomicAdd(&cnt[d], 1u);
                atomicAdd(&sm[d], (unsigned long long)(p * kFix));
            }
        }
    }
    __syncthreads();
    if (t < 256) {
        a.w.hcnt[((size_t)b * kBlocks + blk) * 256 + t] = cnt[t];
        if (cnt[t]) {
            __hip_atomic_fetch_add(a.w.gcnt + b * 256 + t, cnt[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(a.w.gsum + b * 256 + t, sm[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's histogram atomics have completed
    __syncthreads();
    if (t == 0) {
        unsigned* c = a.w.arrived + b;
        const unsigned prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == (unsigned)(kBlocks - 1);
        if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_s = last;
    }
    __syncthreads();
    if (!last_s) return;
    // the row histogram, read once and cleared for the next pass
    if (t < 256) {
        cnt[t] = __hip_atomic_load(a.w.gcnt + b * 256 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sm[t] = __hip_atomic_load(a.w.gsum + b * 256 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.w.gcnt + b * 256 + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.w.gsum + b * 256 + t, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (t < 64 && searching) select_digit(a, b, level, target, cnt, sm);
}

// Membership of the nucleus: values > p* and the first `take` (by index) of the values == p*.
struct Nucleus {
    int mode;                   // 0: everything (no top-p), 1: everything (top-p kept all), 2: cut
    unsigned long long pstar, take;
};

__device__ inline Nucleus nucleus_of(const Args& a, int b) {
    Nucleus n{0, 0, 0};
    if (!a.topp) return n;
    const unsigned long long* sel = a.w.sel + b * 8;
    if (sel[2] != 2) {
        n.mode = 1;
        return n;
    }
    n.mode = 2;
    n.pstar = sel[0];
    n.take = sel[3];
    return n;
}

__device__ inline void thread_range(int c0, int c1, int* r0, int* r1) {
    const int per = (c1 - c0 + kThreads - 1) / kThreads;
    *r0 = min(c1, c0 + (int)threadIdx.x * per);
    *r1 = min(c1, *r0 + per);
}

// Number of values == p* before this thread's contiguous range: earlier chunks (their last-pass
// histograms) plus earlier threads of this chunk (a block scan).
__device__ inline unsigned long long tie_base(const Args& a, const Nucleus& n, int b, int blk, int r0, int r1,
                                              double D, unsigned long long* red) {
    unsigned long long mine = 0;
    if (n.mode == 2) {
        const double* buf = a.w.buf + (size_t)b * a.V;
        for (int i = r0; i < r1; i++)
            mine += (unsigned long long)__double_as_longlong(buf[i] / D) == n.pstar;
    }
    unsigned long long before_chunk = 0;
    if (n.mode == 2) {
        const int lane = threadIdx.x & 63;
        const int d = (int)(n.pstar & 255);
        unsigned long long v = lane < blk ? a.w.hcnt[((size_t)b * kBlocks + lane) * 256 + d] : 0ull;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        before_chunk = v;
    }
    return before_chunk + block_incl_scan(mine, red) - mine;
}

__device__ inline double kept(const Nucleus& n, double q, unsigned long long* rank) {
    if (n.mode != 2) return q;
    const unsigned long long key = (unsigned long long)__double_as_longlong(q);
    if (key > n.pstar) return q;
    if (key == n.pstar) return (*rank)++ < n.take ? q : 0.0;
    return 0.0;
}

// 5. kept probability mass per chunk (before the nucleus renormalisation)
__global__ __launch_bounds__(kThreads) void smp_mass_kernel(Args a) {
    __shared__ unsigned long long ured[kWaves];
    __shared__ double red[kWaves];
    const int blk = blockIdx.x, b = blockIdx.y;
    int c0, c1, r0, r1;
    chunk_of(a.V, blk, &c0, &c1);
    thread_range(c0, c1, &r0, &r1);
    const double D = denom(a, b);
    const Nucleus n = nucleus_of(a, b);
    unsigned long long rank = tie_base(a, n, b, blk, r0, r1, D, ured);
    const double* buf = a.w.buf + (size_t)b * a.V;
    double s = 0.0;
    for (int i = r0; i < r1; i++) s += kept(n, buf[i] / D, &rank);
    s = block_sum_d(s, red);
    if (threadIdx.x == 0) a.w.pmass[b * kBlocks + blk] = s;
}

__device__ inline double java_next_double(unsigned long long* s) {
    constexpr unsigned long long mult = 0x5DEECE66DULL, add = 0xBULL, mask = (1ULL << 48) - 1;
    unsigned long long x = *s;
    x = (x * mult + add) & mask;
    const long long hi = (long long)(x >> 22);  // next(26)
    x = (x * mult + add) & mask;
    const long long lo = (long long)(x >> 21);  // next(27)
    *s = x;
    return (double)((hi << 27) + lo) * 0x1.0p-53;
}

// 6. one block per row: the uniform draw and the index whose cumulative interval holds it
__global__ __launch_bounds__(kThreads) void smp_draw_kernel(Args a) {
    __shared__ unsigned long long ured[kWaves];
    __shared__ double dred[kWaves];
    __shared__ int ifirst[kWaves], ilast[kWaves];
    __shared__ double sh_r, sh_c, sh_Z;
    __shared__ int sh_blk, sh_idx;
    const int b = blockIdx.x, t = threadIdx.x, lane = t & 63;
    // The model draws only when the next step feeds a sampled token (past the prompt), as
    // AutoregressiveModel.next applies its sample function (AutoregressiveModel.java:295-308).
    if (a.state && a.state[2] < a.state[1]) return;
    const double D = denom(a, b);
    const Nucleus n = nucleus_of(a, b);
    if (t < 64) {
        // chunk masses in index order; the first chunk whose running total exceeds r
        const double pm = a.w.pmass[b * kBlocks + lane];
        const double Z = a.topp ? wave_sum_d(pm) : 1.0;
        const double m = a.topp ? pm / Z : pm;
        const double incl = wave_incl_scan(m);
        const double excl = __shfl_up(incl, 1, 64);
        double r = 0.0;
        if (lane == 0) r = java_next_double(a.rng + b);
        r = __shfl(r, 0, 64);
        const unsigned long long hits = __ballot(r < incl);
        if (lane == 0) {
            sh_r = r;
            sh_Z = Z;
            sh_blk = hits ? __builtin_ctzll(hits) : -1;
            sh_idx = a.V - 1;  // the reference's result when no running sum exceeds r
        }
        if (hits && lane == __builtin_ctzll(hits)) sh_c = lane ? excl : 0.0;
    }
    __syncthreads();
    const int blk = sh_blk;
    if (blk >= 0) {
        int c0, c1, r0, r1;
        chunk_of(a.V, blk, &c0, &c1);
        thread_range(c0, c1, &r0, &r1);
        const unsigned long long rank0 = tie_base(a, n, b, blk, r0, r1, D, ured);
        const double* buf = a.w.buf + (size_t)b * a.V;
        const double Z = sh_Z, r = sh_r, c = sh_c;
        double s = 0.0;
        int last = -1;
        unsigned long long rank = rank0;
        for (int i = r0; i < r1; i++) {
            double q = kept(n, buf[i] / D, &rank);
            if (a.topp) q /= Z;
            s += q;
            if (q > 0.0) last = i;
        }
        const double incl = block_incl_scan(s, dred);
        // first thread whose running total exceeds r (thread order = index order), and the last
        // positive value of the chunk: the fallback when rounding of the grouped sums leaves r
        // past the chunk's total
        const unsigned long long wh = __ballot(r < c + incl);
        int wl = last;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) wl = max(wl, __shfl_xor(wl, o, 64));
        if (lane == 0) {
            ifirst[t >> 6] = wh ? (t & ~63) + __builtin_ctzll(wh) : 0x7FFFFFFF;
            ilast[t >> 6] = wl;
        }
        __syncthreads();
        int first = 0x7FFFFFFF, lastpos = -1;
        for (int w = 0; w < kWaves; w++) {
            first = min(first, ifirst[w]);
            lastpos = max(lastpos, ilast[w]);
        }
        if (first == 0x7FFFFFFF) {
            if (t == 0) sh_idx = lastpos >= 0 ? lastpos : c1 - 1;
        } else if (t == first) {
            double cc = c + (incl - s);
            rank = rank0;
            int idx = last >= 0 ? last : r1 - 1;
            for (int i = r0; i < r1; i++) {
                double q = kept(n, buf[i] / D, &rank);
                if (a.topp) q /= Z;
                cc += q;
                if (r < cc) {
                    idx = i;
                    break;
                }
            }
            sh_idx = idx;
        }
    }
    __syncthreads();
    if (t == 0) {
        const int idx = sh_idx;
        if (a.out) a.out[b] = idx;
        if (a.keys)  // beats every value key of the greedy epilogue: the next step feeds idx
            a.keys[(size_t)b * a.keys_stride] = (0xFFFFFFFFull << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)idx);
    }
}

}  // namespace

bool sample_is_greedy(int mode, double temperature) {
    // sampleToken: temperature <= 0 is greedy; the model's sample function: temperature == 0
    return mode == AR_SAMPLE_TOKEN ? !(temperature > 0.0) : temperature == 0.0;
}

size_t sample_workspace_bytes(int rows, int vocab) {
    size_t total = 0;
    carve(nullptr, rows, vocab, &total, nullptr);
    return total;
}

int sample_workspace_clear(void* work, int rows, int vocab, hipStream_t st) {
    size_t zero = 0;
    carve(work, rows, vocab, nullptr, &zero);
    return launch_fill_i32((int*)work, 0, zero / 4, st);  // a kernel: safe inside a captured graph
}

int launch_sample(const SampleLaunch& s, hipStream_t st) {
    AR_CHECK_ARG(s.logits && s.work && s.rng && s.rows > 0 && s.vocab > 0 && s.logits_stride >= s.vocab,
                 "sample: bad arguments");
    AR_CHECK_ARG(s.mode == AR_SAMPLE_TOKEN || s.mode == AR_SAMPLE_MODEL, "sample: unknown mode %d", s.mode);
    AR_CHECK_ARG(!sample_is_greedy(s.mode, s.temperature), "sample: temperature %g selects the greedy path",
                 s.temperature);
    Args a{};
    a.logits = s.logits;
    a.ls = s.logits_stride;
    a.V = s.vocab;
    a.mode = s.mode;
    a.T = s.temperature;
    a.topp = s.mode == AR_SAMPLE_TOKEN && s.top_p < 1.0;
    a.w = carve(s.work, s.rows, s.vocab, nullptr, nullptr);
    a.rng = s.rng;
    a.state = s.state;
    a.keys = s.keys;
    a.keys_stride = s.keys_stride;
    a.out = s.out;
    const dim3 grid(kBlocks, s.rows), block(kThreads);
    hipLaunchKernelGGL(smp_max_kernel, grid, block, 0, st, a);
    AR_LAUNCH_CHECK();
    hipLaunchKernelGGL(smp_exp_kernel, grid, block, 0, st, a);
    AR_LAUNCH_CHECK();
    if (s.mode == AR_SAMPLE_MODEL) {
        hipLaunchKernelGGL(smp_exp2_kernel, grid, block, 0, st, a);
        AR_LAUNCH_CHECK();
    }
    if (a.topp) {
        // cumulative >= top_p in 2^-60 fixed point (top_p <= 0 keeps the single largest value)
        const double tp = s.top_p > 0.0 ? ceil(s.top_p * kFix) : 0.0;
        const unsigned long long target = (unsigned long long)tp;
        for (int level = 0; level < 8; level++) {
            hipLaunchKernelGGL(smp_hist_kernel, grid, block, 0, st, a, level, target);
            AR_LAUNCH_CHECK();
        }
    }
    hipLaunchKernelGGL(smp_mass_kernel, grid, block, 0, st, a);
    AR_LAUNCH_CHECK();
    hipLaunchKernelGGL(smp_draw_kernel, dim3(s.rows), block, 0, st, a);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}
