// Token sampling on the device: temperature softmax, nucleus (top-p) filtering and the
// categorical draw of AutoregressiveModel.sampleToken (engine/ml/.../AutoregressiveModel.java:323-386),
// and the sample function AutoregressiveModel.of installs (:413-425: logits / temperature, the
// DistributionFeatures.softmax of compute/stats/.../DistributionFeatures.java:129-141, then
// sampleToken(probabilities, V, 1.0, 1.0, random)), with java.util.Random's generator
// (48-bit LCG, nextDouble = ((next(26) << 27) + next(27)) * 2^-53) kept per sequence on the device.
//
// Everything after the fp32 logits is double, the reference's precision.  A row of V values is cut
// into kBlocks chunks; each pass is one grid of (kBlocks, rows) 256-thread blocks whose per-block
// maxima / sums go to the workspace and are combined by the next kernel in a fixed order (a
// wavefront butterfly over the 64 chunk values), so every result is deterministic.
//
// Nucleus filtering does not sort.  The reference keeps the shortest prefix of the probabilities
// sorted in descending order (ties in index order: Arrays.sort is stable) whose running sum
// reaches top_p.  With p* the smallest kept value, that is every value > p* plus the first c
// (by index) of the values == p*; p* is the largest key t with sum(p >= t) >= top_p.  It is found
// by a radix descent over the 64-bit patterns of the probabilities (non-negative doubles order as
// their bit patterns): 8 passes of 8-bit digits, each a per-chunk histogram of (count, sum) and a
// one-block select of the digit.  Bucket sums are 2^-60 fixed point in u64 (exact, associative:
// the histograms are independent of timing); the kept set agrees with the reference's sequential
// double sums except when top_p lies within ~1e-13 of a partial sum.
//
// The draw mirrors the reference's loop `cumulative += probs[i]; if (r < cumulative) return i`:
// chunk masses locate the chunk whose interval holds r, then per-thread sums of contiguous index
// ranges and a walk of the crossing thread's elements locate the index.  Partial sums group
// differently from the reference's single running sum (rounding ~1e-16), so a draw within that
// distance of a boundary may pick the neighbour.
#include "ar_hip_internal.h"

namespace {

constexpr int kBlocks = 64;   // chunks per row (one wavefront of partials)
constexpr int kThreads = 256;
constexpr double kFix = 1152921504606846976.0;     // 2^60
constexpr double kEps64 = 2.220446049250313e-16;   // FP64 machine epsilon (Precision.java:110-121)

struct Ws {
    double* buf;                // [rows][V] exp values
    double* pmax;               // [rows][kBlocks]
    double* psum;
    double* pemax;
    double* psum2;
    double* pmass;
    unsigned* hcnt;             // [rows][kBlocks][256]
    unsigned long long* hsum;   // [rows][kBlocks][256]
    unsigned long long* sel;    // [rows][8]: prefix, above, done, take, -, -, -, -
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

Ws carve(void* base, int rows, int V, size_t* total) {
    Ws w{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const uintptr_t p = reinterpret_cast<uintptr_t>(base) + off;
        off += align256(bytes);
        return reinterpret_cast<void*>(p);
    };
    w.buf = (double*)take((size_t)rows * V * 8);
    w.pmax = (double*)take((size_t)rows * kBlocks * 8);
    w.psum = (double*)take((size_t)rows * kBlocks * 8);
    w.pemax = (double*)take((size_t)rows * kBlocks * 8);
    w.psum2 = (double*)take((size_t)rows * kBlocks * 8);
    w.pmass = (double*)take((size_t)rows * kBlocks * 8);
    w.hcnt = (unsigned*)take((size_t)rows * kBlocks * 256 * 4);
    w.hsum = (unsigned long long*)take((size_t)rows * kBlocks * 256 * 8);
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
// block reductions (256 threads): butterfly per wavefront, then the 4 wavefront values in order
__device__ inline double block_max_d(double v, double* red) {
    v = wave_max_d(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const double r = fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
    __syncthreads();
    return r;
}
__device__ inline double block_sum_d(double v, double* red) {
    v = wave_sum_d(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const double r = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
    return r;
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
    __shared__ double red[4];
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
    __shared__ double red[4];
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
    __shared__ double red[4];
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

// 4. nucleus search, pass `level`: histogram of digit (key >> shift) & 255 over the keys that match
//    the prefix chosen so far
__global__ __launch_bounds__(kThreads) void smp_hist_kernel(Args a, int level) {
    __shared__ unsigned cnt[256];
    __shared__ unsigned long long sm[256];
    const int blk = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    cnt[t] = 0;
    sm[t] = 0;
    __syncthreads();
    int c0, c1;
    chunk_of(a.V, blk, &c0, &c1);
    const double D = denom(a, b);
    const int shift = 56 - 8 * level;
    const int hs = level ? shift + 8 : 0;  // bits above the current digit (none at level 0)
    const unsigned long long want = level ? a.w.sel[b * 8 + 0] >> hs : 0ull;
    const double* buf = a.w.buf + (size_t)b * a.V;
    for (int i = c0 + t; i < c1; i += kThreads) {
        const double p = buf[i] / D;
        const unsigned long long key = (unsigned long long)__double_as_longlong(p);
        if (level == 0 || (key >> hs) == want) {
            const int d = (int)((key >> shift) & 255);
            atomicAdd(&cnt[d], 1u);
            atomicAdd(&sm[d], (unsigned long long)(p * kFix));
        }
    }
    __syncthreads();
    const size_t o = ((size_t)b * kBlocks + blk) * 256 + t;
    a.w.hcnt[o] = cnt[t];
    a.w.hsum[o] = sm[t];
}

// 5. one block per row: add the chunk histograms (fixed order), pick the digit
__global__ __launch_bounds__(kThreads) void smp_select_kernel(Args a, int level, unsigned long long target) {
    __shared__ unsigned cnt[256];
    __shared__ unsigned long long sm[256];
    const int b = blockIdx.x, t = threadIdx.x;
    unsigned long long* sel = a.w.sel + b * 8;
    unsigned c = 0;
    unsigned long long s = 0;
    for (int j = 0; j < kBlocks; j++) {
        const size_t o = ((size_t)b * kBlocks + j) * 256 + t;
        c += a.w.hcnt[o];
        s += a.w.hsum[o];
    }
    cnt[t] = c;
    sm[t] = s;
    __syncthreads();
    if (t != 0) return;
    if (level == 0) {
        sel[0] = 0;  // prefix
        sel[1] = 0;  // fixed-point sum of the values above the prefix range
        sel[2] = 0;  // 0 searching, 1 keep everything, 2 cut found
        sel[3] = 0;  // values == p* kept
    }
    if (sel[2] == 1) return;
    const int shift = 56 - 8 * level;
    unsigned long long acc = sel[1];
    int dstar = -1;
    for (int d = 255; d >= 0; d--) {
        if (cnt[d] && acc + sm[d] >= target) {
            dstar = d;
            break;
        }
        acc += sm[d];
    }
    if (dstar < 0) {  // the whole row sums to less than top_p: the reference keeps every value
        sel[2] = 1;
        return;
    }
    sel[0] |= (unsigned long long)dstar << shift;
    sel[1] = acc;
    if (level == 7) {
        const double pstar = __longlong_as_double((long long)sel[0]);
        const unsigned long long pf = (unsigned long long)(pstar * kFix);
        const unsigned long long ties = cnt[dstar];
        unsigned long long take = 1;
        if (target > acc) take = pf ? (target - acc + pf - 1) / pf : ties;
        take = take < 1 ? 1 : (take > ties ? ties : take);
        sel[3] = take;
        sel[2] = 2;
    }
}

// Membership of the nucleus for the contiguous index range of one thread: `rank` is the number of
// values == p* before the range (a block-level scan of per-thread tie counts).
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

// Per-thread range inside chunk [c0, c1) and the number of p* ties before it.
__device__ inline unsigned long long tie_base(const Args& a, const Nucleus& n, int b, int blk, int r0, int r1,
                                              double D, unsigned long long* scan) {
    const int t = threadIdx.x;
    unsigned long long mine = 0;
    if (n.mode == 2) {
        const double* buf = a.w.buf + (size_t)b * a.V;
        for (int i = r0; i < r1; i++)
            mine += (unsigned long long)__double_as_longlong(buf[i] / D) == n.pstar;
    }
    scan[t] = mine;
    __syncthreads();
    if (t == 0) {
        unsigned long long before = 0;
        if (n.mode == 2) {
            const int d = (int)(n.pstar & 255);
            for (int j = 0; j < blk; j++) before += a.w.hcnt[((size_t)b * kBlocks + j) * 256 + d];
        }
        for (int k = 0; k < kThreads; k++) {
            const unsigned long long v = scan[k];
            scan[k] = before;
            before += v;
        }
    }
    __syncthreads();
    const unsigned long long base = scan[t];
    __syncthreads();
    return base;
}

__device__ inline double kept(const Nucleus& n, double q, unsigned long long* rank) {
    if (n.mode != 2) return q;
    const unsigned long long key = (unsigned long long)__double_as_longlong(q);
    if (key > n.pstar) return q;
    if (key == n.pstar) return (*rank)++ < n.take ? q : 0.0;
    return 0.0;
}

__device__ inline void thread_range(int c0, int c1, int* r0, int* r1) {
    const int per = (c1 - c0 + kThreads - 1) / kThreads;
    *r0 = min(c1, c0 + (int)threadIdx.x * per);
    *r1 = min(c1, *r0 + per);
}

// 6. kept probability mass per chunk (before the nucleus renormalisation)
__global__ __launch_bounds__(kThreads) void smp_mass_kernel(Args a) {
    __shared__ unsigned long long scan[kThreads];
    __shared__ double red[4];
    const int blk = blockIdx.x, b = blockIdx.y;
    int c0, c1, r0, r1;
    chunk_of(a.V, blk, &c0, &c1);
    thread_range(c0, c1, &r0, &r1);
    const double D = denom(a, b);
    const Nucleus n = nucleus_of(a, b);
    unsigned long long rank = tie_base(a, n, b, blk, r0, r1, D, scan);
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

// 7. one block per row: the uniform draw and the index whose cumulative interval holds it
__global__ __launch_bounds__(kThreads) void smp_draw_kernel(Args a) {
    __shared__ unsigned long long scan[kThreads];
    __shared__ double tsum[kThreads];
    __shared__ int tlast[kThreads];
    __shared__ double sh_r, sh_c, sh_Z;
    __shared__ int sh_blk, sh_t, sh_idx;
    const int b = blockIdx.x, t = threadIdx.x;
    // The model draws only when the next step feeds a sampled token (past the prompt), as
    // AutoregressiveModel.next applies its sample function (AutoregressiveModel.java:295-308).
    if (a.state && a.state[2] < a.state[1]) return;
    const double D = denom(a, b);
    const Nucleus n = nucleus_of(a, b);
    if (t == 0) {
        const double r = java_next_double(a.rng + b);
        double Z = 1.0;
        if (a.topp) {
            Z = 0.0;
            for (int j = 0; j < kBlocks; j++) Z += a.w.pmass[b * kBlocks + j];
        }
        double c = 0.0;
        int blk = -1;
        for (int j = 0; j < kBlocks; j++) {
            const double m = a.topp ? a.w.pmass[b * kBlocks + j] / Z : a.w.pmass[b * kBlocks + j];
            if (r < c + m) {
                blk = j;
                break;
            }
            c += m;
        }
        sh_r = r;
        sh_c = c;
        sh_Z = Z;
        sh_blk = blk;
        sh_idx = a.V - 1;  // the reference's result when no running sum exceeds r
    }
    __syncthreads();
    const int blk = sh_blk;
    if (blk >= 0) {
        int c0, c1, r0, r1;
        chunk_of(a.V, blk, &c0, &c1);
        thread_range(c0, c1, &r0, &r1);
        unsigned long long rank0 = tie_base(a, n, b, blk, r0, r1, D, scan);
        const double* buf = a.w.buf + (size_t)b * a.V;
        const double Z = sh_Z;
        double s = 0.0;
        int last = -1;
        unsigned long long rank = rank0;
        for (int i = r0; i < r1; i++) {
            double q = kept(n, buf[i] / D, &rank);
            if (a.topp) q /= Z;
            s += q;
            if (q > 0.0) last = i;
        }
        tsum[t] = s;
        tlast[t] = last;
        __syncthreads();
        if (t == 0) {
            double c = sh_c;
            const double r = sh_r;
            int tc = -1, lastpos = -1;
            for (int k = 0; k < kThreads; k++) {
                if (tlast[k] >= 0) lastpos = tlast[k];
                if (r < c + tsum[k]) {
                    tc = k;
                    break;
                }
                c += tsum[k];
            }
            sh_t = tc;
            sh_c = c;
            // rounding of the grouped sums left r past this chunk's total: its last positive value
            if (tc < 0) sh_idx = lastpos >= 0 ? lastpos : c1 - 1;
        }
        __syncthreads();
        if (t == sh_t) {
            double c = sh_c;
            const double r = sh_r;
            rank = rank0;
            int idx = last >= 0 ? last : r1 - 1;
            for (int i = r0; i < r1; i++) {
                double q = kept(n, buf[i] / D, &rank);
                if (a.topp) q /= Z;
                c += q;
                if (r < c) {
                    idx = i;
                    break;
                }
            }
            sh_idx = idx;
        }
        __syncthreads();
    }
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
    carve(nullptr, rows, vocab, &total);
    return total;
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
    a.w = carve(s.work, s.rows, s.vocab, nullptr);
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
            hipLaunchKernelGGL(smp_hist_kernel, grid, block, 0, st, a, level);
            AR_LAUNCH_CHECK();
            hipLaunchKernelGGL(smp_select_kernel, dim3(s.rows), block, 0, st, a, level, target);
            AR_LAUNCH_CHECK();
        }
    }
    hipLaunchKernelGGL(smp_mass_kernel, grid, block, 0, st, a);
    AR_LAUNCH_CHECK();
    hipLaunchKernelGGL(smp_draw_kernel, dim3(s.rows), block, 0, st, a);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}
