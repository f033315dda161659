// Internal declarations shared by the HIP backend translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_ext.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/ar_hip.h"

// ---- error channel ---------------------------------------------------------------
// Every C-ABI entry point returns an AR_HIP_* code; the message for the calling thread
// is kept here and returned by ar_hip_last_error().
void ar_set_error(const char* fmt, ...);
// A notice on stderr when AR_HIP_LOG is set (no error state).
void ar_log(const char* fmt, ...);
// Debug pointer check (AR_HIP_CHECK_PTRS=1): [p, p + bytes) must lie inside the device allocation
// holding p; null p or zero bytes pass.  A no-op returning AR_HIP_OK when the flag is off.
bool ar_check_ptrs_enabled();
int ar_check_range(const void* p, size_t bytes, const char* kernel, const char* what);
void ar_clear_error();

#define AR_CHECK_ARG(cond, ...)                  \
    do {                                         \
        if (!(cond)) {                           \
            ar_set_error(__VA_ARGS__);           \
            return AR_HIP_ERR_INVALID;           \
        }                                        \
    } while (0)

#define AR_HIP_TRY(expr)                                                                   \
    do {                                                                                   \
        hipError_t _e = (expr);                                                            \
        if (_e != hipSuccess) {                                                            \
            ar_set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, \
                         __LINE__);                                                        \
            return AR_HIP_ERR_HIP;                                                         \
        }                                                                                  \
    } while (0)

#define AR_TRY(expr)                 \
    do {                             \
        int _rc = (expr);            \
        if (_rc != AR_HIP_OK) return _rc; \
    } while (0)

#define AR_LAUNCH_CHECK()                                                                 \
    do {                                                                                  \
        hipError_t _e = hipGetLastError();                                                \
        if (_e != hipSuccess) {                                                           \
            ar_set_error("kernel launch failed: %s (%s:%d)", hipGetErrorString(_e),       \
                         __FILE__, __LINE__);                                             \
            return AR_HIP_ERR_HIP;                                                        \
        }                                                                                 \
    } while (0)

// ---- data / compute context ------------------------------------------------------
struct ar_hip_ctx {
    int device = 0;
    int num_cus = 0;
    size_t hbm_bytes = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;
    std::unordered_map<void*, size_t> device_allocs;  // memory-provider bookkeeping
    std::unordered_map<void*, size_t> host_allocs;
    size_t device_bytes = 0;
    // device address of this device's copy of the allocation-free attention entry point's scratch
    // array (ops.hip), looked up once by ar_hip_init
    float* noalloc_scratch = nullptr;
    // rocBLAS handle of the prefill products on rocBLAS (gemm_blas.hip), created by their first call
    void* blas = nullptr;
};

// Looks up the device addresses the operator entry points need on ctx's device (called by
// ar_hip_init with that device current).
int ar_ops_init(ar_hip_ctx* ctx);

// Device allocation owned by the context's memory provider.
int ar_ctx_alloc(ar_hip_ctx* ctx, size_t bytes, void** out);
int ar_ctx_free(ar_hip_ctx* ctx, void* p);

// Uncached device memory for cross-block exchange words: its loads and stores go past the XCD
// L2s to memory, which shortens a device-scope exchange round (measured on the persistent decode
// step).  Such memory is never returned to the driver while the process runs (device allocations
// made after uncached memory was freed have held wrong values on these parts): a block given back
// with ar_uncached_put joins a per-device free list and is handed out again by a later
// ar_uncached_get of at most its size.  The caller clears what it gets; `device` must be current.
int ar_uncached_get(int device, size_t bytes, void** out);
void ar_uncached_put(void* p);

// Per-device caches of launch facts (CU count, resident-grid size, function attributes set):
// indexed by the device of the stream a launch goes to.
constexpr int kMaxDevices = 64;
// Device of `stream` (the device its launches run on) as a cache index, or -1 (unknown device, or an
// index past the cache).
int ar_device_slot(hipStream_t stream);
// Compute units of the device of `stream` (cached per device; 256 if it cannot be read).
int ar_device_cus(hipStream_t stream);

// ---- kernel timing hook ------------------------------------------------------------
// While a LaunchTiming is installed on the calling thread, the decode launchers that go through
// ar_launch (the GEMVs, the decode attention and its combine) put `start` into the dispatch of the
// first kernel they launch and `stop` into every dispatch after it (hipExtLaunchKernel records the
// events as part of the dispatch), so stop - start spans the class's kernels' execution, as a
// profiler's kernel trace measures it, without the enqueue gaps around them.  Eager launches only.
struct LaunchTiming {
    hipEvent_t start = nullptr, stop = nullptr;
    bool started = false;
};
extern thread_local LaunchTiming* g_launch_timing;

template <typename... Args, typename F = void (*)(Args...)>
inline void ar_launch(F kernel, const dim3& grid, const dim3& block, uint32_t shmem, hipStream_t stream, Args... args) {
    LaunchTiming* t = g_launch_timing;
    if (!t) {
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream, args...);
        return;
    }
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, t->started ? nullptr : t->start, t->stop, 0u, args...);
    t->started = true;
}

// ---- kernel launchers (device pointers, enqueue on `stream`) ----------------------
struct GemvLaunch {
    const void* w = nullptr;       // rows x cols, row-major, weight dtype
    const void* w2 = nullptr;      // second matrix (SwiGLU up projection), same shape
    int wdtype = AR_DTYPE_F32;
    int rows = 0, cols = 0, batch = 1;
    const float* x = nullptr;      // [batch][x_stride]
    int x_stride = 0;
    const float* norm_w = nullptr; // RMSNorm gain over cols (prologue), or null
    float eps = 1e-6f;
    const float* bias = nullptr;   // [rows] or null
    float* y = nullptr;            // [batch][y_stride]
    int y_stride = 0;
    int epilogue = 0;              // GEMV_EPI_*
    // argmax epilogue: packed (value, index) maxima, [batch][kArgmaxSlots], zero before use
    unsigned long long* keys = nullptr;
    // bf16 operand planes (MFMA path: batch >= 3, bf16 weights).  x_hi / x_lo [batch][x_stride]:
    // hi = bf16(g*x), lo = bf16(g*x - hi) of the input (g = norm_w, or 1), written by the kernel
    // that produced x, so the GEMV does not convert its input; null: converted from x.  y_hi / y_lo
    // [batch][y_stride]: the same planes of this GEMV's output (the value stored to y) scaled by
    // y_gain (the next GEMV's RMSNorm gain, or null for 1), for the next GEMV.
    const uint16_t* x_hi = nullptr;
    const uint16_t* x_lo = nullptr;
    uint16_t* y_hi = nullptr;
    uint16_t* y_lo = nullptr;
    const float* y_gain = nullptr;
    // workspace of the MFMA path's k-split form (fewer 16-row tiles than CUs, no RMSNorm, no argmax):
    // k-slice partial tiles (kpart_floats floats) and one arrival counter per tile (zero between
    // launches: the block that completes a tile resets it); null: no split
    float* kpart = nullptr;
    int kpart_floats = 0;
    unsigned* kcount = nullptr;
    int kcount_n = 0;
    // fragment-ordered copies of w / w2 (launch_frag_copy; batch <= 8, rows % 16 == 0, store / residual /
    // SwiGLU epilogue, operand planes given): the GEMV reads these instead, over an even split of the
    // fragments (gemv_frag.hip), with kpart / kcount (gemv_frag_part_floats, one counter per 16-row tile)
    // as the workspace of tiles shared by wavefronts.  ss_in [cols/16][16]: per-16-row sums of squares
    // of x, published by x's producer (needed with norm_w); ss_out [rows/16][16]: the same of the
    // residual epilogue's output, or null
    const uint16_t* w_frag = nullptr;
    const uint16_t* w2_frag = nullptr;
    const float* ss_in = nullptr;
    float* ss_out = nullptr;
};

// fragment order of a bf16 matrix for the GEMV above: 16 x 32 blocks, each 64 lanes x 8 values
size_t gemv_frag_elems(int rows, int cols);
size_t gemv_frag_part_floats(int rows, int cus, int nmat);
bool gemv_frag_fits(int rows, int cols, int batch, int cus);
int launch_frag_copy(const uint16_t* w, uint16_t* out, int rows, int cols, hipStream_t st);

// Splits v into bf16 operand planes: hi = bf16(v) (round to nearest even), lo = bf16(v - hi), so
// hi + lo keeps 16 significant bits of v.
__host__ __device__ inline unsigned bf16_rne_bits(float f) {
    unsigned u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u) return (u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}
__host__ __device__ inline void bf16_planes(float v, uint16_t* hi, uint16_t* lo) {
    const unsigned h = bf16_rne_bits(v);
    const unsigned hb = h << 16;
    float hf;
    __builtin_memcpy(&hf, &hb, 4);
    *hi = (uint16_t)h;
    *lo = (uint16_t)bf16_rne_bits(v - hf);
}

constexpr int kArgmaxSlots = 1024;

// Cross-lane steps without the LDS crossbar (ds_bpermute): DPP within 16-lane rows, gfx950's
// permlane swaps across rows (below).
template <int CTRL, int ROW_MASK>
__device__ inline float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, true));
}
// sum over each 16-lane row, in every lane of the row: quad swaps, half-row mirror, row mirror
__device__ inline float row16_sum(float v) {
    v += dpp_mov<0xB1, 0xF>(v);   // quad_perm 1,0,3,2
    v += dpp_mov<0x4E, 0xF>(v);   // quad_perm 2,3,0,1
    v += dpp_mov<0x141, 0xF>(v);  // row_half_mirror: the other quad of the half row
    v += dpp_mov<0x140, 0xF>(v);  // row_mirror: the other half row
    return v;
}
// total over the 64 lanes, in lane 63 only (row shifts, then row broadcasts)
__device__ inline float wave_sum_lane63(float v) {
    v += dpp_mov<0xB1, 0xF>(v);
    v += dpp_mov<0x4E, 0xF>(v);
    v += dpp_mov<0x114, 0xF>(v);  // row_shr:4
    v += dpp_mov<0x118, 0xF>(v);  // row_shr:8
    v += dpp_mov<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_mov<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}
// maximum over the 64 lanes, in lane 63 only (lanes without a source read -inf)
template <int CTRL, int ROW_MASK>
__device__ inline float dpp_max_step(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), CTRL,
                                                               ROW_MASK, 0xF, false)));
}
__device__ inline float wave_max_lane63(float v) {
    v = dpp_max_step<0xB1, 0xF>(v);
    v = dpp_max_step<0x4E, 0xF>(v);
    v = dpp_max_step<0x114, 0xF>(v);
    v = dpp_max_step<0x118, 0xF>(v);
    v = dpp_max_step<0x142, 0xA>(v);
    v = dpp_max_step<0x143, 0xC>(v);
    return v;
}

// The value held by lane ^ 16 (permlane16_swap of v with itself: the first result holds the even
// rows in both halves of each row pair, the second the odd rows), without the LDS crossbar.
__device__ inline float xor16(float v, int lane) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((lane & 16) ? r[0] : r[1]);
}
// The value held by lane ^ 32 (permlane32_swap: lower half in the first result, upper in the second).
__device__ inline float xor32(float v, int lane) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((lane & 32) ? r[0] : r[1]);
}
// max / sum of the values held by lanes l and l ^ 32, in every lane (the swap's two results are the
// lower and the upper half in every lane, so no lane select; the sum is lower + upper in both lanes)
__device__ inline float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// fp32 values from 65520 up (and infinities) round to an infinite fp16.  The prefill path stores
// its MFMA operands as fp16; every conversion checks this and marks *range_flag (when given), so the
// caller can recompute without fp16 operands instead of carrying an infinity.
constexpr float kF16Overflow = 65520.f;
__device__ inline void f16_range_check(float v, int* range_flag) {
    if (__builtin_expect(fabsf(v) >= kF16Overflow, 0) && range_flag) *range_flag = 1;
}

enum {
    GEMV_EPI_STORE = 0,     // y = W x (+ b)
    GEMV_EPI_RESIDUAL = 1,  // y += W x
    GEMV_EPI_SWIGLU = 2,    // y = (W2 x) * silu(W x)
    GEMV_EPI_ARGMAX = 3,    // optional y = W x; greedy-token keys
};

int launch_gemv(const GemvLaunch& a, hipStream_t stream);

// Prefill GEMM on MFMA: C[M x N] = A[M x K] . W[N x K]^T, 16-bit operands (bf16, or fp16 when
// f16 is set), fp32 accumulation.
// epilogue GEMV_EPI_STORE (C = acc + bias), GEMV_EPI_RESIDUAL (C += acc) with fp32 C, or
// GEMV_EPI_SWIGLU (O = 16-bit((W2-product) * silu(W-product))).  N % 128 == 0, K % 64 == 0.
struct GemmLaunch {
    const uint16_t* A = nullptr;
    const uint16_t* W = nullptr;
    const uint16_t* W2 = nullptr;
    int M = 0, N = 0, K = 0, lda = 0, ldw = 0;
    const float* bias = nullptr;
    float* C = nullptr;
    int ldc = 0;
    uint16_t* O = nullptr;
    int ldo = 0;
    int epilogue = GEMV_EPI_STORE;
    bool f16 = false;
    int ksplit = 1;  // > 1 (store epilogue): k-slice s of the product goes to C + s*M*ldc, for the
                     // consumer to add up in a fixed order (more blocks for small M x N, no atomics)
    int* range_flag = nullptr;  // set when an fp16 SwiGLU output value overflows (f16_range_check)
};
int launch_gemm(const GemmLaunch& a, hipStream_t stream);
// The same products on rocBLAS (gemm_blas.hip; fp16 operands, ksplit 1, no bias): store / residual
// epilogues as beta 0 / 1 on fp32 C; SwiGLU as one fp16 product of 2N outputs into `gu` (at least
// M x 2N values) and a SwiGLU pass into O with the fp16 range check.
int launch_gemm_blas(ar_hip_ctx* ctx, const GemmLaunch& a, uint16_t* gu, size_t gu_elems, hipStream_t stream);
void gemm_blas_release(ar_hip_ctx* ctx);

// fp32 prefill GEMM on MFMA (gemm_f32.hip): C[M x N] = A[M x K] . W[N x K]^T, all fp32.  Epilogues as
// GemmLaunch (SwiGLU writes fp32 C).  N % 64 == 0, K % (32 * ksplit) == 0.
struct GemmF32Launch {
    const float* A = nullptr;
    const float* W = nullptr;
    const float* W2 = nullptr;
    const float* bias = nullptr;
    float* C = nullptr;
    int M = 0, N = 0, K = 0, lda = 0, ldw = 0, ldc = 0;
    int epilogue = GEMV_EPI_STORE;
    int ksplit = 1;  // > 1 (store epilogue): k-slice s goes to C + s*M*ldc, added up by the consumer
};
int launch_gemm_f32(const GemmF32Launch& a, hipStream_t stream);
// k-slices for an fp32 prefill product whose 32 x 64 tiles would not give every CU two blocks.
int gemm_f32_ksplit(int M, int N, int K, int cus);

// ---- prefill (prefill.hip) ---------------------------------------------------------
// x[r] = E[tokens[b][t]] for r = b*T + t.
int launch_embed_rows(const void* table, int wdtype, int dim, const int* tokens, int token_stride, int T, int rows,
                      float* x, hipStream_t stream);
int launch_rmsnorm_rows_f16(const float* x, const float* w, uint16_t* out, int rows, int n, float eps,
                            int* range_flag, hipStream_t stream);
// x[r] += sum_s parts[s][r] (s in order; nparts may be 0), then out[r] = fp16 RMSNorm(x[r]) as above.
int launch_fold_rmsnorm_rows_f16(float* x, const float* parts, int nparts, const float* w, uint16_t* out, int rows,
                                 int n, float eps, int* range_flag, hipStream_t stream);
// dst[b] = src[rows[b]] + sum_s parts[s][rows[b]] for b < count (rows of n floats).
int launch_fold_rows(const float* src, const float* parts, int nparts, size_t part_rows, int first, int step,
                     int count, int n, float* dst, hipStream_t stream);
// fp16 copy of bf16 data (exact for |v| >= 2^-17 inside the fp16 range; values below 2^-17 round to
// the fp16 grid of 2^-24), for the prefill GEMMs; range_flag as f16_range_check.
int launch_bf16_to_f16(const uint16_t* src, uint16_t* dst, size_t n, int* range_flag, hipStream_t stream);
struct PrefillPrep {
    const float* qkv = nullptr;
    int qkv_stride = 0;
    const float* q_norm = nullptr;
    const float* k_norm = nullptr;
    float eps = 1e-6f;
    int per_head = 0;
    const float2* rope_tab = nullptr;
    void* kcache = nullptr;    // [B][KV][S][hd] fp32, or fp16 when kv16
    void* vcache = nullptr;
    bool kv16 = false;
    int B = 1, S = 0, T = 0, p0 = 0, heads = 0, kv_heads = 0, hd = 0;
    uint16_t* qb = nullptr;
    uint16_t* k16 = nullptr;   // [B][KV][Tp][hd] fp16 keys of the prompt rows
    uint16_t* vt16 = nullptr;  // [B][KV][hd][Tp] fp16 values, transposed
    int Tp = 0;                // rows reserved per (sequence, KV head), multiple of 64
    int* range_flag = nullptr; // set when a value stored as fp16 overflows (f16_range_check)
    float* q32 = nullptr;      // fp32-weight prefill: queries go here as fp32 [R][heads*hd] (no fp16
                               // q / K / Vᵀ copies are written; qb, k16, vt16 unused)
};
int launch_qk_prep(const PrefillPrep& a, hipStream_t stream);
// x[r] += sum_s parts[s][r] (s in order; nparts may be 0), then out[r] = fp32 RMSNorm(x[r]) (the
// fp32-weight prefill's GEMM input).
int launch_fold_rmsnorm_rows_f32(float* x, const float* parts, int nparts, const float* w, float* out, int rows,
                                 int n, float eps, hipStream_t stream);
// Causal attention of the prompt rows of an fp32-weight prefill (attention.hip): row t of sequence b
// attends cache rows 0..p0+t; q32 [B*T][heads*hd] normalised rotated queries, fp32 caches
// [B][KV][S][hd] holding the prompt rows, out [B*T][heads*hd] fp32.
int launch_attention_prefill_f32(const float* q32, const float* kcache, const float* vcache, float* out, int B, int T,
                                 int p0, int S, int heads, int kv_heads, int hd, hipStream_t stream);
// Causal attention over prompt rows 0..T-1 (prefill from position 0), fp16 MFMAs, fp16 output.
int launch_flash_prefill(const uint16_t* qb, const uint16_t* k16, const uint16_t* vt16, uint16_t* out, int B, int T,
                         int Tp, int heads, int kv_heads, int hd, hipStream_t stream);

struct AttnLaunch {
    const float* qkv = nullptr;   // [batch][qkv_stride]: q | k | v raw projections, or null:
    const float* q = nullptr;     //   separate q, k, v rows (same stride)
    const float* k = nullptr;
    const float* v = nullptr;
    int qkv_stride = 0;
    const float* q_norm = nullptr;
    const float* k_norm = nullptr;
    float qk_eps = 1e-6f;
    int per_head_norm = 0;
    void* kcache = nullptr;       // [batch][kv_heads][max_seq][hd], fp32 or fp16 (kv16)
    void* vcache = nullptr;
    bool kv16 = false;
    int max_seq = 0;
    const int* pos = nullptr;     // device position (same for every sequence), or null: pos_value
    int pos_value = 0;
    int heads = 0, kv_heads = 0, head_dim = 0;
    double rope_theta = 1e6;
    const float2* rope_tab = nullptr;  // [max_seq][hd/2] (cos, sin) of pos*invf, or null: computed
    int max_splits = 0;           // grid.x; the live context pos+1 is cut into at most this many
                                  // splits of >= 16 rows (splits past it exit at once)
    float* part_o = nullptr;      // [batch][heads][max_splits][hd]
    float* part_ml = nullptr;     // [batch][heads][max_splits][2]
    float* out = nullptr;         // [batch][out_stride]
    int out_stride = 0;
    uint16_t* out_hi = nullptr;   // bf16 planes of out ([batch][out_stride], bf16_planes) for the
    uint16_t* out_lo = nullptr;   // next GEMV's MFMA path, or null
    int batch = 1;
};

// Split plan of a live context of n rows over at most max_splits splits of >= kAttnMinTile rows
// (the last may be short); the attention and combine kernels evaluate it from the device position.
constexpr int kAttnMinTile = 16;
__host__ __device__ inline void attn_split_plan(int n, int max_splits, int* nsplit, int* tile) {
    int ns = (n + kAttnMinTile - 1) / kAttnMinTile;
    if (ns > max_splits) ns = max_splits;
    if (ns < 1) ns = 1;
    const int t = (n + ns - 1) / ns;
    *tile = t;
    *nsplit = (n + t - 1) / t;
}

// Attention partials + (when the context is split) the combine kernel.
int launch_attention_decode(const AttnLaunch& a, hipStream_t stream);

// Persistent decode step (decode_persistent.hip): every layer of a batch-1 decode step in one launch
// of one block per CU.  `layers` is a device table of layer_count entries written
// by decode_persistent_layer_entry; `ll` holds decode_persistent_ll_words() zeroed words at first
// use; state[0] is the position and state[3] the exchange epoch base, which every launch advances.
struct DecodePersistentLaunch {
    const void* layers = nullptr;
    int layer_count = 0;
    int wdtype = AR_DTYPE_F32;  // projection / head weights: AR_DTYPE_F32 or AR_DTYPE_BF16
    int dim = 0, hidden_dim = 0, heads = 0, kv_heads = 0, head_dim = 0;
    float* x = nullptr;        // [dim] the step's input and, after the launch, its output
    void* kcache = nullptr;    // [L][KV][S][HD], fp32 or (kv16) fp16
    void* vcache = nullptr;
    bool kv16 = false;
    int max_seq = 0;
    const float2* rope_tab = nullptr;
    int* state = nullptr;
    uint64_t* ll = nullptr;
    int* err = nullptr;        // 1: a cross-block wait timed out; 2: position outside the cache
    unsigned wait_limit = 0;   // polls before a cross-block wait is abandoned (0: the kernel's default)
    float eps = 1e-6f;
    int per_head_norm = 0;
    // after the last layer: final RMSNorm, logits (stored when logits is non-null) and greedy keys
    const float* final_norm = nullptr;
    const void* lm_head = nullptr;  // weight type
    int vocab = 0;
    float* logits = nullptr;
    unsigned long long* keys = nullptr;  // [kArgmaxSlots], zero before the launch
};
size_t decode_persistent_layer_bytes();
size_t decode_persistent_ll_words(int wdtype, int dim, int F, int heads, int kv_heads, int hd);  // 0: none
int decode_persistent_layer_entry(void* dst, const void* wqkv, const void* wo, const void* w1, const void* w3,
                                  const void* w2, const float* attn_norm, const float* ffn_norm, const float* q_norm,
                                  const float* k_norm, const float* bqkv);
bool decode_persistent_supported(int wdtype, int dim, int F, int heads, int kv_heads, int hd, bool kv16);
int launch_decode_persistent(const DecodePersistentLaunch& a, hipStream_t stream);
size_t attention_partial_floats(int batch, int heads, int max_splits, int hd);
// Splits for a cache of max_seq rows: about one block per CU, rows per split <= 256 (1040 for an
// fp16 cache; one split, no combine, for caches of at most 256 rows).
int attention_max_splits(int max_seq, int kv_heads, int batch, bool kv16);

// Start of a decode step (one block).  state = device {current position, prompt length, next
// position}.  Position p = next: the token fed is the prompt token tokens[b][p] while p is inside
// the prompt, else the greedy choice decoded from keys[b] (the previous step's logits), which is
// also stored at tokens[b][p]; keys are then cleared, x[b] = E[token], current = p, next = p+1.
// x_hi / x_lo (optional): bf16 planes of x_gain * x (bf16_planes) for the first GEMV's MFMA path;
// ss_out (optional, [dim/16][16]): sums of squares of each 16 consecutive entries of x[b] (column b),
// for the fragment-ordered GEMV's RMSNorm.
// AutoregressiveModel.next + the embedding copy (engine/ml/.../AutoregressiveModel.java:295-308,430).
int launch_step_begin(const void* table, int wdtype, int dim, int vocab, int* tokens, int token_stride,
                      unsigned long long* keys, int* state, int batch, float* x, int x_stride,
                      uint16_t* x_hi, uint16_t* x_lo, const float* x_gain, float* ss_out, hipStream_t stream);
int launch_rmsnorm(const float* x, const float* w, float* y, int rows, int n, float eps,
                   hipStream_t stream);
int launch_rope(float* x, int heads, int hd, int pos, double theta, int rows, int row_stride,
                hipStream_t stream);
int launch_index_of_max(const float* x, int rows, int n, int* out, hipStream_t stream);
int launch_f32_to_bf16(const float* src, uint16_t* dst, size_t n, hipStream_t stream);
int launch_fill_i32(int* dst, int value, size_t n, hipStream_t stream);

// Token sampling (sample.hip): AR_SAMPLE_TOKEN = AutoregressiveModel.sampleToken(logits, V,
// temperature, top_p, random), AR_SAMPLE_MODEL = the sample function of AutoregressiveModel.of.
// Each of `rows` rows draws once from its java.util.Random state rng[row] (advanced in place);
// with `state` set (the model's loop state) nothing is drawn unless the next step is past the
// prompt.  The drawn index goes to out[row] and/or to keys[row * keys_stride] as a key above
// every greedy key (step_begin feeds it).  `work` holds sample_workspace_bytes(rows, vocab).
struct SampleLaunch {
    const float* logits = nullptr;
    int logits_stride = 0, rows = 0, vocab = 0;
    int mode = AR_SAMPLE_MODEL;
    double temperature = 0.0, top_p = 1.0;
    void* work = nullptr;
    unsigned long long* rng = nullptr;
    const int* state = nullptr;
    unsigned long long* keys = nullptr;
    int keys_stride = 0;
    int* out = nullptr;
};
bool sample_is_greedy(int mode, double temperature);
size_t sample_workspace_bytes(int rows, int vocab);
// Zeroes the part of the workspace that must start at zero (row histograms, arrival counters);
// launches keep it zero afterwards, so a workspace used with one (rows, vocab) is cleared once.
int sample_workspace_clear(void* work, int rows, int vocab, hipStream_t stream);
int launch_sample(const SampleLaunch& s, hipStream_t stream);

void ar_ops_release(ar_hip_ctx* ctx);
