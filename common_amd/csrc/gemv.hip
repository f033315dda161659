// Host side of the decode GEMV: argument checks and launch shape.
#include "gemv_impl.h"

int launch_gemv(const GemvLaunch& a, hipStream_t stream) {
    AR_CHECK_ARG(a.w && a.x, "GEMV: null weight or input");
    AR_CHECK_ARG(a.rows > 0 && a.cols > 0, "GEMV: empty shape %dx%d", a.rows, a.cols);
    AR_CHECK_ARG(a.batch >= 1 && a.batch <= 8, "GEMV: batch %d outside 1..8", a.batch);
    AR_CHECK_ARG(a.cols % 8 == 0, "GEMV: cols %d must be a multiple of 8", a.cols);
    AR_CHECK_ARG(a.x_stride % 4 == 0 && a.x_stride >= a.cols, "GEMV: bad input stride %d", a.x_stride);
    AR_CHECK_ARG((reinterpret_cast<uintptr_t>(a.w) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0,
                 "GEMV: weight and input must be 16-byte aligned");
    AR_CHECK_ARG(!a.norm_w || (reinterpret_cast<uintptr_t>(a.norm_w) & 15) == 0, "GEMV: norm gain not aligned");
    AR_CHECK_ARG(a.wdtype == AR_DTYPE_F32 || a.wdtype == AR_DTYPE_BF16, "GEMV: unknown weight dtype %d", a.wdtype);
    if (a.epilogue == GEMV_EPI_SWIGLU)
        AR_CHECK_ARG(a.w2 && (reinterpret_cast<uintptr_t>(a.w2) & 15) == 0, "GEMV: SwiGLU needs an aligned up matrix");
    if (a.epilogue == GEMV_EPI_ARGMAX) {
        AR_CHECK_ARG(a.keys, "GEMV argmax: missing key buffer");
        AR_CHECK_ARG(!a.y || a.y_stride >= a.rows, "GEMV argmax: short logits stride");
    } else {
        AR_CHECK_ARG(a.y && a.y_stride >= a.rows, "GEMV: null output or short stride");
    }
    if (ar_check_ptrs_enabled()) {  // extents the kernels read and write
        const char* k = "GEMV";
        const size_t wb = a.wdtype == AR_DTYPE_BF16 ? 2 : 4, R = a.rows, Cn = a.cols, B1 = a.batch - 1;
        AR_TRY(ar_check_range(a.w, R * Cn * wb, k, "weights"));
        AR_TRY(ar_check_range(a.w2, R * Cn * wb, k, "up weights"));
        AR_TRY(ar_check_range(a.x, (B1 * a.x_stride + Cn) * 4, k, "input"));
        AR_TRY(ar_check_range(a.norm_w, Cn * 4, k, "norm gain"));
        AR_TRY(ar_check_range(a.bias, R * 4, k, "bias"));
        AR_TRY(ar_check_range(a.y, (B1 * a.y_stride + R) * 4, k, "output"));
        AR_TRY(ar_check_range(a.keys, (B1 + 1) * kArgmaxSlots * 8, k, "argmax keys"));
        AR_TRY(ar_check_range(a.x_hi, (B1 * a.x_stride + Cn) * 2, k, "input hi plane"));
        AR_TRY(ar_check_range(a.x_lo, (B1 * a.x_stride + Cn) * 2, k, "input lo plane"));
        AR_TRY(ar_check_range(a.y_hi, (B1 * a.y_stride + R) * 2, k, "output hi plane"));
        AR_TRY(ar_check_range(a.y_lo, (B1 * a.y_stride + R) * 2, k, "output lo plane"));
        AR_TRY(ar_check_range(a.y_gain, R * 4, k, "output plane gain"));
        AR_TRY(ar_check_range(a.kpart, (size_t)a.kpart_floats * 4, k, "k-split partials"));
        AR_TRY(ar_check_range(a.kcount, (size_t)a.kcount_n * 4, k, "k-split counters"));
        AR_TRY(ar_check_range(a.w_frag, gemv_frag_elems(a.rows, a.cols) * 2, k, "fragment-ordered weights"));
        AR_TRY(ar_check_range(a.w2_frag, gemv_frag_elems(a.rows, a.cols) * 2, k, "fragment-ordered up weights"));
        AR_TRY(ar_check_range(a.ss_in, (size_t)((Cn + 15) / 16) * 16 * 4, k, "input sums of squares"));
        AR_TRY(ar_check_range(a.ss_out, (size_t)((R + 15) / 16) * 16 * 4, k, "output sums of squares"));
    }
    gemv::Params p;
    p.w = a.w; p.w2 = a.w2; p.rows = a.rows; p.cols = a.cols; p.batch = a.batch;
    p.x = a.x; p.x_stride = a.x_stride; p.norm_w = a.norm_w; p.eps = a.eps; p.bias = a.bias;
    p.y = a.y; p.y_stride = a.y_stride; p.keys = a.keys;
    p.x_hi = a.x_hi; p.x_lo = a.x_lo; p.y_hi = a.y_hi; p.y_lo = a.y_lo; p.y_gain = a.y_gain;
    p.kpart = a.kpart; p.kpart_floats = a.kpart_floats; p.kcount = a.kcount; p.kcount_n = a.kcount_n;
    p.wf = a.w_frag; p.wf2 = a.w2_frag; p.ss_in = a.ss_in; p.ss_out = a.ss_out;
    AR_CHECK_ARG(!a.kpart == !a.kcount, "GEMV: k-split workspace needs both partials and counters");
    const bool mfma = a.batch >= 3 && a.wdtype == AR_DTYPE_BF16 && a.cols % 32 == 0;
    AR_CHECK_ARG(mfma || (!a.x_hi && !a.y_hi), "GEMV: operand planes need the MFMA path (batch >= 3, bf16, cols %% 32)");
    AR_CHECK_ARG(!a.x_hi == !a.x_lo && !a.y_hi == !a.y_lo, "GEMV: operand planes come in hi/lo pairs");
    AR_CHECK_ARG(!a.y_hi || a.epilogue != GEMV_EPI_ARGMAX, "GEMV: no output planes for the argmax epilogue");
    if (a.w_frag) {
        AR_CHECK_ARG(a.wdtype == AR_DTYPE_BF16, "GEMV: fragment-ordered weights are bf16");
        return gemv_launch_frag(p, a.epilogue, stream);
    }
    AR_CHECK_ARG(!a.ss_in && !a.ss_out, "GEMV: per-tile sums of squares need the fragment-ordered form");
    if (mfma) return gemv_launch_mfma(p, a.epilogue, stream);
    if (a.batch >= 3) return gemv_launch_batched(p, a.wdtype, a.epilogue, stream);
    if (a.epilogue == GEMV_EPI_ARGMAX && gemv_argmax_fits(a.cols, a.batch, a.wdtype) && a.x_stride % 4 == 0)
        return gemv_launch_argmax(p, a.wdtype, stream);
    if (gemv_rx_fits(a.rows, a.cols, a.batch, a.wdtype, a.epilogue, a.norm_w != nullptr) && (a.cols * 4) % 16 == 0)
        return gemv_launch_rx(p, a.wdtype, a.epilogue, stream);
    const gemv::Shape s = gemv::shape_for(a.rows, a.cols, a.batch, a.wdtype, a.epilogue);
    if (a.wdtype == AR_DTYPE_F32) return gemv_launch_f32(p, a.epilogue, s, stream);
    return gemv_launch_bf16(p, a.epilogue, s, stream);
}

