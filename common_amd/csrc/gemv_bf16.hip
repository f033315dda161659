// bf16-weight instantiations of the decode GEMV (kernel in gemv_impl.h); fp32 accumulation.
#include "gemv_impl.h"

int gemv_launch_bf16(const gemv::Params& p, int epi, const gemv::Shape& s, hipStream_t st) {
    return gemv::dispatch_epi<uint16_t>(p, epi, s, st);
}
