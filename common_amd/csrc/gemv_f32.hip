// fp32-weight instantiations of the decode GEMV (kernel in gemv_impl.h).
#include "gemv_impl.h"

int gemv_launch_f32(const gemv::Params& p, int epi, const gemv::Shape& s, hipStream_t st) {
    return gemv::dispatch_epi<float>(p, epi, s, st);
}
