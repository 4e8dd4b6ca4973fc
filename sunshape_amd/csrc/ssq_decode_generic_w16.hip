// Instantiations of the generic decode kernel (ssq_decode_generic.h) for 16-bit codes in 16-byte
// aligned rows, one unit of several that compile in parallel.
#include "ssq_decode_generic.h"

int ssq_generic_w16(const SsqGenericParams& dp, const SsqGenericLaunch& gl, hipStream_t st) {
    return launch_generic<true>(dp, gl, st);
}
