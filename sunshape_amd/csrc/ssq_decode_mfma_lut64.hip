// Instantiations of the paged LUT decode kernel (ssq_decode_mfma.h), one unit of several that
// compile in parallel.
#include "ssq_decode_mfma.h"

SSQ_MFMA_UNIT(ssq_mfma_lut64) {
    return mp.a.code_bits == 6 ? lut64_rp<6>(mp, pl, st) : lut64_rp<0>(mp, pl, st);
}
