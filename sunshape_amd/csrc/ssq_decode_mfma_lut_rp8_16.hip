// Instantiations of the paged LUT decode kernel (ssq_decode_mfma.h), one unit of several that
// compile in parallel.
#include "ssq_decode_mfma.h"

SSQ_MFMA_UNIT(ssq_mfma_lut_rp8_16) {
    return pl.RP == 8 ? launch_vt<8>(mp, pl, st) : launch_vt<16>(mp, pl, st);
}
