// Instantiations of the paged LUT decode kernel (ssq_decode_mfma.h), one unit of several that
// compile in parallel.
#include "ssq_decode_mfma.h"

SSQ_MFMA_UNIT(ssq_mfma_lut_rp2) {
    return launch_vt<2>(mp, pl, st);
}
