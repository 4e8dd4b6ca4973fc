// Instantiations of the paged LUT decode kernel (ssq_decode_mfma.h), one unit of several that
// compile in parallel.
#include "ssq_decode_mfma.h"

SSQ_MFMA_UNIT(ssq_mfma_lut_rp4) {
    return launch_vt<4>(mp, pl, st);
}
