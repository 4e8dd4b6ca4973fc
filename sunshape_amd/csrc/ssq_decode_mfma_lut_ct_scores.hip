// Instantiations of the LUT kernel over contiguous rows (ssq_decode_mfma.h, CT = true) for scores
// only (NV = true: no values, no softmax), one unit of several that compile in parallel.
#include "ssq_decode_mfma.h"

SSQ_MFMA_UNIT(ssq_mfma_lut_ct_scores) {
    return launch_ct<SSQ_BF16, false, true>(mp, pl, st);
}
