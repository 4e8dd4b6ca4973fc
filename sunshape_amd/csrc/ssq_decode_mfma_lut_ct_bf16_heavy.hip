// Instantiations of the LUT decode kernel over contiguous rows (ssq_decode_mfma.h, CT = true) with
// bf16 values and SunShape-Mixed passthrough blocks, one unit of several that compile in parallel.
#include "ssq_decode_mfma.h"

SSQ_MFMA_UNIT(ssq_mfma_lut_ct_bf16_heavy) {
    return launch_ct<SSQ_BF16, false, false, true>(mp, pl, st);
}
