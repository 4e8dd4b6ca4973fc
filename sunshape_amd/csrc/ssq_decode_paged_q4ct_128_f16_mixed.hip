// 4x4-MFMA decode instantiations over contiguous rows: head_dim 128, f16 values, byte codes, with
// an additive mask and / or passthrough blocks.
#include "ssq_decode_paged_q4.h"

SSQ_Q4_UNIT(ssq_q4ct_128_f16_mixed) {
    return q4_dispatch_mixed<128, SSQ_F16, true>(mp, R4, DT, grid, smem, st);
}
