// 4x4-MFMA paged decode instantiations: head_dim 64, bf16 values, byte codes, with an additive
// mask and / or passthrough blocks.
#include "ssq_decode_paged_q4.h"

SSQ_Q4_UNIT(ssq_q4_64_bf16_mixed) {
    return q4_dispatch_mixed<64, SSQ_BF16, false>(mp, R4, DT, grid, smem, st);
}
