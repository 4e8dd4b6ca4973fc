// 4x4-MFMA decode instantiations over contiguous rows: head_dim 128, f16 values, byte codes.
#include "ssq_decode_paged_q4.h"

SSQ_Q4_UNIT(ssq_q4ct_128_f16_bytes) {
    return q4_dispatch<128, SSQ_F16, 0, true>(mp, R4, DT, grid, smem, st);
}
