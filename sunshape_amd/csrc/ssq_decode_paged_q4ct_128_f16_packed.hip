// 4x4-MFMA decode instantiations over contiguous rows: head_dim 128, f16 values, 4- and 6-bit
// packed codes.
#include "ssq_decode_paged_q4.h"

SSQ_Q4_UNIT(ssq_q4ct_128_f16_packed) {
    return mp.a.code_bits == 4 ? q4_dispatch<128, SSQ_F16, 4, true>(mp, R4, DT, grid, smem, st)
                               : q4_dispatch<128, SSQ_F16, 6, true>(mp, R4, DT, grid, smem, st);
}
