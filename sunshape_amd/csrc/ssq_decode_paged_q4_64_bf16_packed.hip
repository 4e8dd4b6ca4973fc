// 4x4-MFMA paged decode instantiations: head_dim 64, bf16 values, 4- and 6-bit packed codes.
#include "ssq_decode_paged_q4.h"

SSQ_Q4_UNIT(ssq_q4_64_bf16_packed) {
    return mp.a.code_bits == 4 ? q4_dispatch<64, SSQ_BF16, 4>(mp, R4, DT, grid, smem, st)
                               : q4_dispatch<64, SSQ_BF16, 6>(mp, R4, DT, grid, smem, st);
}
