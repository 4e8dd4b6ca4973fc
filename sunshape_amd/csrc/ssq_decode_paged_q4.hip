// Dispatch of the 4x4-MFMA paged decode kernel (ssq_decode_paged_q4.h) over its instantiation units.
#include "ssq_decode_paged_q4.h"

// Shapes this kernel serves (the caller has checked the layout -- 16-token pages, or contiguous rows
// at head_dim 128 with 128-dim values --, bf16/f16 V, alignment, code widths 0/4/6/8, and that masks
// and passthrough blocks (at most 16 dims) come with byte codes): head_dim 64 or 128, block_dim 1, 2,
// 4 or 8 with at most 64 blocks, value_dim 64 or 128, at most 256 codewords.
bool ssq_decode_q4_shape(const ssq_decode_args* a) {
    if (a->head_dim != 64 && a->head_dim != 128) return false;
    const int bd = a->block_dim;
    if (bd != 1 && bd != 2 && bd != 4 && bd != 8) return false;
    if (a->head_dim / bd > 64) return false;
    if (a->value_dim != 64 && a->value_dim != 128) return false;
    return a->n_centroids >= 1 && a->n_centroids <= kNC;
}

// LDS bytes for rg query rows per group and split_len tokens per split
size_t ssq_decode_q4_smem(const ssq_decode_args* a, int rg, int split_len) {
    return q4_smem(*a, 4 * ((rg + 3) / 4), split_len, SSQ_Q4_WAVES);
}

// Launches the 4x4-MFMA kernel for a planned problem (grid: batch*KV heads, splits, row groups);
// mp.rg rows per group (<= 16).  The caller launches the split merge.
int ssq_decode_q4_launch(const SsqPagedParams& mp, const dim3& grid, hipStream_t st) {
    const int R4 = (mp.rg + 3) / 4;
    const int DT = mp.a.value_dim / 16;
    const size_t smem = 0;  // launch_q4 sizes the LDS for its wave count
    const bool bf = mp.a.v_dtype == SSQ_BF16;
    const bool packed = mp.a.code_bits == 4 || mp.a.code_bits == 6;
    const bool mixed = mp.a.mask != nullptr || mp.a.heavy_mask[0] != 0;  // byte codes (the plan checks)
    if (mixed && (packed || mp.a.heavy_mask[1] != 0))
        return ssq_fail(SSQ_ERR_UNSUPPORTED, "4x4-MFMA decode: masks and passthrough need byte codes, blocks < 64");
    if (mp.a.layout == SSQ_CONTIGUOUS) {  // contiguous rows: head_dim 128, 128-dim values
        if (mp.a.head_dim != 128) return ssq_fail(SSQ_ERR_UNSUPPORTED, "4x4-MFMA decode: contiguous rows at head_dim %d",
                                                  mp.a.head_dim);
        if (mixed) return bf ? ssq_q4ct_128_bf16_mixed(mp, R4, DT, grid, smem, st) : ssq_q4ct_128_f16_mixed(mp, R4, DT, grid, smem, st);
        if (bf) return packed ? ssq_q4ct_128_bf16_packed(mp, R4, DT, grid, smem, st) : ssq_q4ct_128_bf16_bytes(mp, R4, DT, grid, smem, st);
        return packed ? ssq_q4ct_128_f16_packed(mp, R4, DT, grid, smem, st) : ssq_q4ct_128_f16_bytes(mp, R4, DT, grid, smem, st);
    }
    if (mixed) {
        if (mp.a.head_dim == 64)
            return bf ? ssq_q4_64_bf16_mixed(mp, R4, DT, grid, smem, st) : ssq_q4_64_f16_mixed(mp, R4, DT, grid, smem, st);
        return bf ? ssq_q4_128_bf16_mixed(mp, R4, DT, grid, smem, st) : ssq_q4_128_f16_mixed(mp, R4, DT, grid, smem, st);
    }
    if (mp.a.head_dim == 64) {
        if (bf) return packed ? ssq_q4_64_bf16_packed(mp, R4, DT, grid, smem, st) : ssq_q4_64_bf16_bytes(mp, R4, DT, grid, smem, st);
        return packed ? ssq_q4_64_f16_packed(mp, R4, DT, grid, smem, st) : ssq_q4_64_f16_bytes(mp, R4, DT, grid, smem, st);
    }
    if (bf) return packed ? ssq_q4_128_bf16_packed(mp, R4, DT, grid, smem, st) : ssq_q4_128_bf16_bytes(mp, R4, DT, grid, smem, st);
    return packed ? ssq_q4_128_f16_packed(mp, R4, DT, grid, smem, st) : ssq_q4_128_f16_bytes(mp, R4, DT, grid, smem, st);
}
