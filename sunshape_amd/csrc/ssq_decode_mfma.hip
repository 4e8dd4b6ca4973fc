// Host side of the paged LUT decode (kernel: ssq_decode_mfma.h): which problems it serves, the
// launch plan, and dispatch over the instantiation units.
#include "ssq_decode_mfma.h"

int ssq_launch_merge(const ssq_decode_args& a, int n_splits, const float* ws_o, const float* ws_m,
                     const float* ws_l, hipStream_t st);
// the 4x4-MFMA-scores kernel (ssq_decode_paged_q4.hip)
bool ssq_decode_q4_shape(const ssq_decode_args* a);
size_t ssq_decode_q4_smem(const ssq_decode_args* a, int rg, int split_len);
int ssq_decode_q4_launch(const SsqPagedParams& mp, const dim3& grid, hipStream_t st);

namespace {

int pow2_at_least(int x) {
    int q = 1;
    while (q < x) q <<= 1;
    return q;
}

// the 64-codeword LUT kernel's instantiations
bool lut64_shape(const ssq_decode_args& a, int RP, int DT) {
    return a.v_dtype == SSQ_BF16 && (DT == 4 || DT == 8) && (RP == 2 || RP == 4 || RP == 8) &&
           (a.n_blocks == 16 || a.n_blocks == 32 || a.n_blocks == 64);
}

// passthrough dims (heavy blocks ascending, then d): record slot = block (dense) or ordinal; pt_vec
// when they are 8 or 16 consecutive 16-bit values with 16-byte aligned rows
void pt_dims(const ssq_decode_args& a, SsqPagedParams& mp) {
    mp.n_hd = 0;
    for (int i = 0; i < 16; ++i) mp.hoff[i] = mp.hdim[i] = 0;  // entries past n_hd: dim 0, never an index past D
    for (int blk = 0, h = 0; blk < a.n_blocks && blk < 64; ++blk) {
        if (!((a.heavy_mask[0] >> blk) & 1ull)) continue;
        const int slot = a.pt_dense ? blk : h;
        for (int d = 0; d < a.block_dim && mp.n_hd < 16; ++d) {
            mp.hoff[mp.n_hd] = slot * a.block_dim + d;
            mp.hdim[mp.n_hd] = blk * a.block_dim + d;
            ++mp.n_hd;
        }
        ++h;
    }
    mp.pt_vec = a.heavy_mask[0] && a.pt_dtype != SSQ_F32 && (mp.n_hd == 8 || mp.n_hd == 16) &&
                ((uintptr_t)a.pt + 2 * (uintptr_t)mp.hoff[0]) % 16 == 0 && (a.pt_sb * 2) % 16 == 0 &&
                (a.pt_sh * 2) % 16 == 0 && (a.pt_st * 2) % 16 == 0;
    for (int i = 1; i < mp.n_hd; ++i) mp.pt_vec = mp.pt_vec && mp.hoff[i] == mp.hoff[0] + i;
}

bool plan(const ssq_decode_args* a, SsqMfmaPlan& pl) {
    // contiguous rows take the LUT kernel (CT) for 128-dim values past head_dim 64, which the
    // contiguous MFMA kernel (ssq_decode_contig.hip) serves, and the 4x4-MFMA-scores kernel (CT) at
    // head_dim 128 where the LUT would need row groups
    const bool ct = a->layout == SSQ_CONTIGUOUS;
    if (!ct && (a->layout != SSQ_PAGED || a->page_size != kPage)) return false;
    // Codes: bytes, 8-bit words (the byte rows, strides scaled to bytes), or 4- / 6-bit words.
    // The LUT kernel serves 256-codeword codebooks with byte codes, and 64-codeword codebooks
    // with byte or 6-bit codes (bf16 V, 2-8 rows, 16-64 blocks: lut64_shape); the 4x4-MFMA-scores
    // kernel serves the rest of its shapes.  Other widths take the generic kernel.
    const int cbits = a->code_bits;
    if (cbits != 0 && cbits != 4 && cbits != 6 && cbits != 8) return false;
    if (a->n_centroids > kNC) return false;
    // scores only (no values, no mask): contiguous rows
    const bool nv = a->v == nullptr;
    if (nv && (!ct || !a->scores || a->mask)) return false;
    if (!nv && a->v_dtype != SSQ_BF16 && a->v_dtype != SSQ_F16) return false;
    // Passthrough blocks (decode, <= 16 dims among the first 64 blocks) and additive masks: the
    // contiguous LUT kernel takes passthrough as 8 or 16 consecutive 16-bit values per token without a
    // mask, and masks without passthrough; the 4x4-MFMA-scores kernel takes both, in any layout, with
    // byte codes, on pages and on contiguous rows.
    const bool heavy = a->heavy_mask[0] || a->heavy_mask[1];
    const bool masked = a->mask != nullptr;
    SsqPagedParams dims;
    pt_dims(*a, dims);
    if (heavy) {
        if (nv || a->heavy_mask[1] || !a->pt) return false;
        if (a->pt_dtype != SSQ_F32 && a->pt_dtype != SSQ_BF16 && a->pt_dtype != SSQ_F16) return false;
        if (__builtin_popcountll(a->heavy_mask[0]) * a->block_dim > 16) return false;
    }
    const bool mixed_bytes = !(heavy || masked) || cbits == 0 || cbits == 8;  // q4 masks / passthrough
    if (!nv && a->value_dim != 64 && a->value_dim != 128 && a->value_dim != 256) return false;
    if ((uintptr_t)a->cent % 16 || (a->cent_sh * 4) % 16) return false;  // float4 codeword loads
    if (a->n_blocks != 8 && a->n_blocks != 16 && a->n_blocks != 32 && a->n_blocks != 64) return false;
    if (a->head_dim > 256) return false;  // query staging covers at most 256 dims per row
    // contiguous rows: the LUT kernel (CT) or the 4x4-MFMA-scores kernel (CT; head_dim 128, 128-dim
    // values, no mask, no passthrough, not scores only)
    const bool ct_lut = ct && a->head_dim != 64 && (nv || a->value_dim == 128) && a->kernel != 4 &&
                        a->n_centroids == kNC && (cbits == 0 || cbits == 8) && (!heavy || (dims.pt_vec && !masked));
    const bool ct_q4 = ct && !nv && mixed_bytes && a->head_dim == 128 && a->value_dim == 128 && ssq_decode_q4_shape(a);
    if (ct) {
        if (!ct_lut && !ct_q4) return false;
        // tile loads take 32-bit byte offsets from the tile's first token, token strides >= 0
        const int64_t kLim = (int64_t)1 << 31;
        if (a->c_st < 0 || (!nv && a->v_st < 0)) return false;
        if ((int64_t)kTileTok * a->c_st * (cbits ? 4 : 1) + 64 >= kLim) return false;
        if (!nv && (int64_t)kTileTok * 2 * a->v_st + 256 >= kLim) return false;
    }
    if (cbits == 4 || cbits == 6) {  // word loads
        if ((uintptr_t)a->codes % 4) return false;
    } else {  // code rows: 8-byte (nb 8) or 16-byte (nb >= 16) vector loads
        const int cal = a->n_blocks >= 16 ? 16 : 8;
        const int64_t cs = cbits == 8 ? 4 : 1;  // stride unit in bytes
        if ((a->c_st * cs) % cal || (a->c_sb * cs) % cal || (a->c_sh * cs) % cal || (uintptr_t)a->codes % cal)
            return false;
    }
    if (!nv && ((uintptr_t)a->v % 16 || (a->v_sb * 2) % 16 || (a->v_sh * 2) % 16 || (a->v_st * 2) % 16)) return false;
    // Query rows of one (batch, KV head) share a LUT of n_blocks x nc x RP fp32 (<= 128 KiB).
    // More rows than one LUT holds split into row groups, each streaming the codes and values
    // again: twice the bytes at 8 query heads per KV head with 32 blocks, far less than the
    // LUT-less generic kernel costs.
    // Contiguous rows take long causal chunks too (up to 2048 rows, e.g. 512 new tokens at 4 query
    // heads per KV head): every row group re-streams the cache, as in the generic kernel's groups
    // of 8, but at this kernel's rate.
    const int rows = (a->num_q_heads / a->num_kv_heads) * a->q_len;
    if (rows > (ct ? 2048 : 64)) return false;
    const int lcap = 32768 / (a->n_blocks * lut_nc(*a));  // rows per 128 KiB LUT, a power of two
    const int rcap = ct ? 8 : 16;  // contiguous: the V buffer leaves room for 8-row LUTs
    const int cap = lcap < rcap ? lcap : rcap;
    pl.rg = rows < cap ? rows : cap;
    pl.n_groups = (rows + pl.rg - 1) / pl.rg;
    pl.RP = pow2_at_least(pl.rg);
    pl.DT = nv ? 8 : a->value_dim / 16;
    const bool lut_ok = ct ? ct_lut
                           : heavy || masked ? false  // pages: masks and passthrough take the 4x4-MFMA kernel
                           : a->n_centroids == kNC ? cbits == 0 || cbits == 8
                                                   : a->n_centroids == 64 && cbits != 4 && lut64_shape(*a, pl.RP, pl.DT);
    // Where the LUT needs row groups (or cannot serve the codes), the 4x4-MFMA-scores kernel serves
    // up to 16 rows per pass over the pages or rows instead (its codebook is head_dim x nc fp32
    // whatever the block size); kernel 4 asks for it wherever it applies
    const bool q4_ok = ct ? ct_q4 : mixed_bytes && ssq_decode_q4_shape(a);
    if (a->kernel == 4 && !q4_ok) return false;
    if (!lut_ok && !q4_ok) return false;
    pl.ct = ct;
    // Contiguous passthrough blocks at head_dim 128 also take the 4x4-MFMA kernel: its passthrough
    // dims cost one MFMA each where the LUT kernel adds a VALU product per row (config-4 layer with 4
    // bf16 blocks of dim 4: 0.806 against 0.889 ms); kernel 2 still asks for the LUT kernel.
    const bool q4_pt = ct && heavy && a->kernel != 2;
    pl.q4 = q4_ok && (a->kernel == 4 || !lut_ok || pl.n_groups > 1 || q4_pt);
    if (pl.q4) {
        pl.rg = rows < 16 ? rows : 16;
        pl.n_groups = (rows + 15) / 16;
        pl.RP = 4 * ((pl.rg + 3) / 4);
    }
    const int units = a->batch * a->num_kv_heads * pl.n_groups;
    const int tiles = (a->seq_len + kTileTok - 1) / kTileTok;
    const int cus = ssq_device_cus();  // one workgroup per CU (the LUT fills the LDS)
    int splits = a->num_splits > 0 ? a->num_splits : (cus + units - 1) / units;
    const int max_splits = (tiles + kWaves - 1) / kWaves;  // keep every wave busy
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    int tiles_per_split = (tiles + splits - 1) / splits;
    pl.split_len = tiles_per_split * kTileTok;
    // the split's block-table slice lives in LDS too: long contexts split until it fits
    while (tiles_per_split > 1 &&
           (pl.q4 ? ssq_decode_q4_smem(a, pl.rg, pl.split_len) : mfma_smem(*a, pl.RP, pl.split_len, ct)) > kMaxSmem) {
        tiles_per_split = (tiles_per_split + 1) / 2;
        pl.split_len = tiles_per_split * kTileTok;
    }
    pl.n_splits = (a->seq_len + pl.split_len - 1) / pl.split_len;
    if (pl.n_splits < 1) pl.n_splits = 1;
    pl.smem = pl.q4 ? ssq_decode_q4_smem(a, pl.rg, pl.split_len) : mfma_smem(*a, pl.RP, pl.split_len, ct);
    if (pl.smem > kMaxSmem) return false;
    const size_t n_rows_all = (size_t)a->batch * a->num_q_heads * a->q_len;
    pl.ws_bytes = !nv && pl.n_splits > 1 ? (size_t)pl.n_splits * n_rows_all * (a->value_dim + 2) * 4 : 0;
    return true;
}

}  // namespace

int ssq_decode_mfma_supported(const ssq_decode_args* a) {
    SsqMfmaPlan pl;
    return plan(a, pl) ? 1 : 0;
}

size_t ssq_decode_mfma_workspace(const ssq_decode_args* a) {
    SsqMfmaPlan pl;
    return plan(a, pl) ? pl.ws_bytes : 0;
}

int ssq_decode_mfma(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st) {
    SsqMfmaPlan pl;
    if (!plan(a, pl)) return ssq_fail(SSQ_ERR_UNSUPPORTED, "MFMA decode kernel does not support this problem");
    if (a->seq_len == 0) return ssq_fail(SSQ_ERR_INVALID, "seq_len == 0: softmax over an empty context");
    SSQ_REQUIRE(ws_bytes >= pl.ws_bytes, "workspace too small: %zu < %zu bytes", ws_bytes, pl.ws_bytes);
    SSQ_REQUIRE(pl.ws_bytes == 0 || workspace, "workspace is NULL");
    MfmaParams mp{};
    mp.a = *a;
    if (a->code_bits == 8) {  // 8-bit words are the byte rows: byte strides, the byte-code path
        mp.a.c_sb *= 4; mp.a.c_sh *= 4; mp.a.c_st *= 4;
        mp.a.code_bits = 0;
    }
    pt_dims(*a, mp);
    mp.G = a->num_q_heads / a->num_kv_heads;
    mp.rows = mp.G * a->q_len;
    mp.rg = pl.rg;
    mp.split_len = pl.split_len;
    mp.n_splits = pl.n_splits;
    const size_t n_rows_all = (size_t)a->batch * a->num_q_heads * a->q_len;
    float* ws = reinterpret_cast<float*>(workspace);
    mp.ws_o = ws;
    mp.ws_m = ws ? ws + (size_t)pl.n_splits * n_rows_all * a->value_dim : nullptr;
    mp.ws_l = ws ? mp.ws_m + (size_t)pl.n_splits * n_rows_all : nullptr;
    int rc;
    if (pl.q4) {
        rc = ssq_decode_q4_launch(mp, dim3(mp.a.batch * mp.a.num_kv_heads, pl.n_splits, pl.n_groups), st);
        if (rc) return rc;
        if (pl.n_splits > 1) rc = ssq_launch_merge(*a, pl.n_splits, mp.ws_o, mp.ws_m, mp.ws_l, st);
        return rc;
    }
    if (pl.ct && !a->v) return ssq_mfma_lut_ct_scores(mp, pl, st);  // scores only: no merge
    if (pl.ct) {
        if (a->heavy_mask[0])
            rc = a->v_dtype == SSQ_BF16 ? ssq_mfma_lut_ct_bf16_heavy(mp, pl, st) : ssq_mfma_lut_ct_f16_heavy(mp, pl, st);
        else if (a->mask)
            rc = a->v_dtype == SSQ_BF16 ? ssq_mfma_lut_ct_bf16_mask(mp, pl, st) : ssq_mfma_lut_ct_f16_mask(mp, pl, st);
        else
            rc = a->v_dtype == SSQ_BF16 ? ssq_mfma_lut_ct_bf16(mp, pl, st) : ssq_mfma_lut_ct_f16(mp, pl, st);
        if (rc) return rc;
        if (pl.n_splits > 1) rc = ssq_launch_merge(*a, pl.n_splits, mp.ws_o, mp.ws_m, mp.ws_l, st);
        return rc;
    }
    if (mp.a.n_centroids == 64) {
        rc = ssq_mfma_lut64(mp, pl, st);
        if (rc) return rc;
        if (pl.n_splits > 1) rc = ssq_launch_merge(*a, pl.n_splits, mp.ws_o, mp.ws_m, mp.ws_l, st);
        return rc;
    }
    switch (pl.RP) {
        case 1: rc = ssq_mfma_lut_rp1(mp, pl, st); break;
        case 2: rc = ssq_mfma_lut_rp2(mp, pl, st); break;
        case 4: rc = ssq_mfma_lut_rp4(mp, pl, st); break;
        default: rc = ssq_mfma_lut_rp8_16(mp, pl, st); break;
    }
    if (rc) return rc;
    if (pl.n_splits > 1) rc = ssq_launch_merge(*a, pl.n_splits, mp.ws_o, mp.ws_m, mp.ws_l, st);
    return rc;
}
