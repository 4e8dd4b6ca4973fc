// Host side of the contiguous-layout decode (kernel: ssq_decode_contig.h): which problems it
// serves, the launch plan, and dispatch over the instantiation units.
#include "ssq_decode_contig.h"

int ssq_launch_merge(const ssq_decode_args& a, int n_splits, const float* ws_o, const float* ws_m,
                     const float* ws_l, hipStream_t st);

namespace {

// passthrough dims of the heavy blocks, blocks ascending then d: the token record element and
// the permuted head dim of each (n_hd of them), and whether they are 8 contiguous 16-bit
// elements from slot 0 in 16-byte aligned rows (the one-load variant)
struct PtLayout {
    int n_hd = 0, vec = 0;
    int hoff[kHP] = {}, hdim[kHP] = {};
};
PtLayout pt_layout(const ssq_decode_args& a) {
    PtLayout L;
    for (int blk = 0, h = 0; blk < a.n_blocks && blk < 64; ++blk) {
        if (!((a.heavy_mask[0] >> blk) & 1ull)) continue;
        const int slot = a.pt_dense ? blk : h;  // record slot = block (dense) or ordinal
        for (int d = 0; d < a.block_dim && L.n_hd < kHP; ++d) {
            L.hoff[L.n_hd] = slot * a.block_dim + d;
            L.hdim[L.n_hd] = blk * a.block_dim + d;
            ++L.n_hd;
        }
        ++h;
    }
    for (int i = L.n_hd; i < kHP; ++i) L.hoff[i] = L.hoff[0];  // loaded, then zeroed in the kernel
    if (L.n_hd == 8 && (a.pt_dtype == SSQ_BF16 || a.pt_dtype == SSQ_F16) && (uintptr_t)a.pt % 16 == 0 &&
        (a.pt_sb * 2) % 16 == 0 && (a.pt_sh * 2) % 16 == 0 && (a.pt_st * 2) % 16 == 0) {
        L.vec = 1;
        for (int i = 0; i < 8; ++i) L.vec &= L.hoff[i] == i ? 1 : 0;
    }
    return L;
}

bool plan(const ssq_decode_args* a, bool has_v, SsqContigPlan& pl) {
    if (a->layout != SSQ_CONTIGUOUS) return false;
    // packed codes: words of 1-7-bit codes are unpacked in the kernel (4 and 6 bits at compile
    // time, other widths at run time; without passthrough or mask); 8-bit words are byte rows
    // (strides scaled to bytes)
    const int cbits = a->code_bits;
    if (cbits < 0 || cbits > 8) return false;
    if (cbits > 0 && cbits < 8 && (a->heavy_mask[0] || a->mask)) return false;
    if (!has_v && a->mask) return false;  // scores only: the reference's score kernels take no mask
    if (a->heavy_mask[1]) return false;
    if (a->heavy_mask[0]) {
        const int n_hd = __builtin_popcountll(a->heavy_mask[0]) * a->block_dim;
        if (n_hd > kHP || !a->pt || a->pt_dtype < SSQ_F32 || a->pt_dtype > SSQ_F16) return false;
    }
    if (a->head_dim != kD) return false;
    const int bd = a->block_dim;
    if (bd != 1 && bd != 2 && bd != 4 && bd != 8) return false;
    if (a->n_centroids > 256) return false;
    const int rows = (a->num_q_heads / a->num_kv_heads) * a->q_len;
    if (rows > 16) return false;
    if ((uintptr_t)a->cent % 16 || (a->cent_sh * 4) % 16) return false;
    const int nb = a->n_blocks;
    if (cbits > 0 && cbits < 8) {  // word loads
        if ((uintptr_t)a->codes % 4) return false;
    } else {
        const int cal = nb >= 16 ? 16 : 8;  // code row loads of 16 (or 8) bytes
        const int64_t cs = cbits == 8 ? 4 : 1;  // stride unit in bytes
        if ((uintptr_t)a->codes % cal || (a->c_st * cs) % cal || (a->c_sh * cs) % cal || (a->c_sb * cs) % cal)
            return false;
    }
    // tile loads take 32-bit offsets from the tile's first token: a tile must span < 2^31 elements,
    // with non-negative token strides
    const int64_t kLim = (int64_t)1 << 31;
    if (a->c_st < 0 || (has_v && a->v_st < 0) || (a->heavy_mask[0] && a->pt_st < 0)) return false;
    if ((int64_t)kTile * a->c_st * (cbits == 8 ? 4 : 1) + 64 >= kLim) return false;
    if (has_v && (int64_t)kTile * a->v_st + a->value_dim >= kLim) return false;
    if (a->heavy_mask[0] && (int64_t)kTile * a->pt_st + 64 >= kLim) return false;
    pl.DT = 4;
    if (has_v) {
        if (a->v_dtype != SSQ_BF16 && a->v_dtype != SSQ_F16) return false;
        if (a->value_dim != 64 && a->value_dim != 128) return false;
        if ((uintptr_t)a->v % 16 || (a->v_sb * 2) % 16 || (a->v_sh * 2) % 16 || (a->v_st * 2) % 16) return false;
        pl.DT = a->value_dim / 16;
    }
    pl.r4 = rows <= 4 ? 1 : rows <= 8 ? 2 : 4;
    const PtLayout L = pt_layout(*a);
    const int hv = L.n_hd == 0 ? 0 : L.vec && !a->mask ? 2 : 1;  // the kernel's passthrough variant
    pl.waves = contig_waves(pl.DT, hv, has_v && a->mask, pl.r4);
    pl.smem = contig_smem(*a, pl.DT, pl.waves);
    if (pl.smem > kMaxSmem) return false;
    const int units = a->batch * a->num_kv_heads;
    const int tiles = (a->seq_len + kTile - 1) / kTile;
    const int cus = ssq_device_cus();
    int splits = a->num_splits > 0 ? a->num_splits : (cus + units - 1) / units;
    const int max_splits = (tiles + pl.waves - 1) / pl.waves;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    const int tiles_per_split = (tiles + splits - 1) / splits;
    pl.split_len = tiles_per_split * kTile;
    pl.n_splits = (a->seq_len + pl.split_len - 1) / pl.split_len;
    if (pl.n_splits < 1) pl.n_splits = 1;
    const size_t n_rows_all = (size_t)a->batch * a->num_q_heads * a->q_len;
    pl.ws_bytes = (has_v && pl.n_splits > 1) ? (size_t)pl.n_splits * n_rows_all * (a->value_dim + 2) * 4 : 0;
    return true;
}

int dispatch(const SsqContigParams& cp, const SsqContigPlan& pl, hipStream_t st) {
    const bool mixed = cp.n_hd > 0;
    if (!cp.a.v) return mixed ? ssq_contig_scores_mixed(cp, pl, st) : ssq_contig_scores_plain(cp, pl, st);
    const bool bf = cp.a.v_dtype == SSQ_BF16;
    if (pl.DT == 4) {
        if (bf) return mixed ? ssq_contig_64_bf16_mixed(cp, pl, st) : ssq_contig_64_bf16_plain(cp, pl, st);
        return mixed ? ssq_contig_64_f16_mixed(cp, pl, st) : ssq_contig_64_f16_plain(cp, pl, st);
    }
    if (bf) return mixed ? ssq_contig_128_bf16_mixed(cp, pl, st) : ssq_contig_128_bf16_plain(cp, pl, st);
    return mixed ? ssq_contig_128_f16_mixed(cp, pl, st) : ssq_contig_128_f16_plain(cp, pl, st);
}

}  // namespace

int ssq_decode_contig_supported(const ssq_decode_args* a) {
    SsqContigPlan pl;
    return plan(a, a->v != nullptr, pl) ? 1 : 0;
}

size_t ssq_decode_contig_workspace(const ssq_decode_args* a) {
    SsqContigPlan pl;
    return plan(a, a->v != nullptr, pl) ? pl.ws_bytes : 0;
}

// decode (a->v != NULL) or scores only (a->v == NULL, a->scores != NULL)
int ssq_decode_contig(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st) {
    const bool has_v = a->v != nullptr;
    SsqContigPlan pl;
    if (!plan(a, has_v, pl)) return ssq_fail(SSQ_ERR_UNSUPPORTED, "contiguous MFMA kernel does not support this problem");
    if (a->seq_len == 0) {
        if (!has_v) return SSQ_OK;
        return ssq_fail(SSQ_ERR_INVALID, "seq_len == 0: softmax over an empty context");
    }
    SSQ_REQUIRE(ws_bytes >= pl.ws_bytes, "workspace too small: %zu < %zu bytes", ws_bytes, pl.ws_bytes);
    SSQ_REQUIRE(pl.ws_bytes == 0 || workspace, "workspace is NULL");
    SsqContigParams cp;
    cp.a = *a;
    if (a->code_bits == 8) {  // 8-bit words are the byte rows: byte strides, the byte-code path
        cp.a.c_sb *= 4; cp.a.c_sh *= 4; cp.a.c_st *= 4;
        cp.a.code_bits = 0;
    }
    if (cp.a.code_bits > 0) {  // packing of the word rows (used by the run-time-width variants)
        const uint32_t bits = (uint32_t)cp.a.code_bits, vpe = 32u / bits;
        cp.pk = SsqPackFmt{bits, vpe, (65536u + vpe - 1u) / vpe, ((uint32_t)a->n_blocks + vpe - 1u) / vpe};
    } else {
        cp.pk = SsqPackFmt{8u, 4u, 16384u, 1u};
    }
    cp.G = a->num_q_heads / a->num_kv_heads;
    cp.rows = cp.G * a->q_len;
    cp.split_len = pl.split_len;
    cp.n_splits = pl.n_splits;
    const size_t n_rows_all = (size_t)a->batch * a->num_q_heads * a->q_len;
    float* ws = reinterpret_cast<float*>(workspace);
    cp.ws_o = ws;
    cp.ws_m = ws ? ws + (size_t)pl.n_splits * n_rows_all * a->value_dim : nullptr;
    cp.ws_l = ws ? cp.ws_m + (size_t)pl.n_splits * n_rows_all : nullptr;
    // passthrough dims: heavy blocks ascending, then d; record slot = block (dense) or ordinal
    const PtLayout L = pt_layout(*a);
    cp.n_hd = L.n_hd;
    cp.pt_vec = L.vec;
    for (int i = 0; i < kHP; ++i) { cp.hoff[i] = L.hoff[i]; cp.hdim[i] = L.hdim[i]; }
    const int rc = dispatch(cp, pl, st);
    if (rc) return rc;
    if (has_v && pl.n_splits > 1) return ssq_launch_merge(*a, pl.n_splits, cp.ws_o, cp.ws_m, cp.ws_l, st);
    return SSQ_OK;
}
