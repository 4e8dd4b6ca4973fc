// VQ-key decode entry points: argument checks, kernel choice, the generic kernel's plan and
// launch (kernel template in ssq_decode_generic.h), and the split merge shared by the decode kernels.
#include "ssq_decode_generic.h"

namespace {

// Combine split partials: out = sum_s o_s e^{m_s-M} / sum_s l_s e^{m_s-M}, lse = M + log L.
// One wave per query row, kMergeRows rows per workgroup.  Lane j merges value dims j, j + 64, ...;
// every lane loads the row's (m_s, l_s) and its dims' o_s for up to kMergeSplits splits before
// using any of them, so a merge of that many splits costs one memory round trip (more splits take
// further passes, merged online).  No LDS and no workgroup barrier.
constexpr int kMergeRows = 4;
constexpr int kMergeSplits = 16;
constexpr int kMergeDims = 4;  // value dims per lane per pass: 256 per wave

__global__ __launch_bounds__(kMergeRows * SSQ_WAVE) void k_merge(const ssq_decode_args a, int n_splits,
                                                                  const float* ws_o, const float* ws_m,
                                                                  const float* ws_l) {
    const int lane = threadIdx.x & (SSQ_WAVE - 1);
    const int n_rows_all = a.batch * a.num_q_heads * a.q_len;
    const int rid = blockIdx.x * kMergeRows + (int)(threadIdx.x / SSQ_WAVE);
    if (rid >= n_rows_all) return;  // whole waves
    const int qi = rid % a.q_len;
    const int h = (rid / a.q_len) % a.num_q_heads;
    const int b = rid / (a.q_len * a.num_q_heads);
    const int Dv = a.value_dim;
    const size_t mstep = (size_t)n_rows_all;       // between splits in ws_m / ws_l
    const size_t ostep = (size_t)n_rows_all * Dv;  // between splits in ws_o
    float M = -INFINITY, L = 0.f;
    for (int d0 = 0; d0 < Dv; d0 += kMergeDims * SSQ_WAVE) {
        float Mr = -INFINITY, Lr = 0.f;
        float o[kMergeDims];
#pragma unroll
        for (int k = 0; k < kMergeDims; ++k) o[k] = 0.f;
        for (int c0 = 0; c0 < n_splits; c0 += kMergeSplits) {
            float mv[kMergeSplits], lv[kMergeSplits], ov[kMergeSplits][kMergeDims];
#pragma unroll
            for (int i = 0; i < kMergeSplits; ++i) {
                mv[i] = -INFINITY;
                lv[i] = 0.f;
#pragma unroll
                for (int k = 0; k < kMergeDims; ++k) ov[i][k] = 0.f;
                if (c0 + i < n_splits) {  // uniform
                    const size_t s = (size_t)(c0 + i);
                    mv[i] = ws_m[s * mstep + rid];
                    lv[i] = ws_l[s * mstep + rid];
#pragma unroll
                    for (int k = 0; k < kMergeDims; ++k)
                        if (d0 + k * SSQ_WAVE < Dv)  // uniform; the lane's dim is clamped
                            ov[i][k] = ws_o[s * ostep + (size_t)rid * Dv + min(d0 + k * SSQ_WAVE + lane, Dv - 1)];
                }
            }
            float Mc = Mr;
#pragma unroll
            for (int i = 0; i < kMergeSplits; ++i) Mc = fmaxf(Mc, mv[i]);
            const float f = Mr == -INFINITY ? 0.f : __expf(Mr - Mc);  // earlier passes, rescaled
            Lr *= f;
#pragma unroll
            for (int k = 0; k < kMergeDims; ++k) o[k] *= f;
#pragma unroll
            for (int i = 0; i < kMergeSplits; ++i) {
                const float w = mv[i] == -INFINITY ? 0.f : __expf(mv[i] - Mc);
                Lr += lv[i] * w;
#pragma unroll
                for (int k = 0; k < kMergeDims; ++k) o[k] += ov[i][k] * w;
            }
            Mr = Mc;
        }
#pragma unroll
        for (int k = 0; k < kMergeDims; ++k) {
            const int dv = d0 + k * SSQ_WAVE + lane;
            if (dv < Dv)
                ssq_store_elem(a.out, a.v_dtype, (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)qi * a.o_sl + dv,
                               o[k] / Lr);
        }
        M = Mr;
        L = Lr;
    }
    if (a.lse && lane == 0) a.lse[rid] = M + logf(L);
}

static int launch_merge(const ssq_decode_args& a, int n_splits, const float* ws_o, const float* ws_m,
                        const float* ws_l, hipStream_t st) {
    const int n_rows_all = a.batch * a.num_q_heads * a.q_len;
    hipLaunchKernelGGL(k_merge, dim3((unsigned)((n_rows_all + kMergeRows - 1) / kMergeRows)),
                       dim3(kMergeRows * SSQ_WAVE), 0, st, a, n_splits, ws_o, ws_m, ws_l);
    return ssq_check_hip(hipGetLastError(), "k_merge launch");
}

// --------------------------------------------------------------------------
// host side
// --------------------------------------------------------------------------
struct Plan {
    int G, rows, R, RP, n_groups, split_len, n_splits;
    size_t smem;
    size_t ws_bytes;
    bool has_v;
    bool wide;  // the staged-codebook kernel (ssq_decode_wide.hip)
};

int pow2_at_least(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

size_t smem_bytes(const ssq_decode_args& a, int RP, bool has_v) {
    return (red_offset(a, RP, has_v) + 2 * (kThreads / SSQ_WAVE) * RP) * sizeof(float);
}

// the codebook is 16-byte aligned (per head too) and so is qp after the LUT: vector loads of both
bool vec_cent_ok(const ssq_decode_args& a) {
    return (uintptr_t)a.cent % 16 == 0 && (a.cent_sh * 4) % 16 == 0 && a.head_dim % 4 == 0 &&
           (a.n_blocks * a.n_centroids) % 4 == 0;
}

// 16-bit codes in 16-byte aligned rows of a multiple of 8 blocks (at most 64) with codewords of 2
// or 4 dims in a 16-byte aligned codebook: the generic kernel's variants that load a token's code
// row in 16-byte pieces and gather its codewords in batches (ssq_decode_generic_w16.hip), and the
// staged-codebook kernel
bool use_w16(const ssq_decode_args& a) {
    return ssq_code_width(a.n_centroids) == 2 && a.code_bits == 0 && vec_cent_ok(a) && a.n_blocks % 8 == 0 &&
           a.n_blocks <= 64 && (a.block_dim == 2 || a.block_dim == 4) && (uintptr_t)a.codes % 16 == 0 &&
           a.c_sb % 8 == 0 && a.c_sh % 8 == 0 && a.c_st % 8 == 0;
}

// Splits of at least this many tokens take the staged-codebook kernel: below it a split's codebook
// copies (nb * nc * bd floats per super-tile) cost more than the per-token gathers they replace.
constexpr int kWideMinTokens = 2048;

// the splits of a plan with `slots` workgroups running at once
void plan_splits(const ssq_decode_args& a, Plan& pl, int slots) {
    const int units = a.batch * a.num_kv_heads * pl.n_groups;
    const int tiles = (a.seq_len + kTile - 1) / kTile;
    int splits = a.num_splits > 0 ? a.num_splits : (slots + units - 1) / units;
    if (splits > tiles) splits = tiles;
    if (splits < 1) splits = 1;
    const int tiles_per_split = (tiles + splits - 1) / splits;
    pl.split_len = tiles_per_split * kTile;
    pl.n_splits = (a.seq_len + pl.split_len - 1) / pl.split_len;
    if (pl.n_splits < 1) pl.n_splits = 1;
    const size_t n_rows_all = (size_t)a.batch * a.num_q_heads * a.q_len;
    pl.ws_bytes = (pl.has_v && pl.n_splits > 1) ? (size_t)pl.n_splits * n_rows_all * (a.value_dim + 2) * 4 : 0;
}

int make_plan(const ssq_decode_args& a, Plan& pl) {
    pl.has_v = a.v != nullptr;
    pl.G = a.num_q_heads / a.num_kv_heads;
    pl.rows = pl.G * a.q_len;
    pl.wide = false;
    if (pl.has_v && use_w16(a) && (a.heavy_mask[0] | a.heavy_mask[1]) == 0 && ssq_decode_wide_fits(a)) {
        // one workgroup per CU (its LDS), up to 4 rows per workgroup
        pl.R = pl.rows < 4 ? pl.rows : 4;
        pl.RP = pow2_at_least(pl.R);
        pl.n_groups = (pl.rows + pl.R - 1) / pl.R;
        pl.smem = ssq_decode_wide_smem(a, pl.RP);
        if (pl.smem <= kMaxSmem) {
            plan_splits(a, pl, ssq_device_cus());
            if (pl.split_len >= kWideMinTokens) {
                pl.wide = true;
                return SSQ_OK;
            }
        }
    }
    int R = pl.rows < kMaxRows ? pl.rows : kMaxRows;
    for (; R >= 1; --R) {
        if (smem_bytes(a, pow2_at_least(R), pl.has_v) <= kMaxSmem) break;
    }
    SSQ_UNSUPPORTED(R >= 1, "codebook too large for LDS: n_blocks*n_centroids=%d", a.n_blocks * a.n_centroids);
    pl.R = R;
    pl.RP = pow2_at_least(R);
    pl.n_groups = (pl.rows + R - 1) / R;
    pl.smem = smem_bytes(a, pl.RP, pl.has_v);
    // one round of workgroups: as many as the device runs at once at this LDS footprint
    // (each split rebuilds the LUT, so a second round costs more than it hides)
    const int per_cu = pl.smem > 0 ? (int)(kMaxSmem / pl.smem) : 1;
    plan_splits(a, pl, ssq_device_cus() * (per_cu < 1 ? 1 : per_cu > 2 ? 2 : per_cu));
    return SSQ_OK;
}

int validate(const ssq_decode_args* a, bool need_v) {
    if (!a) return ssq_fail(SSQ_ERR_INVALID, "args is NULL");
    if (a->struct_size != sizeof(ssq_decode_args))
        return ssq_fail(SSQ_ERR_ABI, "ssq_decode_args size %u != library's %zu", a->struct_size, sizeof(ssq_decode_args));
    SSQ_REQUIRE(a->q && a->perm && a->cent && a->codes, "q, perm, cent and codes must be non-NULL");
    SSQ_REQUIRE(a->batch >= 1 && a->num_q_heads >= 1 && a->q_len >= 1 && a->num_kv_heads >= 1, "empty batch/heads");
    SSQ_REQUIRE(a->num_q_heads % a->num_kv_heads == 0, "Query head count must be divisible by kv-head count.");
    SSQ_REQUIRE(a->block_dim >= 1 && a->head_dim % a->block_dim == 0, "head_dim must be divisible by block_dim");
    SSQ_REQUIRE(a->n_blocks == a->head_dim / a->block_dim, "n_blocks != head_dim / block_dim");
    SSQ_REQUIRE(a->head_dim <= 1024, "head_dim > 1024");
    SSQ_REQUIRE(a->n_centroids >= 1 && a->n_centroids <= kMaxCentroids, "n_centroids must be in [1, %d]", kMaxCentroids);
    SSQ_REQUIRE(a->n_blocks <= 128, "n_blocks > 128");
    SSQ_REQUIRE(a->code_bits >= 0 && a->code_bits <= 8, "code_bits must be 0 (uint8) or 1..8 (packed)");
    SSQ_REQUIRE(a->n_centroids <= 256 || a->code_bits == 0,
                "n_centroids=%d takes 16- or 32-bit codes (code_bits 0)", a->n_centroids);
    if (a->n_centroids > 256) {
        const int cw = ssq_code_width(a->n_centroids);
        SSQ_REQUIRE((uintptr_t)a->codes % cw == 0, "%d-bit codes must be %d-byte aligned", 8 * cw, cw);
    }
    if (a->code_bits) {
        SSQ_REQUIRE(a->n_centroids <= (1 << a->code_bits), "n_centroids=%d needs more than %d-bit codes",
                    a->n_centroids, a->code_bits);
        SSQ_REQUIRE((uintptr_t)a->codes % 4 == 0, "packed codes must be 4-byte aligned");
    }
    SSQ_REQUIRE(a->q_dtype >= SSQ_F32 && a->q_dtype <= SSQ_F16, "bad q_dtype");
    SSQ_REQUIRE(a->seq_len >= 0, "negative seq_len");
    const bool any_heavy = a->heavy_mask[0] || a->heavy_mask[1];
    SSQ_REQUIRE(!any_heavy || a->pt, "Mixed-precision quantized keys are missing passthrough values.");
    if (any_heavy) SSQ_REQUIRE(a->pt_dtype >= SSQ_F32 && a->pt_dtype <= SSQ_F16, "bad pt_dtype");
    SSQ_REQUIRE(a->layout == SSQ_CONTIGUOUS || a->layout == SSQ_PAGED, "bad layout");
    if (a->layout == SSQ_PAGED) {
        SSQ_REQUIRE(a->block_table && a->seq_lens, "paged layout needs block_table and seq_lens");
        SSQ_REQUIRE(a->page_size >= 8 && a->page_size <= kTile && kTile % a->page_size == 0,
                    "page_size must divide %d and be >= 8", kTile);
    }
    if (need_v) {
        SSQ_REQUIRE(a->v && a->out, "decode needs v and out");
        SSQ_REQUIRE(a->v_dtype >= SSQ_F32 && a->v_dtype <= SSQ_F16, "bad v_dtype");
        SSQ_REQUIRE(a->value_dim >= 8 && a->value_dim % 8 == 0 && a->value_dim <= kThreads &&
                        (a->layout == SSQ_PAGED ? kThreads % a->value_dim == 0 : kThreads % (a->value_dim / 8) == 0),
                    "unsupported value_dim %d", a->value_dim);
        SSQ_REQUIRE(a->layout == SSQ_CONTIGUOUS || a->page_size % 8 == 0, "paged V needs page_size % 8 == 0");
    }
    return SSQ_OK;
}

int run_generic(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st) {
    Plan pl;
    int rc = make_plan(*a, pl);
    if (rc) return rc;
    if (a->seq_len == 0) return ssq_fail(SSQ_ERR_INVALID, "seq_len == 0: softmax over an empty context");
    SSQ_REQUIRE(ws_bytes >= pl.ws_bytes, "workspace too small: %zu < %zu bytes", ws_bytes, pl.ws_bytes);
    SSQ_REQUIRE(pl.ws_bytes == 0 || workspace, "workspace is NULL");
    DecodeParams dp;
    dp.a = *a;
    dp.G = pl.G;
    dp.rows = pl.rows;
    dp.R = pl.R;
    dp.split_len = pl.split_len;
    dp.n_splits = pl.n_splits;
    dp.cw = ssq_code_width(a->n_centroids);
    const bool aligned = dp.cw == 1 && a->code_bits == 0 && ((uintptr_t)a->codes % 4 == 0) && a->n_blocks % 4 == 0 &&
                         a->c_st % 4 == 0 && a->c_sh % 4 == 0 && a->c_sb % 4 == 0;
    dp.word_codes = aligned ? 1 : 0;
    dp.vec_cent = vec_cent_ok(*a) ? 1 : 0;
    const size_t n_rows_all = (size_t)a->batch * a->num_q_heads * a->q_len;
    float* ws = reinterpret_cast<float*>(workspace);
    dp.ws_o = ws;
    dp.ws_m = ws ? ws + (size_t)pl.n_splits * n_rows_all * a->value_dim : nullptr;
    dp.ws_l = ws ? dp.ws_m + (size_t)pl.n_splits * n_rows_all : nullptr;
    if (pl.has_v) {
        // 16-byte vector loads of V
        const int esz = a->v_dtype == SSQ_F32 ? 4 : 2;
        SSQ_REQUIRE((uintptr_t)a->v % 16 == 0 && (a->v_sb * esz) % 16 == 0 && (a->v_sh * esz) % 16 == 0 &&
                        (a->v_st * esz) % 16 == 0,
                    "V must be 16-byte aligned with 16-byte aligned strides");
    }
    if (pl.wide) {
        rc = ssq_decode_wide(dp, pl.RP, pl.n_groups, pl.smem, st);
        if (rc == SSQ_OK && pl.n_splits > 1) rc = launch_merge(*a, pl.n_splits, dp.ws_o, dp.ws_m, dp.ws_l, st);
        return rc;
    }
    SsqGenericLaunch gl;
    gl.RP = pl.RP;
    gl.n_splits = pl.n_splits;
    gl.n_groups = pl.n_groups;
    gl.smem = pl.smem;
    gl.has_v = pl.has_v;
    rc = use_w16(*a) ? ssq_generic_w16(dp, gl, st) : launch_generic<false>(dp, gl, st);
    if (rc) return rc;
    if (pl.has_v && pl.n_splits > 1) {
        rc = launch_merge(*a, pl.n_splits, dp.ws_o, dp.ws_m, dp.ws_l, st);
    }
    return rc;
}

}  // namespace

// Launches the split merge (shared with the MFMA decode kernel).
int ssq_launch_merge(const ssq_decode_args& a, int n_splits, const float* ws_o, const float* ws_m,
                     const float* ws_l, hipStream_t st) {
    return launch_merge(a, n_splits, ws_o, ws_m, ws_l, st);
}

int ssq_decode_mfma_supported(const ssq_decode_args* a);
size_t ssq_decode_mfma_workspace(const ssq_decode_args* a);
int ssq_decode_mfma(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st);
int ssq_decode_contig_supported(const ssq_decode_args* a);
size_t ssq_decode_contig_workspace(const ssq_decode_args* a);
int ssq_decode_contig(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st);

namespace {
// kernel choice: 2 = MFMA paged, 3 = MFMA contiguous, 1 = generic; 0 picks the first that serves
int pick_kernel(const ssq_decode_args* a) {
    if (a->kernel == 4) return 2;  // the paged MFMA path, with its 4x4-MFMA-scores kernel forced
    if (a->kernel != 0) return a->kernel;
    // (the MFMA kernel's plan takes scores-only problems on contiguous rows past head_dim 64)
    if (ssq_decode_mfma_supported(a)) return 2;
    // scores only or decode: the contiguous MFMA kernel where it applies (its 4x4-MFMA scores need no
    // per-workgroup LUT: config-2 scores 11.9 us against the LUT kernel's 18.3 us), else the generic one
    if (ssq_decode_contig_supported(a)) return 3;
    return 1;
}
}  // namespace

extern "C" size_t ssq_decode_workspace_size(const ssq_decode_args* a) {
    if (validate(a, a && a->v != nullptr) != SSQ_OK) return 0;
    const int k = pick_kernel(a);
    if (k == 2 && a->v && ssq_decode_mfma_supported(a)) return ssq_decode_mfma_workspace(a);
    if (k == 3 && ssq_decode_contig_supported(a)) return ssq_decode_contig_workspace(a);
    Plan pl;
    if (make_plan(*a, pl) != SSQ_OK) return 0;
    return pl.ws_bytes;
}

extern "C" int ssq_decode(const ssq_decode_args* a, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = validate(a, true);
    if (rc) return rc;
    const int k = pick_kernel(a);
    if (k == 2) {
        SSQ_UNSUPPORTED(ssq_decode_mfma_supported(a), "MFMA decode kernel does not support this problem");
        return ssq_decode_mfma(a, workspace, workspace_bytes, (hipStream_t)stream);
    }
    if (k == 3) {
        SSQ_UNSUPPORTED(ssq_decode_contig_supported(a), "contiguous MFMA kernel does not support this problem");
        return ssq_decode_contig(a, workspace, workspace_bytes, (hipStream_t)stream);
    }
    return run_generic(a, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int ssq_attention_scores(const ssq_decode_args* a, void* stream) {
    int rc = validate(a, false);
    if (rc) return rc;
    SSQ_REQUIRE(a->v == nullptr && a->scores != nullptr, "scores-only call needs v == NULL and scores != NULL");
    if (a->seq_len == 0) return SSQ_OK;
    const int k = pick_kernel(a);
    if (k == 2) {
        SSQ_UNSUPPORTED(ssq_decode_mfma_supported(a), "MFMA LUT kernel does not support this scores-only problem");
        return ssq_decode_mfma(a, nullptr, 0, (hipStream_t)stream);
    }
    if (k == 3) {
        SSQ_UNSUPPORTED(ssq_decode_contig_supported(a), "contiguous MFMA kernel does not support this problem");
        return ssq_decode_contig(a, nullptr, 0, (hipStream_t)stream);
    }
    return run_generic(a, nullptr, 0, (hipStream_t)stream);
}
