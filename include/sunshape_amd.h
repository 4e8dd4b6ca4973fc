/*
 * sunshape_amd -- C ABI of the MI355X (gfx950) VQ-key decode-attention library.
 *
 * Plain pointers, sizes and strides only.  Every tensor pointer is a device
 * pointer; strides are in ELEMENTS of the tensor's own dtype.  `stream` is a
 * hipStream_t passed as void* (NULL = the null stream).  All entry points are
 * asynchronous on `stream`, allocate no device memory, and return SSQ_OK or an
 * error code whose message ssq_last_error() returns (thread-local).  Call them with
 * the device that holds the tensors and `stream` current (hipSetDevice): launch
 * planning reads that device's properties.
 *
 * Each argument struct starts with `struct_size`; the library rejects a caller
 * whose struct layout differs from this header (SSQ_ERR_ABI).
 *
 * Reference interfaces (paths relative to the gauravsaini/sunshape tree):
 *   ssq_attention_scores  <- sunshape/triton_kernels.py:549-609
 *                            sunshape_attention_scores[_strict](codec, query, quantized_key)
 *                            and sunshape/codec.py:403-422 SunShapeBlockCodec.attention_scores
 *   ssq_decode            <- sunshape/vllm_attn_backend.py:216-253 _apply_quantized_attention
 *                            (called from SunShapeAttentionImpl.forward, :271-305)
 *   ssq_lut_build         <- sunshape/triton_kernels.py:381-408 _precompute_query_centroid_dots
 *   ssq_encode            <- sunshape/codec.py:362-385 SunShapeBlockCodec.quantize and
 *                            sunshape/vllm_attn_backend.py:101-123 quantize_key_states
 *   ssq_dequantize        <- sunshape/codec.py:387-398 SunShapeBlockCodec.dequantize
 *   ssq_transform_rows    <- sunshape/codec.py:247-259 _forward/_inverse_transform (rotated mode)
 */
#ifndef SUNSHAPE_AMD_H
#define SUNSHAPE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SSQ_ABI_VERSION 5

enum ssq_status {
    SSQ_OK = 0,
    SSQ_ERR_INVALID = 1,   /* argument check failed; message names the argument */
    SSQ_ERR_HIP = 2,       /* a HIP runtime call failed (launch, attribute) */
    SSQ_ERR_ABI = 3,       /* struct_size mismatch between caller and library */
    SSQ_ERR_UNSUPPORTED = 4 /* valid input outside what the kernels implement */
};

enum ssq_dtype { SSQ_F32 = 0, SSQ_BF16 = 1, SSQ_F16 = 2 };

/* Width of the stored codes, as the reference's _compact_index_dtype (sunshape/codec.py:78-83):
 * one byte for n_centroids <= 256, 16 bits (read unsigned) up to 65535, 32 bits beyond, at most
 * SSQ_MAX_CENTROIDS.  Every `codes` pointer below has that element type; code strides count
 * elements of it (int32 words for the packed codes of code_bits 1..8, which take n_centroids <= 256). */
#define SSQ_MAX_CENTROIDS (1 << 20)

/* Layout of the key codes and values. */
enum ssq_layout {
    SSQ_CONTIGUOUS = 0, /* codes [B, Hkv, T, nb], V [B, Hkv, T, Dv] (token-major) */
    SSQ_PAGED = 1       /* vLLM-style pages: codes [P, Hkv, page, nb],
                           V [P, Hkv, Dv, page] (dim-major inside a page, vLLM's value layout),
                           block_table [B, max_pages] int32, seq_lens [B] int32 */
};

/*
 * One decode (or scores-only) problem.  Rows: for batch b and KV head kv the
 * G*Lq query rows q[b, kv*G + g, i, :] (g < G = Hq/Hkv, i < Lq) share the KV
 * head's codes and values; row index r = g*Lq + i, as in the reference's
 * query_slice.reshape(-1, D).
 *
 * Codec: permutation perm[kv*perm_sh + j] (int64, x_perm[j] = x[perm[j]]),
 * codebook cent[kv*cent_sh + (blk*nc + c)*bd + d] fp32.  perm_sh / cent_sh are
 * 0 for the reference's one-codec-per-layer layout.
 *
 * Passthrough (SunShape-Mixed) blocks: heavy_mask bit blk (blk < 128) marks a
 * block scored from stored values instead of codes.  pt holds them; the slot of
 * heavy block blk is blk itself when pt_dense != 0 (the reference's dense
 * [T, nb, bd] layout, codec.py:368) and its ordinal among heavy blocks otherwise.
 * Contiguous: pt[b*pt_sb + kv*pt_sh + t*pt_st + slot*bd + d].
 * Paged:      pt[page*pt_sb + kv*pt_sh + (t % page_size)*pt_st + slot*bd + d].
 */
typedef struct ssq_decode_args {
    uint32_t struct_size;
    /* query [B, Hq, Lq, D]; D contiguous */
    const void* q; int32_t q_dtype; int64_t q_sb, q_sh, q_sl;
    int32_t batch, num_q_heads, q_len, head_dim, num_kv_heads;
    int32_t has_scale;   /* 1: q <- round_to_q_dtype(q * scale), as query_slice * float(scale) */
    float scale;
    /* codec */
    const int64_t* perm; int64_t perm_sh;
    const float* cent; int64_t cent_sh;
    int32_t block_dim, n_blocks, n_centroids;
    /* passthrough blocks */
    uint64_t heavy_mask[2];
    int32_t pt_dense; int32_t pt_dtype;
    const void* pt; int64_t pt_sb, pt_sh, pt_st;
    /* keys */
    int32_t layout;      /* enum ssq_layout */
    int32_t seq_len;     /* T (contiguous) / max context (paged) */
    const uint8_t* codes; int64_t c_sb, c_sh, c_st;  /* contiguous: b,kv,t strides; paged: page,kv,t strides
                                                        (elements of the code width, SSQ_MAX_CENTROIDS) */
    const int32_t* block_table; int64_t bt_sb; const int32_t* seq_lens; int32_t page_size;
    /* values (NULL for scores-only); Dv contiguous (contiguous) / page contiguous (paged) */
    const void* v; int32_t v_dtype; int32_t value_dim;
    int64_t v_sb, v_sh, v_st;   /* contiguous: b,kv,t strides; paged: page,kv,dv strides */
    /* additive fp32 mask [b, h, i, t] via strides (0 = broadcast); NULL = none */
    const float* mask; int64_t m_sb, m_sh, m_sl, m_st;
    /* outputs */
    void* out; int64_t o_sb, o_sh, o_sl;      /* [B, Hq, Lq, Dv] in v_dtype; NULL for scores-only */
    float* lse;                                /* [B, Hq, Lq] fp32 contiguous or NULL */
    float* scores; int64_t s_sb, s_sh, s_sl;  /* raw logits [B, Hq, Lq, T] fp32 (t contiguous) or NULL;
                                                 paged: entries t >= seq_lens[b] are not written */
    /* tuning: 0 = library heuristic */
    int32_t num_splits;
    int32_t kernel;      /* 0 auto, 1 generic LUT/VALU kernel (past 256 codewords: codewords gathered from
                            memory, or with 16-bit codes over splits of >= 2048 tokens each block's
                            codebook staged in LDS per super-tile), 2 MFMA LUT kernels (paged: LUT scores, or 4x4-MFMA scores where the
                            LUT does not fit or a mask / passthrough blocks come; contiguous rows past
                            head_dim 64 with 128-dim values, or scores only; at head_dim 128 the 4x4-MFMA
                            kernel where the LUT needs row groups), 3 MFMA contiguous kernel (head_dim 64),
                            4 the 4x4-MFMA-scores kernel (paged, or contiguous at head_dim 128) wherever it
                            applies */
    /* code storage: 0 = one code per block, of the width n_centroids gives (SSQ_MAX_CENTROIDS; c_*
     * strides in those elements); 1..8 (n_centroids <= 256) = packing in uint32 words,
     * vpe = 32 / code_bits codes per word, block blk = p*vpe + v at bits
     * [v*code_bits, (v+1)*code_bits) of word p (the layout of sunshape/triton_kernels.py:213-283);
     * c_* strides then count words.  8-bit words are read as byte rows; 6-bit words run on
     * every MFMA decode kernel and 4-bit words on the contiguous and 4x4-MFMA-scores ones
     * (without mask or passthrough); other widths take the generic kernel.  Results equal the
     * same kernel's launch over uint8 codes bit for bit. */
    int32_t code_bits;
} ssq_decode_args;

/* Bytes of device workspace ssq_decode / ssq_attention_scores need (0 if none). */
size_t ssq_decode_workspace_size(const ssq_decode_args* a);

/* Fused decode: out = softmax(q.k_hat + mask) @ V per row, plus lse / raw scores on request.
 * Replaces sunshape/vllm_attn_backend.py:216-253 (scores from :238, mask :241-249,
 * softmax and cast :251, P.V :252) for all batches and KV heads in one call. */
int ssq_decode(const ssq_decode_args* a, void* workspace, size_t workspace_bytes, void* stream);

/* ssq_decode without device allocation.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  The caller passes inputs and outputs only; the split workspace ssq_decode would
 * take from the caller lives in a library-owned scratch array of SSQ_NOALLOC_SCRATCH_BYTES per
 * device (held until the process ends).  A problem whose ssq_decode_workspace_size exceeds it
 * fails with SSQ_ERR_UNSUPPORTED before anything is launched.  Calls and results are otherwise
 * those of ssq_decode (same kernels).  Every call on one device shares that device's array:
 * calls that overlap on one device race and must be serialised by the caller. */
#define SSQ_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int ssq_decode_noalloc(const ssq_decode_args* a, void* stream);

/* Scores only (a->v == NULL, a->scores != NULL): scores[r, t] = q_r . k_hat_t (unscaled
 * unless has_scale).  Replaces sunshape/triton_kernels.py:570-609 and codec.py:403-422. */
int ssq_attention_scores(const ssq_decode_args* a, void* stream);

/* LUT[r, blk, c] = sum_d q_perm[r, blk*bd + d] * cent[blk, c, d], fp32 [R, nb, nc].
 * q: [R, D] (row stride q_sr), perm [D], cent [nb, nc, bd].
 * Replaces sunshape/triton_kernels.py:381-408. */
int ssq_lut_build(const void* q, int32_t q_dtype, int64_t q_sr, int32_t rows, int32_t head_dim,
                  const int64_t* perm, const float* cent, int32_t block_dim, int32_t n_centroids,
                  int32_t has_scale, float scale, float* lut, void* stream);

/*
 * Nearest-codeword encode of keys [B, Hkv, S, D] (k[b*k_sb + kv*k_sh + s*k_ss + d]).
 * codes[b, kv, s, blk] = argmin_c sqrt(max(0, |x_blk|^2 - 2 x_blk.c + |c|^2)) evaluated
 * with torch.cdist's mm formulation (or its direct one, direct_dist), lowest index on ties.  With a block metric
 * (SunShape-Pro, metric != NULL: E [D, D] fp32 row-major at metric + kv*metric_sh, of which
 * only the diagonal bd x bd blocks E_b are read, as codec.py:375-376 slices them) x_blk and
 * every codeword c are first mapped to E_b x and E_b c (y_k = sum_j E_b[k][j] x_j, j
 * ascending, first product rounded, then fused multiply-adds).  Heavy blocks get code 0 and
 * their values are copied to pt in pt_dtype (slot = ordinal among heavy blocks, or the
 * block index itself when pt_dense != 0: the reference's dense [.., nb, bd] layout, whose
 * light-block entries the caller pre-fills with zeros).
 * Contiguous output: codes[b*c_sb + kv*c_sh + s*c_st + blk], pt[b*pt_sb + kv*pt_sh + s*pt_st + slot*bd + d].
 * Paged output (slot_mapping != NULL, [B, S] int64 token slots): slot -> page = slot / page_size,
 *   off = slot % page_size; codes[page*c_sb + kv*c_sh + off*c_st + blk] (pt likewise).
 * Replaces sunshape/codec.py:362-385 and the loop of sunshape/vllm_attn_backend.py:101-123.
 */
typedef struct ssq_encode_args {
    uint32_t struct_size;
    const void* keys; int32_t k_dtype; int64_t k_sb, k_sh, k_ss;
    int32_t batch, num_kv_heads, seq_len, head_dim;
    const int64_t* perm; int64_t perm_sh;
    const float* cent; int64_t cent_sh;
    const float* metric; int64_t metric_sh;   /* SunShape-Pro E [D, D] or NULL (identity) */
    int32_t block_dim, n_blocks, n_centroids;
    uint64_t heavy_mask[2];
    uint8_t* codes; int64_t c_sb, c_sh, c_st;   /* code width per n_centroids (SSQ_MAX_CENTROIDS) */
    void* pt; int32_t pt_dtype; int32_t pt_dense; int64_t pt_sb, pt_sh, pt_st;
    const int64_t* slot_mapping; int64_t sm_sb; int32_t page_size;
    int32_t kernel;      /* 0 auto, 1 VALU exact scan, 2 MFMA screen + exact certification, 3 grid search
                            (2 and 3 serve at most 256 codewords; more run the exact scan over LDS chunks
                            of the codebook) */
    const void* grid; uint64_t grid_bytes;  /* optional search grid from ssq_encode_grid_build (or NULL) */
    /* 1: torch.cdist's direct evaluation, sqrt(sum_k (x_k - c_k)^2) with the rounded squares summed
     * in k order, which torch takes in place of the mm formulation when both of its inputs have at
     * most 25 rows (the reference quantizing <= 25 keys per call with <= 25 codewords).  Runs on
     * the exact scan (kernel 0 or 1; 2 and 3 are refused). */
    int32_t direct_dist;
} ssq_encode_args;

int ssq_encode(const ssq_encode_args* a, void* stream);

/*
 * Search grid for the encode (block_dim 2, no block metric; no counterpart in the reference: a
 * search structure of this library, built once per codebook and reused by every encode with
 * that codebook).  For each codebook (one, or one per KV head) and block, a 128 x 128 grid of
 * cells covers the whole plane: each coordinate x maps to u = (x - mid) * inv, t = u / (1 + |u|),
 * cell floor((t + 1) * 64), with mid the codewords' bounding-box centre and 1/inv their RMS
 * spread, so cells are finest where codewords crowd and the end cells reach to +-infinity.
 * Each cell lists, ascending, every codeword that can be the reference's first minimum for a
 * key in the cell (rounding of the reference's fp32 evaluation included), up to 15 (a longer
 * list, an unbounded end cell, a block whose codewords are all one point or a non-finite key
 * falls back to scanning all codewords).  ssq_encode then evaluates only those candidates, with
 * the reference's exact arithmetic, so its codes equal kernels 1 and 2 bit for bit.  Layout,
 * head-major: per codebook head, its block headers (32 bytes each, padded to 256), the cells'
 * first 4 bytes (count and three indices), then the cells' other 16 bytes, so head h's bytes
 * [h * size / heads, (h + 1) * size / heads) of a per-KV-head grid are the grid of that head's
 * codebook alone.  Size per head and block: 320 KiB.  The grid buffer must be 16-byte aligned.
 * The grid depends only on perm-independent codebook values (cent, cent_sh, n_blocks,
 * n_centroids, num_kv_heads when cent_sh != 0); rebuild it when the codebook changes.  Each
 * block's header holds a fingerprint of its codebook: ssq_encode scans every codeword of a
 * block whose codebook no longer matches, so a stale grid is slow, not wrong.
 */
uint64_t ssq_encode_grid_bytes(const ssq_encode_args* a);
int ssq_encode_grid_build(const ssq_encode_args* a, void* grid, uint64_t grid_bytes, void* stream);

/* Dense transform of rows, fp32 out [rows, dim] (row stride o_sr):
 *   out[r, j] = sum_k xs[r, k] * M[j, k]   (transpose 0: x @ M^T)   or   sum_k xs[r, k] * M[k, j]
 *   (transpose 1: x @ M), k ascending, the first product rounded, then fused multiply-adds;
 * xs = x (x_dtype, row stride x_sr), or round_to_x_dtype(x * scale) when has_scale (ssq_decode's
 * query scaling).  M: [dim, dim] fp32 row-major.
 * Replaces the rotated mode of sunshape/codec.py:247-259: _forward_transform (x @ rotation.T)
 * before scoring and encoding, _inverse_transform (x @ rotation) after dequantizing. */
int ssq_transform_rows(const void* x, int32_t x_dtype, int64_t x_sr, int64_t rows, int32_t dim,
                       int32_t has_scale, float scale, const float* mat, int32_t transpose,
                       float* out, int64_t o_sr, void* stream);

/* k_hat[t, j] (original basis, fp32 [T, D] with row stride o_st) from codes [T, nb] of the width
 * n_centroids gives (row stride c_st elements) and optional passthrough pt (dense [T, nb, bd] fp32 when pt_dense,
 * else compact [T, n_heavy, bd]; row stride pt_st).  Replaces sunshape/codec.py:387-398. */
int ssq_dequantize(const uint8_t* codes, int64_t c_st, int32_t tokens,
                   const int64_t* perm, const float* cent, int32_t head_dim, int32_t block_dim,
                   int32_t n_centroids, const uint64_t* heavy_mask, int32_t pt_dense,
                   const void* pt, int32_t pt_dtype, int64_t pt_st,
                   float* out, int64_t o_st, void* stream);

/* Pack uint8 codes [rows, n_blocks] (row stride c_st bytes) into uint32 words
 * [rows, ceil(n_blocks / (32 / bits))] (row stride o_st words) in the code_bits layout above.
 * Precondition: every code < 2^bits (bits above are dropped); unused high bits of a word are 0.
 * The reference has the reader of this layout (sunshape/triton_kernels.py:213-283) but no writer. */
int ssq_pack_codes(const uint8_t* codes, int64_t c_st, int64_t rows, int32_t n_blocks, int32_t bits,
                   uint32_t* out, int64_t o_st, void* stream);
/* Inverse of ssq_pack_codes. */
int ssq_unpack_codes(const uint32_t* packed, int64_t p_st, int64_t rows, int32_t n_blocks, int32_t bits,
                     uint8_t* out, int64_t o_st, void* stream);

const char* ssq_last_error(void);
int ssq_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SUNSHAPE_AMD_H */
