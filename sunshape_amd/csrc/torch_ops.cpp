// Torch operators over the sunshape_amd C ABI (host code only; the kernels live in
// libsunshape_amd.so): torch.ops.sunshape.decode, .scores and .encode_into.
//
// Each operator validates its tensors (the checks and messages of the Python surface,
// sunshape_amd/hip_ops.py), allocates outputs and workspace through torch's caching allocator
// (encode_into writes into outputs its caller allocates: fresh tensors, or cache pages), and
// calls the library on torch's current HIP stream of the first tensor's device.  Registered for the
// CUDA dispatch key, which HIP tensors carry in PyTorch-ROCm, so the operators are visible to the
// dispatcher and to graph capture.  A library error raises RuntimeError whose message starts with
// "sunshape_amd status <code>: ".
#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <ATen/ops/full.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cmath>
#include <limits>
#include <optional>
#include <string>
#include <tuple>

#include "../../include/sunshape_amd.h"

namespace {

using at::Tensor;

int dtype_code(const Tensor& t) {
    switch (t.scalar_type()) {
        case at::kFloat: return SSQ_F32;
        case at::kBFloat16: return SSQ_BF16;
        case at::kHalf: return SSQ_F16;
        default: TORCH_CHECK(false, "unsupported dtype ", t.scalar_type(), "; expected float32, bfloat16 or float16");
    }
    return -1;
}

void on_gpu(const char* name, const Tensor& t) {
    TORCH_CHECK(t.is_cuda(), name, " must be a HIP device tensor (got device ", t.device(),
                "); this library has no CPU path");
}

void check_status(int rc) {
    TORCH_CHECK(rc == SSQ_OK, "sunshape_amd status ", rc, ": ", ssq_last_error());
}

hipStream_t stream_of(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

const void* ptr(const std::optional<Tensor>& t) { return t.has_value() && t->defined() ? t->data_ptr() : nullptr; }

struct Codec {
    Tensor perm, cent;
    int64_t perm_sh, cent_sh;
    int64_t bd, nb, nc;
};

// codec arrays: perm [D] or [Hkv, D] int64, centroids [nb, nc, bd] or [Hkv, nb, nc, bd] fp32
Codec codec_arrays(const Tensor& perm_in, const Tensor& cent_in, int64_t D, int64_t n_kv) {
    on_gpu("permutation", perm_in);
    on_gpu("centroids", cent_in);
    TORCH_CHECK(perm_in.scalar_type() == at::kLong, "permutation must be int64");
    TORCH_CHECK(cent_in.scalar_type() == at::kFloat, "centroids must be float32");
    Codec c;
    c.perm = perm_in.contiguous();
    c.cent = cent_in.contiguous();
    const Tensor& cent = c.cent;
    if (cent.dim() == 3) {
        c.nb = cent.size(0); c.nc = cent.size(1); c.bd = cent.size(2);
        c.cent_sh = 0;
    } else if (cent.dim() == 4) {
        c.nb = cent.size(1); c.nc = cent.size(2); c.bd = cent.size(3);
        TORCH_CHECK(n_kv < 0 || cent.size(0) == n_kv, "centroids hold ", cent.size(0), " KV heads, expected ", n_kv);
        c.cent_sh = c.nb * c.nc * c.bd;
    } else {
        TORCH_CHECK(false, "Expected codec.centroids.ndim == 3 (or 4 for per-KV-head codebooks), got ", cent.dim(), ".");
    }
    const Tensor& perm = c.perm;
    if (perm.dim() == 1) {
        c.perm_sh = 0;
        TORCH_CHECK(perm.size(0) == D, "permutation length ", perm.size(0), " != head_dim ", D);
    } else {
        TORCH_CHECK(perm.dim() == 2 && perm.size(1) == D, "permutation must be [D] or [Hkv, D]");
        TORCH_CHECK(n_kv < 0 || perm.size(0) == n_kv, "permutation holds ", perm.size(0), " KV heads, expected ", n_kv);
        c.perm_sh = D;
    }
    TORCH_CHECK(c.nb * c.bd == D, "centroids [", c.nb, ", ", c.nc, ", ", c.bd, "] do not tile head_dim ", D);
    return c;
}

int64_t words_per_row(int64_t nb, int64_t bits) {
    const int64_t vpe = 32 / bits;
    return (nb + vpe - 1) / vpe;
}

// the stored index dtype, as the reference's _compact_index_dtype (sunshape/codec.py:78-83)
at::ScalarType index_dtype(int64_t nc) { return nc <= 256 ? at::kByte : nc <= 65535 ? at::kShort : at::kInt; }

void check_codes(const Tensor& codes, int64_t nb, int64_t nc, int64_t code_bits) {
    if (code_bits == 0) {
        const at::ScalarType want = index_dtype(nc);
        TORCH_CHECK(codes.scalar_type() == want, "codes must be ", want, " for n_centroids=", nc, ", got ",
                    codes.scalar_type());
        TORCH_CHECK(codes.size(-1) == nb, "codes must be [.., ", nb, "] ", want);
    } else {
        TORCH_CHECK(nc <= 256, "n_centroids=", nc, " takes 16- or 32-bit codes, not packed words");
        TORCH_CHECK(code_bits >= 1 && code_bits <= 8, "code_bits must be 0 (uint8) or 1..8 (packed words)");
        const int64_t nw = words_per_row(nb, code_bits);
        TORCH_CHECK(codes.scalar_type() == at::kInt, "packed codes must be int32 words, got ", codes.scalar_type());
        TORCH_CHECK(codes.size(-1) == nw, "packed codes must be [.., ", nw, "] int32 for nb=", nb, ", bits=", code_bits);
    }
}

// passthrough values for heavy blocks: contiguous per token
void check_pt(const std::optional<Tensor>& pt, bool any_heavy) {
    if (!any_heavy) return;
    TORCH_CHECK(pt.has_value() && pt->defined(), "Mixed-precision quantized keys are missing passthrough values.");
    on_gpu("passthrough_values", *pt);
    TORCH_CHECK(pt->stride(-1) == 1 && pt->stride(-2) == pt->size(-1), "passthrough values must be contiguous per token");
}

// ---------------------------------------------------------------------------------------------
// decode: sunshape/vllm_attn_backend.py:216-253 for all batches and KV heads in one launch
// ---------------------------------------------------------------------------------------------
std::tuple<Tensor, Tensor, Tensor> decode(const Tensor& q_in, const Tensor& codes, const Tensor& v,
                                          const Tensor& perm_in, const Tensor& cent_in, std::optional<double> scale,
                                          const std::optional<Tensor>& mask_in, int64_t hm0, int64_t hm1,
                                          const std::optional<Tensor>& pt, bool pt_dense,
                                          const std::optional<Tensor>& block_table, const std::optional<Tensor>& seq_lens,
                                          bool return_lse, bool return_scores, int64_t num_splits, int64_t kernel,
                                          int64_t code_bits, bool no_alloc) {
    on_gpu("query", q_in);
    on_gpu("codes", codes);
    on_gpu("value", v);
    TORCH_CHECK(q_in.dim() == 4, "Quantized attention expects query/value tensors with shape [batch, heads, seq, dim].");
    const Tensor q = q_in.stride(-1) == 1 ? q_in : q_in.contiguous();
    TORCH_CHECK(codes.stride(-1) == 1, "codes must be contiguous in the last dim");
    const int64_t B = q.size(0), Hq = q.size(1), Lq = q.size(2), D = q.size(3);
    const bool paged = block_table.has_value() && block_table->defined();
    TORCH_CHECK(codes.dim() >= 2, "codes must be 4-D");
    const int64_t Hkv = codes.size(1);
    TORCH_CHECK(Hq % Hkv == 0, "Query head count must be divisible by kv-head count.");
    const Codec c = codec_arrays(perm_in, cent_in, D, Hkv);
    TORCH_CHECK(codes.dim() == 4, "codes must be 4-D [.., ", c.nb, "]");
    check_codes(codes, c.nb, c.nc, code_bits);
    int64_t T, Dv, page, layout;
    if (paged) {
        const Tensor& bt = *block_table;
        on_gpu("block_table", bt);
        TORCH_CHECK(seq_lens.has_value() && seq_lens->defined(), "paged decode needs seq_lens");
        on_gpu("seq_lens", *seq_lens);
        TORCH_CHECK(bt.scalar_type() == at::kInt && seq_lens->scalar_type() == at::kInt,
                    "block_table/seq_lens must be int32");
        TORCH_CHECK(bt.dim() == 2 && bt.size(0) == B && bt.stride(1) == 1, "block_table [B, max_pages]");
        page = codes.size(2);
        TORCH_CHECK(v.dim() == 4 && v.size(0) == codes.size(0) && v.size(1) == Hkv && v.size(3) == page,
                    "paged V must be [P, Hkv, Dv, page]");
        TORCH_CHECK(v.stride(-1) == 1, "paged V pages must be contiguous over tokens");
        Dv = v.size(2);
        T = bt.size(1) * page;
        layout = SSQ_PAGED;
    } else {
        TORCH_CHECK(codes.size(0) == B, "Quantized key batch size does not match query batch size.");
        TORCH_CHECK(v.dim() == 4 && v.size(0) == B, "Quantized key batch size does not match value batch size.");
        TORCH_CHECK(v.size(1) == Hkv, "Quantized key kv-head count does not match value kv-head count.");
        TORCH_CHECK(v.size(2) == codes.size(2), "Quantized key sequence length does not match value sequence length.");
        TORCH_CHECK(v.stride(-1) == 1, "value must be contiguous in the last dim");
        T = codes.size(2);
        Dv = v.size(3);
        page = 0;
        layout = SSQ_CONTIGUOUS;
    }
    c10::hip::HIPGuard guard(q.device().index());
    Tensor out = at::empty({B, Hq, Lq, Dv}, v.options());
    Tensor lse = at::empty({return_lse ? B : 0, Hq, Lq}, q.options().dtype(at::kFloat));
    Tensor scores;
    if (return_scores)  // paged: slots past a sequence's length are never scored and read -inf
        scores = paged ? at::full({B, Hq, Lq, T}, -std::numeric_limits<float>::infinity(), q.options().dtype(at::kFloat))
                       : at::empty({B, Hq, Lq, T}, q.options().dtype(at::kFloat));
    else
        scores = at::empty({0}, q.options().dtype(at::kFloat));
    Tensor mask;
    if (mask_in.has_value() && mask_in->defined()) {
        on_gpu("attn_mask", *mask_in);
        mask = mask_in->to(at::kFloat);
        TORCH_CHECK(mask.dim() == 4, "decode() takes a 4-D mask view broadcastable to [B, Hq, Lq, T]");
        mask = mask.expand({B, Hq, Lq, T});
    }
    const bool any_heavy = hm0 != 0 || hm1 != 0;
    check_pt(pt, any_heavy);

    ssq_decode_args a{};
    a.struct_size = sizeof(ssq_decode_args);
    a.q = q.data_ptr(); a.q_dtype = dtype_code(q);
    a.q_sb = q.stride(0); a.q_sh = q.stride(1); a.q_sl = q.stride(2);
    a.batch = (int32_t)B; a.num_q_heads = (int32_t)Hq; a.q_len = (int32_t)Lq; a.head_dim = (int32_t)D;
    a.num_kv_heads = (int32_t)Hkv;
    a.has_scale = scale.has_value() ? 1 : 0;
    a.scale = scale.has_value() ? (float)*scale : 0.f;
    a.perm = c.perm.data_ptr<int64_t>(); a.perm_sh = c.perm_sh;
    a.cent = c.cent.data_ptr<float>(); a.cent_sh = c.cent_sh;
    a.block_dim = (int32_t)c.bd; a.n_blocks = (int32_t)c.nb; a.n_centroids = (int32_t)c.nc;
    a.heavy_mask[0] = (uint64_t)hm0; a.heavy_mask[1] = (uint64_t)hm1;
    if (any_heavy) {
        a.pt_dense = pt_dense ? 1 : 0;
        a.pt_dtype = dtype_code(*pt);
        a.pt = pt->data_ptr();
        a.pt_sb = pt->stride(0); a.pt_sh = pt->stride(1); a.pt_st = pt->stride(2);
    } else {
        a.pt_dtype = SSQ_F32;
    }
    a.layout = (int32_t)layout;
    a.seq_len = (int32_t)T;
    a.codes = reinterpret_cast<const uint8_t*>(codes.data_ptr());
    a.c_sb = codes.stride(0); a.c_sh = codes.stride(1); a.c_st = codes.stride(2);
    if (paged) {
        a.block_table = block_table->data_ptr<int32_t>(); a.bt_sb = block_table->stride(0);
        a.seq_lens = seq_lens->data_ptr<int32_t>();
        a.page_size = (int32_t)page;
    }
    a.v = v.data_ptr(); a.v_dtype = dtype_code(v); a.value_dim = (int32_t)Dv;
    a.v_sb = v.stride(0); a.v_sh = v.stride(1); a.v_st = v.stride(2);
    if (mask.defined()) {
        a.mask = mask.data_ptr<float>();
        a.m_sb = mask.stride(0); a.m_sh = mask.stride(1); a.m_sl = mask.stride(2); a.m_st = mask.stride(3);
    }
    a.out = out.data_ptr(); a.o_sb = out.stride(0); a.o_sh = out.stride(1); a.o_sl = out.stride(2);
    a.lse = return_lse ? lse.data_ptr<float>() : nullptr;
    if (return_scores) {
        a.scores = scores.data_ptr<float>();
        a.s_sb = scores.stride(0); a.s_sh = scores.stride(1); a.s_sl = scores.stride(2);
    }
    a.num_splits = (int32_t)num_splits; a.kernel = (int32_t)kernel; a.code_bits = (int32_t)code_bits;
    hipStream_t st = stream_of(q);
    if (no_alloc) {
        check_status(ssq_decode_noalloc(&a, st));
    } else {
        const size_t ws_bytes = ssq_decode_workspace_size(&a);
        Tensor ws = ws_bytes ? at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte)) : Tensor();
        check_status(ssq_decode(&a, ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, st));
    }
    return {out, lse, scores};
}

// ---------------------------------------------------------------------------------------------
// scores: sunshape/triton_kernels.py:570-609 (one query row set per KV head, all batches and KV
// heads in one launch); q [B, Hq, Lq, D], codes [B, Hkv, T, nb] -> fp32 [B, Hq, Lq, T]
// ---------------------------------------------------------------------------------------------
Tensor scores(const Tensor& q_in, const Tensor& codes, const Tensor& perm_in, const Tensor& cent_in,
              std::optional<double> scale, int64_t hm0, int64_t hm1, const std::optional<Tensor>& pt, bool pt_dense,
              int64_t code_bits, int64_t num_splits, int64_t kernel) {
    on_gpu("query", q_in);
    on_gpu("codes", codes);
    TORCH_CHECK(q_in.dim() == 4 && codes.dim() == 4, "scores expects q [B, Hq, Lq, D] and codes [B, Hkv, T, nb]");
    const Tensor q = q_in.stride(-1) == 1 ? q_in : q_in.contiguous();
    TORCH_CHECK(codes.stride(-1) == 1, "codes must be contiguous in the last dim");
    const int64_t B = q.size(0), Hq = q.size(1), Lq = q.size(2), D = q.size(3);
    const int64_t Hkv = codes.size(1), T = codes.size(2);
    TORCH_CHECK(codes.size(0) == B, "Quantized key batch size does not match query batch size.");
    TORCH_CHECK(Hq % Hkv == 0, "Query head count must be divisible by kv-head count.");
    const Codec c = codec_arrays(perm_in, cent_in, D, Hkv);
    check_codes(codes, c.nb, c.nc, code_bits);
    const bool any_heavy = hm0 != 0 || hm1 != 0;
    check_pt(pt, any_heavy);
    c10::hip::HIPGuard guard(q.device().index());
    Tensor out = at::empty({B, Hq, Lq, T}, q.options().dtype(at::kFloat));
    if (T == 0 || B * Hq * Lq == 0) return out;
    ssq_decode_args a{};
    a.struct_size = sizeof(ssq_decode_args);
    a.q = q.data_ptr(); a.q_dtype = dtype_code(q);
    a.q_sb = q.stride(0); a.q_sh = q.stride(1); a.q_sl = q.stride(2);
    a.batch = (int32_t)B; a.num_q_heads = (int32_t)Hq; a.q_len = (int32_t)Lq; a.head_dim = (int32_t)D;
    a.num_kv_heads = (int32_t)Hkv;
    a.has_scale = scale.has_value() ? 1 : 0;
    a.scale = scale.has_value() ? (float)*scale : 0.f;
    a.perm = c.perm.data_ptr<int64_t>(); a.perm_sh = c.perm_sh;
    a.cent = c.cent.data_ptr<float>(); a.cent_sh = c.cent_sh;
    a.block_dim = (int32_t)c.bd; a.n_blocks = (int32_t)c.nb; a.n_centroids = (int32_t)c.nc;
    a.heavy_mask[0] = (uint64_t)hm0; a.heavy_mask[1] = (uint64_t)hm1;
    a.pt_dtype = SSQ_F32;
    if (any_heavy) {
        a.pt_dense = pt_dense ? 1 : 0;
        a.pt_dtype = dtype_code(*pt);
        a.pt = pt->data_ptr();
        a.pt_sb = pt->stride(0); a.pt_sh = pt->stride(1); a.pt_st = pt->stride(2);
    }
    a.layout = SSQ_CONTIGUOUS;
    a.seq_len = (int32_t)T;
    a.codes = reinterpret_cast<const uint8_t*>(codes.data_ptr());
    a.c_sb = codes.stride(0); a.c_sh = codes.stride(1); a.c_st = codes.stride(2);
    a.scores = out.data_ptr<float>();
    a.s_sb = out.stride(0); a.s_sh = out.stride(1); a.s_sl = out.stride(2);
    a.num_splits = (int32_t)num_splits; a.kernel = (int32_t)kernel; a.code_bits = (int32_t)code_bits;
    check_status(ssq_attention_scores(&a, stream_of(q)));
    return out;
}

// ---------------------------------------------------------------------------------------------
// encode_into: sunshape/codec.py:362-385 for keys [B, Hkv, S, D], written into the caller's codes
// ([B, Hkv, S, nb] uint8, or pages [P, Hkv, page, nb] with slot_mapping [B, S]) and, for heavy
// blocks, passthrough values ([B, Hkv, S, slots, bd], or pages [P, Hkv, page, slots, bd])
// ---------------------------------------------------------------------------------------------
void encode_into(const Tensor& keys_in, const Tensor& perm_in, const Tensor& cent_in, int64_t hm0, int64_t hm1,
                 bool pt_dense, const Tensor& codes, const std::optional<Tensor>& pt,
                 const std::optional<Tensor>& slot_mapping, const std::optional<Tensor>& metric_in,
                 const std::optional<Tensor>& grid, int64_t kernel, bool direct) {
    on_gpu("key_states", keys_in);
    TORCH_CHECK(keys_in.dim() == 4,
                "quantize_key_states expects key_states with shape [batch, kv_heads, seq_len, head_dim].");
    const Tensor keys = keys_in.stride(-1) == 1 ? keys_in : keys_in.contiguous();
    const int64_t B = keys.size(0), Hkv = keys.size(1), S = keys.size(2), D = keys.size(3);
    const Codec c = codec_arrays(perm_in, cent_in, D, Hkv);
    on_gpu("codes", codes);
    TORCH_CHECK(codes.scalar_type() == index_dtype(c.nc) && codes.dim() == 4 && codes.size(1) == Hkv &&
                    codes.size(3) == c.nb && codes.stride(3) == 1,
                "codes must be ", index_dtype(c.nc), " [.., ", Hkv, ", .., ", c.nb, "] with unit last stride");
    const bool any_heavy = hm0 != 0 || hm1 != 0;
    const bool paged = slot_mapping.has_value() && slot_mapping->defined();
    if (paged) {
        on_gpu("slot_mapping", *slot_mapping);
        TORCH_CHECK(slot_mapping->scalar_type() == at::kLong && slot_mapping->dim() == 2 &&
                        slot_mapping->size(0) == B && slot_mapping->size(1) == S && slot_mapping->stride(1) == 1,
                    "slot_mapping must be int64 [B, S]");
    } else {
        TORCH_CHECK(codes.size(0) == B && codes.size(2) == S, "codes must be [", B, ", ", Hkv, ", ", S, ", ", c.nb, "]");
    }
    if (any_heavy) {
        TORCH_CHECK(pt.has_value() && pt->defined(), "heavy blocks need a passthrough output");
        on_gpu("passthrough_values", *pt);
        TORCH_CHECK(pt->dim() == 5 && pt->size(1) == Hkv && pt->size(4) == c.bd && pt->stride(4) == 1 &&
                        pt->stride(3) == c.bd,
                    "passthrough output must be [.., ", Hkv, ", .., slots, ", c.bd, "] with packed rows");
    }
    Tensor metric;
    int64_t metric_sh = 0;
    if (metric_in.has_value() && metric_in->defined()) {
        on_gpu("metric", *metric_in);
        metric = metric_in->to(at::kFloat).contiguous();
        TORCH_CHECK((metric.dim() == 2 || metric.dim() == 3) && metric.size(-1) == D && metric.size(-2) == D,
                    "metric must be [D, D] or [Hkv, D, D]");
        if (metric.dim() == 3) {
            TORCH_CHECK(metric.size(0) == Hkv, "per-head metric holds ", metric.size(0), " heads, keys have ", Hkv);
            metric_sh = D * D;
        }
    }
    if (B * S == 0) return;
    c10::hip::HIPGuard guard(keys.device().index());
    ssq_encode_args a{};
    a.struct_size = sizeof(ssq_encode_args);
    a.keys = keys.data_ptr(); a.k_dtype = dtype_code(keys);
    a.k_sb = keys.stride(0); a.k_sh = keys.stride(1); a.k_ss = keys.stride(2);
    a.batch = (int32_t)B; a.num_kv_heads = (int32_t)Hkv; a.seq_len = (int32_t)S; a.head_dim = (int32_t)D;
    a.perm = c.perm.data_ptr<int64_t>(); a.perm_sh = c.perm_sh;
    a.cent = c.cent.data_ptr<float>(); a.cent_sh = c.cent_sh;
    a.metric = metric.defined() ? metric.data_ptr<float>() : nullptr; a.metric_sh = metric_sh;
    a.block_dim = (int32_t)c.bd; a.n_blocks = (int32_t)c.nb; a.n_centroids = (int32_t)c.nc;
    a.heavy_mask[0] = (uint64_t)hm0; a.heavy_mask[1] = (uint64_t)hm1;
    a.codes = reinterpret_cast<uint8_t*>(codes.data_ptr());
    a.c_sb = codes.stride(0); a.c_sh = codes.stride(1); a.c_st = codes.stride(2);
    a.pt_dtype = SSQ_F32;
    if (any_heavy) {
        a.pt = pt->data_ptr(); a.pt_dtype = dtype_code(*pt); a.pt_dense = pt_dense ? 1 : 0;
        a.pt_sb = pt->stride(0); a.pt_sh = pt->stride(1); a.pt_st = pt->stride(2);
    }
    if (paged) {
        a.slot_mapping = slot_mapping->data_ptr<int64_t>(); a.sm_sb = slot_mapping->stride(0);
        a.page_size = (int32_t)codes.size(2);
    }
    a.kernel = (int32_t)kernel;
    a.direct_dist = direct ? 1 : 0;
    if (grid.has_value() && grid->defined() && !direct) {
        on_gpu("grid", *grid);
        TORCH_CHECK(grid->scalar_type() == at::kByte && grid->is_contiguous(), "grid must be the uint8 tensor from encode_grid");
        a.grid = grid->data_ptr(); a.grid_bytes = (uint64_t)grid->numel();
    }
    check_status(ssq_encode(&a, stream_of(keys)));
}

}  // namespace

TORCH_LIBRARY(sunshape, m) {
    m.def("decode(Tensor q, Tensor codes, Tensor v, Tensor perm, Tensor cent, float? scale, Tensor? mask, int hm0, "
          "int hm1, Tensor? pt, bool pt_dense, Tensor? block_table, Tensor? seq_lens, bool return_lse, "
          "bool return_scores, int num_splits, int kernel, int code_bits, bool no_alloc) -> (Tensor, Tensor, Tensor)");
    m.def("scores(Tensor q, Tensor codes, Tensor perm, Tensor cent, float? scale, int hm0, int hm1, Tensor? pt, "
          "bool pt_dense, int code_bits, int num_splits, int kernel) -> Tensor");
    m.def("encode_into(Tensor keys, Tensor perm, Tensor cent, int hm0, int hm1, bool pt_dense, Tensor(a!) codes, "
          "Tensor(b!)? pt, Tensor? slot_mapping, Tensor? metric, Tensor? grid, int kernel, bool direct) -> ()");
}

TORCH_LIBRARY_IMPL(sunshape, CUDA, m) {
    m.impl("decode", &decode);
    m.impl("scores", &scores);
    m.impl("encode_into", &encode_into);
}
