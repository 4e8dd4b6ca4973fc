// Error plumbing, LUT build (test hook / standalone op) and dequantize.
#include "ssq_common.h"

#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>

namespace {
thread_local char g_err[512] = "";
}

int ssq_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ssq_check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return SSQ_OK;
    return ssq_fail(SSQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

extern "C" const char* ssq_last_error(void) { return g_err; }

// hipFuncSetAttribute applies per device: remember each (kernel, device) pair it was set for
int ssq_allow_lds(const void* fn, int bytes, const char* what) {
    static std::mutex mu;
    static struct {
        const void* fn;
        int dev, bytes;
    } done[512];
    static int n_done = 0;
    int dev = 0;
    int rc = ssq_check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n_done; ++i)
        if (done[i].fn == fn && done[i].dev == dev && done[i].bytes >= bytes) return SSQ_OK;
    rc = ssq_check_hip(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes), what);
    if (rc) return rc;
    if (n_done < 512) done[n_done++] = {fn, dev, bytes};
    return SSQ_OK;
}

int ssq_device_cus() {
    // per device, filled by the first caller; concurrent first calls store the same value
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}
extern "C" int ssq_abi_version(void) { return SSQ_ABI_VERSION; }

namespace {

// LUT[r, blk, c] = sum_d qp[r, blk*bd + d] * C[blk, c, d]  (fp32 FMA chain, dims ascending,
// the same arithmetic as the decode kernel's in-LDS build)
__global__ __launch_bounds__(256) void k_lut(const void* q, int q_dtype, int64_t q_sr, int head_dim,
                                             const int64_t* perm, const float* cent, int bd, int nc,
                                             int has_scale, float scale, float* lut) {
    extern __shared__ float qp[];
    const int r = blockIdx.y;
    for (int j = threadIdx.x; j < head_dim; j += blockDim.x) {
        float v = ssq_load_elem(q, q_dtype, (int64_t)r * q_sr + perm[j]);
        if (has_scale) v = ssq_round_to(v * scale, q_dtype);
        qp[j] = v;
    }
    __syncthreads();
    const int nb = head_dim / bd;
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nb * nc) return;
    const int blk = e / nc;
    const float* c = cent + (int64_t)e * bd;
    float acc = qp[blk * bd] * c[0];
    for (int d = 1; d < bd; ++d) acc = fmaf(qp[blk * bd + d], c[d], acc);
    lut[(int64_t)r * nb * nc + e] = acc;
}

// k_hat in the original basis: out[t, perm[i]] = k_perm[t, i]
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* codes, int64_t c_st, int tokens,
                                                 const int64_t* perm, const float* cent, int head_dim, int bd,
                                                 int nc, uint64_t hm0, uint64_t hm1, int pt_dense,
                                                 const void* pt, int pt_dtype, int64_t pt_st, float* out,
                                                 int64_t o_st) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (int64_t)tokens * head_dim) return;
    const int t = (int)(e / head_dim);
    const int i = (int)(e - (int64_t)t * head_dim);
    const int blk = i / bd, d = i - blk * bd;
    float v;
    if (ssq_is_heavy(hm0, hm1, blk)) {
        int slot = blk;
        if (!pt_dense)
            slot = blk < 64 ? __popcll(hm0 & ((1ull << blk) - 1ull))
                            : __popcll(hm0) + __popcll(hm1 & ((1ull << (blk - 64)) - 1ull));
        v = ssq_load_elem(pt, pt_dtype, (int64_t)t * pt_st + slot * bd + d);
    } else {
        uint32_t c = ssq_load_code(codes, ssq_code_width(nc), (int64_t)t * c_st + blk);
        if (c >= (uint32_t)nc) c = nc - 1;
        v = cent[((int64_t)blk * nc + c) * bd + d];
    }
    out[(int64_t)t * o_st + perm[i]] = v;
}

// Dense transform of rows (the rotated mode's x @ R^T and x @ R, codec.py:247-259):
// out[r, j] = sum_k xs[r, k] * m_jk with m_jk = M[j, k] (transpose 0) or M[k, j] (transpose 1),
// k ascending, the first product rounded, then fused multiply-adds; xs = x, or x * scale rounded
// to x's dtype (the query scaling of the decode).  A workgroup covers kTrCols output columns
// (gridDim.y chunks of them) for 256 / cw row lanes x kTrAcc rows; M and the rows are staged in
// LDS kTrK columns of k at a time.
constexpr int kTrThreads = 256;
constexpr int kTrAcc = 16;   // rows per thread
constexpr int kTrK = 32;     // k per LDS stage
constexpr int kTrRowsMax = kTrThreads / 64 * kTrAcc;

__global__ __launch_bounds__(kTrThreads) void k_transform_rows(const void* x, int x_dtype, int64_t x_sr, int64_t rows,
                                                               int dim, int cw, int has_scale, float scale,
                                                               const float* M, int transpose, float* out,
                                                               int64_t o_sr) {
    __shared__ float ms[kTrK][kTrThreads + 1];
    __shared__ float xs[kTrRowsMax][kTrK];
    const int t = threadIdx.x;
    const int lanes = kTrThreads / cw;
    const int c = t % cw, lane = t / cw;
    const int j0 = blockIdx.y * cw;
    const int j = j0 + c;
    const int wg_rows = lanes * kTrAcc;
    const int64_t r0 = (int64_t)blockIdx.x * wg_rows;
    float acc[kTrAcc];
#pragma unroll
    for (int i = 0; i < kTrAcc; ++i) acc[i] = 0.f;
    for (int k0 = 0; k0 < dim; k0 += kTrK) {
        const int kc = min(kTrK, dim - k0);
        __syncthreads();
        for (int e = t; e < cw * kTrK; e += kTrThreads) {
            int jj, kk;
            if (transpose) { kk = e / cw; jj = e - kk * cw; }     // M[k, j]: consecutive j
            else { jj = e / kTrK; kk = e - jj * kTrK; }           // M[j, k]: consecutive k
            const int gj = j0 + jj;
            float v = 0.f;
            if (gj < dim && kk < kc) v = transpose ? M[(int64_t)(k0 + kk) * dim + gj] : M[(int64_t)gj * dim + k0 + kk];
            ms[kk][jj] = v;
        }
        for (int e = t; e < wg_rows * kTrK; e += kTrThreads) {
            const int rr = e / kTrK, kk = e - rr * kTrK;
            const int64_t r = r0 + rr;
            float v = 0.f;
            if (r < rows && kk < kc) {
                v = ssq_load_elem(x, x_dtype, r * x_sr + k0 + kk);
                if (has_scale) v = ssq_round_to(v * scale, x_dtype);
            }
            xs[rr][kk] = v;
        }
        __syncthreads();
        for (int kk = 0; kk < kc; ++kk) {
            const float m = ms[kk][c];
            if (k0 + kk == 0) {
#pragma unroll
                for (int i = 0; i < kTrAcc; ++i) acc[i] = xs[lane + i * lanes][kk] * m;
            } else {
#pragma unroll
                for (int i = 0; i < kTrAcc; ++i) acc[i] = fmaf(xs[lane + i * lanes][kk], m, acc[i]);
            }
        }
    }
    if (j >= dim) return;
#pragma unroll
    for (int i = 0; i < kTrAcc; ++i) {
        const int64_t r = r0 + lane + i * lanes;
        if (r < rows) out[r * o_sr + j] = acc[i];
    }
}

}  // namespace

extern "C" int ssq_transform_rows(const void* x, int32_t x_dtype, int64_t x_sr, int64_t rows, int32_t dim,
                                  int32_t has_scale, float scale, const float* mat, int32_t transpose, float* out,
                                  int64_t o_sr, void* stream) {
    SSQ_REQUIRE(x_dtype >= SSQ_F32 && x_dtype <= SSQ_F16, "bad x_dtype");
    SSQ_REQUIRE(rows >= 0 && dim >= 1 && dim <= 4096, "bad rows / dim");
    SSQ_REQUIRE(x_sr >= dim && o_sr >= dim, "row strides too small");
    SSQ_REQUIRE(transpose == 0 || transpose == 1, "transpose must be 0 or 1");
    if (rows == 0) return SSQ_OK;
    SSQ_REQUIRE(x && mat && out, "x, mat and out must be non-NULL");
    const int cw = dim >= kTrThreads ? kTrThreads : (dim <= 64 ? 64 : (dim <= 128 ? 128 : kTrThreads));
    const int wg_rows = kTrThreads / cw * kTrAcc;
    const int64_t gx = (rows + wg_rows - 1) / wg_rows;
    SSQ_REQUIRE(gx <= 0x7fffffff, "too many rows");
    dim3 grid((unsigned)gx, (unsigned)((dim + cw - 1) / cw));
    hipLaunchKernelGGL(k_transform_rows, grid, dim3(kTrThreads), 0, (hipStream_t)stream, x, x_dtype, x_sr, rows, dim,
                       cw, has_scale, scale, mat, transpose, out, o_sr);
    return ssq_check_hip(hipGetLastError(), "k_transform_rows launch");
}

extern "C" int ssq_lut_build(const void* q, int32_t q_dtype, int64_t q_sr, int32_t rows, int32_t head_dim,
                             const int64_t* perm, const float* cent, int32_t block_dim, int32_t n_centroids,
                             int32_t has_scale, float scale, float* lut, void* stream) {
    SSQ_REQUIRE(q && perm && cent && lut, "NULL pointer argument");
    SSQ_REQUIRE(rows >= 1 && rows <= 65535, "rows out of range");
    SSQ_REQUIRE(block_dim >= 1 && head_dim % block_dim == 0 && head_dim <= 4096, "bad head_dim/block_dim");
    SSQ_REQUIRE(n_centroids >= 1 && n_centroids <= 65536, "bad n_centroids");
    SSQ_REQUIRE(q_dtype >= SSQ_F32 && q_dtype <= SSQ_F16, "bad q_dtype");
    const int nb = head_dim / block_dim;
    const int entries = nb * n_centroids;
    dim3 grid((entries + 255) / 256, rows);
    hipLaunchKernelGGL(k_lut, grid, dim3(256), head_dim * sizeof(float), (hipStream_t)stream, q, q_dtype, q_sr,
                       head_dim, perm, cent, block_dim, n_centroids, has_scale, scale, lut);
    return ssq_check_hip(hipGetLastError(), "k_lut launch");
}

extern "C" int ssq_dequantize(const uint8_t* codes, int64_t c_st, int32_t tokens, const int64_t* perm,
                              const float* cent, int32_t head_dim, int32_t block_dim, int32_t n_centroids,
                              const uint64_t* heavy_mask, int32_t pt_dense, const void* pt, int32_t pt_dtype,
                              int64_t pt_st, float* out, int64_t o_st, void* stream) {
    SSQ_REQUIRE(codes && perm && cent && out, "NULL pointer argument");
    SSQ_REQUIRE(block_dim >= 1 && head_dim % block_dim == 0, "head_dim must be divisible by block_dim");
    SSQ_REQUIRE(n_centroids >= 1 && n_centroids <= kMaxCentroids, "n_centroids must be in [1, %d]", kMaxCentroids);
    SSQ_REQUIRE(head_dim / block_dim <= 128, "n_blocks > 128");
    SSQ_REQUIRE(tokens >= 0, "negative token count");
    const uint64_t hm0 = heavy_mask ? heavy_mask[0] : 0, hm1 = heavy_mask ? heavy_mask[1] : 0;
    SSQ_REQUIRE(!(hm0 || hm1) || pt, "Mixed-precision quantized keys are missing passthrough values.");
    if (tokens == 0) return SSQ_OK;
    const int64_t n = (int64_t)tokens * head_dim;
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, codes, c_st,
                       tokens, perm, cent, head_dim, block_dim, n_centroids, hm0, hm1, pt_dense, pt, pt_dtype, pt_st,
                       out, o_st);
    return ssq_check_hip(hipGetLastError(), "k_dequant launch");
}

// ---------------------------------------------------------------------------
// sub-byte code packing: word p of a row holds blocks p*vpe .. p*vpe+vpe-1, vpe = 32 / bits,
// block p*vpe + v at bits [v*bits, (v+1)*bits)  (the layout sunshape/triton_kernels.py:250-266 reads)
// ---------------------------------------------------------------------------
namespace {

__global__ __launch_bounds__(256) void k_pack(const uint8_t* codes, int64_t c_st, int64_t rows, int nb, int bits,
                                              uint32_t* out, int64_t o_st) {
    const int vpe = 32 / bits;
    const int nw = (nb + vpe - 1) / vpe;
    const uint32_t msk = (1u << bits) - 1u;
    const int64_t total = rows * nw;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / nw;
        const int w = (int)(i - r * nw);
        uint32_t word = 0;
        for (int v = 0; v < vpe; ++v) {
            const int blk = w * vpe + v;
            if (blk < nb) word |= ((uint32_t)codes[r * c_st + blk] & msk) << (v * bits);
        }
        out[r * o_st + w] = word;
    }
}

__global__ __launch_bounds__(256) void k_unpack(const uint32_t* packed, int64_t p_st, int64_t rows, int nb, int bits,
                                                uint8_t* out, int64_t o_st) {
    const int vpe = 32 / bits;
    const uint32_t msk = (1u << bits) - 1u;
    const int64_t total = rows * nb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / nb;
        const int blk = (int)(i - r * nb);
        const int w = blk / vpe, v = blk - w * vpe;
        out[r * o_st + blk] = (uint8_t)((packed[r * p_st + w] >> (v * bits)) & msk);
    }
}

int grid_for(int64_t work) {
    const int64_t blocks = (work + 255) / 256;
    return (int)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace

extern "C" int ssq_pack_codes(const uint8_t* codes, int64_t c_st, int64_t rows, int32_t n_blocks, int32_t bits,
                              uint32_t* out, int64_t o_st, void* stream) {
    SSQ_REQUIRE(bits >= 1 && bits <= 8, "bits must be in [1, 8] for uint8 codes");
    SSQ_REQUIRE(rows >= 0 && n_blocks >= 1, "bad rows / n_blocks");
    const int nw = (n_blocks + 32 / bits - 1) / (32 / bits);
    SSQ_REQUIRE(c_st >= n_blocks && o_st >= nw, "row strides too small");
    if (rows == 0) return SSQ_OK;
    SSQ_REQUIRE(codes && out, "codes and out must be non-NULL");
    hipLaunchKernelGGL(k_pack, dim3(grid_for(rows * nw)), dim3(256), 0, (hipStream_t)stream, codes, c_st, rows,
                       n_blocks, bits, out, o_st);
    return ssq_check_hip(hipGetLastError(), "k_pack launch");
}

extern "C" int ssq_unpack_codes(const uint32_t* packed, int64_t p_st, int64_t rows, int32_t n_blocks, int32_t bits,
                                uint8_t* out, int64_t o_st, void* stream) {
    SSQ_REQUIRE(bits >= 1 && bits <= 8, "bits must be in [1, 8] for uint8 codes");
    SSQ_REQUIRE(rows >= 0 && n_blocks >= 1, "bad rows / n_blocks");
    const int nw = (n_blocks + 32 / bits - 1) / (32 / bits);
    SSQ_REQUIRE(p_st >= nw && o_st >= n_blocks, "row strides too small");
    if (rows == 0) return SSQ_OK;
    SSQ_REQUIRE(packed && out, "packed and out must be non-NULL");
    hipLaunchKernelGGL(k_unpack, dim3(grid_for(rows * n_blocks)), dim3(256), 0, (hipStream_t)stream, packed, p_st,
                       rows, n_blocks, bits, out, o_st);
    return ssq_check_hip(hipGetLastError(), "k_unpack launch");
}
