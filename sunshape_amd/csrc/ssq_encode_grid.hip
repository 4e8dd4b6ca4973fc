// Grid-search encode for block_dim 2 (no block metric): exact nearest codeword with the
// reference's rounding, evaluating only the codewords a cell grid certifies as possible winners.
//
// Reference semantics (sunshape/codec.py:362-385): code = first argmin_c sqrt(clamp_min(
// [-2x, |x|^2, 1] . [c, 1, |c|^2], 0)), the dot product a k-ascending FMA chain from the first
// product and the norms left-to-right sums of rounded squares (torch.cdist's mm formulation).
//
//  * k_grid_header / k_grid_cells (built once per codebook, ssq_encode_grid_build): per block, a
//    kG x kG grid of cells under a per-dimension map that is finest where the codewords crowd and
//    whose end cells reach to infinity (cell_edge).  Cell C lists, ascending, every codeword j
//    with dmin(C, c_j)^2 <= min_k dmax(C, c_k)^2 + M_C, where M_C bounds the rounding terms
//    below; more than 31 such codewords (or an unbounded cell) mark the cell "scan all".
//  * k_encode_grid: lane = key.  Per light block: the key's two permuted elements, its cell, the
//    cell's record (16 or 32 bytes from the grid), then the reference chain on each listed
//    candidate in ascending order, keeping the first minimum of the correctly rounded sqrt.
//    Non-finite keys and "scan all" cells evaluate every codeword.
//
// Why the list holds the winner.  Let r_j be the reference's value for codeword j, D_j the exact
// value of the same expression on the same (rounded) norms, d_j = |x - c_j|.  Then |r_j - D_j| <=
// e_j = g (|x| + |c_j|)^2 (1 + 2.001u) with g = 1.001 K 2^-23, K = bd + 2 (any rounding order),
// and D_j = d_j^2 + alpha + beta_j with |alpha| <= 2.001u|x|^2, |beta_j| <= 2.001u|c_j|^2, u = 2^-24.
// The winner j* has sqrt(max(r_j*, 0)) <= sqrt(max(r_k, 0)) for every k, so max(r_j*, 0) <=
// max(r_k, 0)(1 + 2^-21) (correctly rounded sqrt).  Chaining the bounds, for every k:
//   d_j*^2 <= d_k^2 + 2|alpha| + |beta_j*| + |beta_k| + e_j* + e_k + (d_k^2 + |alpha| + |beta_k| + e_k) 2^-21.
// For x in C (R = max |x| over C, Rc = max |c|): d_j*^2 >= dmin(C, c_j*)^2 and, for the k that
// minimises dmax(C, c_k), d_k^2 <= dmax(C, c_k)^2 =: dmm, giving dmin(C, c_j*)^2 <= dmm + M_C with
//   M_C = 1.01 (4.002u (R^2 + Rc^2) + 2.0002 g (R + Rc)^2 + (dmm + 2.001u (R^2 + Rc^2) + g (R + Rc)^2) 2^-21).
// Cells are widened by 0.001 of a cell on each side, far more than the fp32 rounding of the
// search kernel's cell map, so a key always lies in the cell it is looked up in.  The build
// runs in fp64.
#include "ssq_common.h"

#include <math.h>
#include <string.h>

namespace {

constexpr int kG = 128;        // cells per dimension
constexpr int kRec = 32;       // bytes per cell record: count (255 = scan all), then indices, padded
constexpr int kMaxCand = kRec - 1;
constexpr int kHdr = 8;        // floats per block header: mid0, mid1, inv0, inv1, Rc, valid, fingerprint
constexpr int kThreads = 256;

// Layout, head-major: per codebook head, its block headers (padded to 256 bytes) then its cells, so
// one head's part of a per-KV-head grid is itself the grid of that head's codebook.
inline int grid_heads(const ssq_encode_args& a) { return a.cent_sh == 0 ? 1 : a.num_kv_heads; }
__host__ __device__ inline size_t grid_head_hdr_bytes(int nb) { return ((size_t)nb * kHdr * 4 + 255) & ~(size_t)255; }
__host__ __device__ inline size_t grid_head_bytes(int nb) {
    return grid_head_hdr_bytes(nb) + (size_t)nb * kG * kG * kRec;
}
inline size_t grid_total_bytes(const ssq_encode_args& a) { return (size_t)grid_heads(a) * grid_head_bytes(a.n_blocks); }

// ---------------------------------------------------------------------------
// build
// ---------------------------------------------------------------------------
// Order-free fingerprint of one block's codebook (fp32 bit patterns, indices, count).  The
// builder stores it in the block's header; the search recomputes it from the codebook it is
// given and scans every codeword of a block whose fingerprint differs, so a grid built for
// another codebook costs time, never correctness (barring a 32-bit collision).
__device__ __forceinline__ uint32_t cw_mix(float c0, float c1, int j) {
    const uint32_t a = __float_as_uint(c0), b = __float_as_uint(c1);
    uint32_t h = ((a << 7) | (a >> 25)) ^ (b * 0x9E3779B1u) ^ ((uint32_t)j * 0x85EBCA77u);
    h ^= h >> 15;
    h *= 0x2C1B3C6Du;
    h ^= h >> 12;
    return h;
}
__device__ __forceinline__ uint32_t cw_count_mix(int nc) { return (uint32_t)nc * 0xC2B2AE35u; }

// one lane per (block, codebook head), in fp64: the cell map's centre (the codewords' bounding-box
// centre) and scale (their RMS spread about the mean) per dimension, and max |c|
__global__ __launch_bounds__(64) void k_grid_header(const float* cent, int64_t cent_sh, int nb, int nc, uint8_t* grid) {
    if (threadIdx.x != 0) return;
    const int blk = blockIdx.x, h = blockIdx.y;
    const float* c = cent + (int64_t)h * cent_sh + (int64_t)blk * nc * 2;
    double lo[2] = {INFINITY, INFINITY}, hi[2] = {-INFINITY, -INFINITY}, sum[2] = {0.0, 0.0};
    double nrm = 0.0;
    bool finite = true;
    for (int j = 0; j < nc; ++j) {
        for (int d = 0; d < 2; ++d) {
            const double v = c[2 * j + d];
            lo[d] = fmin(lo[d], v); hi[d] = fmax(hi[d], v); sum[d] += v;
            finite = finite && isfinite(v);
        }
        nrm = fmax(nrm, (double)(float)((double)c[2 * j] * c[2 * j] + (double)c[2 * j + 1] * c[2 * j + 1]));
    }
    float mid[2], inv[2];
    bool valid = finite;
    for (int d = 0; d < 2; ++d) {
        const double mean = sum[d] / nc;
        double var = 0.0;
        for (int j = 0; j < nc; ++j) {
            const double e = (double)c[2 * j + d] - mean;
            var += e * e;
        }
        const double m = 0.5 * (lo[d] + hi[d]);
        double sc = sqrt(var / nc);
        if (!(sc > fabs(m) * 0x1.0p-20)) sc = fmax(fabs(m) * 0x1.0p-20, 0x1.0p-60);
        mid[d] = (float)m;
        inv[d] = (float)(1.0 / sc);
        valid = valid && isfinite(mid[d]) && isfinite(inv[d]) && inv[d] > 0.f;
    }
    float* out = reinterpret_cast<float*>(grid + (size_t)h * grid_head_bytes(nb)) + (int64_t)blk * kHdr;
    out[0] = mid[0]; out[1] = mid[1]; out[2] = inv[0]; out[3] = inv[1];
    uint32_t fp = cw_count_mix(nc);
    for (int j = 0; j < nc; ++j) fp ^= cw_mix(c[2 * j], c[2 * j + 1], j);
    out[4] = finite ? (float)(sqrt(nrm) * (1.0 + 0x1.0p-20)) : INFINITY;
    out[5] = valid ? 1.f : 0.f;
    out[6] = __uint_as_float(fp);
    out[7] = 0.f;
}

// The cell map, per dimension: u = (x - mid) inv, t = u / (1 + |u|) in (-1, 1), cell
// floor((t + 1) kG / 2) clamped to [0, kG).  Cells are finest at the centre, where keys and
// codewords crowd, and the two end cells reach to infinity, so every finite key has a cell.
// The search computes t in fp32 with an approximate reciprocal, within 1e-6 of t; each cell is
// widened by 0.001 of its width in t, far more.
__device__ __forceinline__ double cell_edge(double t, double mid, double scale) {
    if (t <= -1.0) return -INFINITY;
    if (t >= 1.0) return INFINITY;
    return mid + scale * (t / (1.0 - fabs(t)));
}

// one thread per cell
__global__ __launch_bounds__(kThreads) void k_grid_cells(const float* cent, int64_t cent_sh, int nb, int nc,
                                                         uint8_t* grid) {
    __shared__ double cw[256][2];
    const int blk = blockIdx.y, h = blockIdx.z, tid = threadIdx.x;
    const int cell = blockIdx.x * kThreads + tid;
    const float* c = cent + (int64_t)h * cent_sh + (int64_t)blk * nc * 2;
    for (int j = tid; j < nc; j += kThreads) { cw[j][0] = c[2 * j]; cw[j][1] = c[2 * j + 1]; }
    __syncthreads();
    uint8_t* head = grid + (size_t)h * grid_head_bytes(nb);
    const float* hd = reinterpret_cast<const float*>(head) + (int64_t)blk * kHdr;
    uint8_t rec[kRec];
#pragma unroll
    for (int i = 0; i < kRec; ++i) rec[i] = 0;
    if (hd[5] == 0.f) {
        rec[0] = 255;
    } else {
        const int i0 = cell / kG, i1 = cell - (cell / kG) * kG;
        const double w = 2.0 / kG, sc0 = 1.0 / (double)hd[2], sc1 = 1.0 / (double)hd[3];
        const double a0 = cell_edge(-1.0 + w * (i0 - 0.001), hd[0], sc0);
        const double b0 = cell_edge(-1.0 + w * (i0 + 1.001), hd[0], sc0);
        const double a1 = cell_edge(-1.0 + w * (i1 - 0.001), hd[1], sc1);
        const double b1 = cell_edge(-1.0 + w * (i1 + 1.001), hd[1], sc1);
        const double R2 = fmax(a0 * a0, b0 * b0) + fmax(a1 * a1, b1 * b1);
        const double R = sqrt(R2), Rc = hd[4];
        double dmm = INFINITY;
        for (int j = 0; j < nc; ++j) {
            const double dx = fmax(fabs(a0 - cw[j][0]), fabs(b0 - cw[j][0]));
            const double dy = fmax(fabs(a1 - cw[j][1]), fabs(b1 - cw[j][1]));
            dmm = fmin(dmm, dx * dx + dy * dy);
        }
        const double u = 0x1.0p-24, g = 1.001 * 4 * 0x1.0p-23;  // K = bd + 2 = 4
        const double S = (R + Rc) * (R + Rc), N2 = R2 + Rc * Rc;
        const double M = 1.01 * (4.002 * u * N2 + 2.0002 * g * S + (dmm + 2.001 * u * N2 + g * S) * 0x1.0p-21);
        const double bound = dmm + M;
        int cnt = 0;
        for (int j = 0; j < nc; ++j) {
            const double dx = fmax(fmax(a0 - cw[j][0], cw[j][0] - b0), 0.0);
            const double dy = fmax(fmax(a1 - cw[j][1], cw[j][1] - b1), 0.0);
            if (dx * dx + dy * dy <= bound) {
                if (cnt < kMaxCand) rec[1 + cnt] = (uint8_t)j;
                ++cnt;
            }
        }
        // count 0 (non-finite values) or more than 31: scan all.  Bytes past the list repeat
        // its last index, so evaluating them again cannot change the search's result.
        if (cnt == 0 || cnt > kMaxCand) {
            rec[0] = 255;
        } else {
            rec[0] = (uint8_t)cnt;
            for (int i = 1 + cnt; i < kRec; ++i) rec[i] = rec[cnt];
        }
    }
    uint4* dst = reinterpret_cast<uint4*>(head + grid_head_hdr_bytes(nb) + ((int64_t)blk * kG * kG + cell) * kRec);
    const uint32_t* w = reinterpret_cast<const uint32_t*>(rec);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// ---------------------------------------------------------------------------
// search
// ---------------------------------------------------------------------------
constexpr int kMaxLight = 128;

struct GridParams {
    ssq_encode_args a;
    const uint8_t* grid;       // head-major: headers then cells per codebook head
    int n_light;
    int row_codes;             // whole code rows in 16-byte stores
    int row_q;                 // 16-byte pieces of a key row when rows are read whole (else 0)
    int fold;                  // short sequences: all sequences of a KV head share one key range (SsqKeyMap)
    int nlc;                   // light blocks per workgroup chunk (blockIdx.z picks the chunk)
    uint8_t light[kMaxLight];  // light block ids, ascending
};

// LDS layout (bytes): cb [nl][256] float2 | cn [nl][256] float | hd [nl] float4 | poff [nl][4] int |
// codes [waves][64][nb]
inline size_t grid_smem(int nl, int nb, int waves) {
    return (size_t)nl * 256 * 12 + (size_t)nl * 16 + (size_t)nl * 16 + (size_t)nb * 16 + (size_t)waves * 64 * nb;
}

struct Cand {  // running first minimum of sqrt(max(d2, 0)) over ascending codeword indices
    float bd;  // clamped pre-sqrt value of the best so far
    int bj;
};

// the reference's chain for codeword (c, |c|^2) of index j, then the first-minimum update
// (ok = false leaves the state alone)
__device__ __forceinline__ void eval_val(float2 c, float cq, int j, float m0, float m1, float xn, bool ok,
                                         Cand& st) {
    float d2 = m0 * c.x;                     // (-2 x0) c0, rounded
    d2 = __builtin_fmaf(m1, c.y, d2);        // + (-2 x1) c1
    d2 = __builtin_fmaf(xn, 1.0f, d2);       // + |x|^2 . 1
    d2 = __builtin_fmaf(1.0f, cq, d2);       // + 1 . |c|^2
    const float dc = d2 > 0.f ? d2 : 0.f;
    // dc < bd (1 - 2^-20) gives a strictly smaller correctly rounded sqrt; values within
    // (1 +- 2^-20) of bd compare their square roots; anything larger loses
    // (bitwise operators, a wave-uniform test and an opaque statement: one rarely taken branch,
    // which the compiler would otherwise flatten into two correctly rounded square roots per
    // candidate)
    bool take = (st.bj < 0) | (dc < st.bd * (1.0f - 0x1.0p-20f));
    const bool near = ok & !take & (dc <= st.bd * (1.0f + 0x1.0p-20f));
    if (__builtin_amdgcn_ballot_w64(near)) {
        __asm__ volatile("" ::: "memory");  // keeps the branch: not speculated
        const bool lt = __builtin_sqrtf(dc) < __builtin_sqrtf(st.bd);
        take = near ? lt : take;
    }
    take &= ok;
    st.bd = take ? dc : st.bd;
    st.bj = take ? j : st.bj;
}


// the reference's value for codeword (c, |c|^2), clamped at 0
__device__ __forceinline__ float chain_val(float2 c, float cq, float m0, float m1, float xn) {
    float d2 = m0 * c.x;
    d2 = __builtin_fmaf(m1, c.y, d2);
    d2 = __builtin_fmaf(xn, 1.0f, d2);
    d2 = __builtin_fmaf(1.0f, cq, d2);
    return d2 > 0.f ? d2 : 0.f;
}

// A later candidate of a cell list: taken iff its correctly rounded sqrt is strictly smaller.
// Both values are non-negative floats, so their bit patterns order like the values.  A gap
// of more than 32 units in the last place of the smaller one makes the ratio exceed
// 1 + 33 2^-24, the square roots' ratio 1 + 16 2^-24, and so the correctly rounded roots
// differ; a smaller value within 32 units compares the roots; an equal or larger one loses.
// Re-evaluating a codeword already seen (the record's padding) always loses.
__device__ __forceinline__ void next_val(float2 c, float cq, int j, float m0, float m1, float xn, Cand& st) {
    const float dc = chain_val(c, cq, m0, m1, xn);
    const int diff = (int)__float_as_uint(st.bd) - (int)__float_as_uint(dc);
    bool take = diff > 32;
    const bool near = (uint32_t)(diff - 1) < 32u;
    if (__builtin_amdgcn_ballot_w64(near)) {
        __asm__ volatile("" ::: "memory");  // keeps the branch: not speculated
        const bool lt = __builtin_sqrtf(dc) < __builtin_sqrtf(st.bd);
        take = near ? lt : take;
    }
    st.bd = take ? dc : st.bd;
    st.bj = take ? j : st.bj;
}

template <bool ROWREG>
__global__ __launch_bounds__(1024) void k_encode_grid(const GridParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_encode_args& a = p.a;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int waves = blockDim.x >> 6;
    const SsqKeyMap km(a, p.fold);
    const int kv = km.kv;
    const int l0 = blockIdx.z * p.nlc;  // this chunk's first light block
    const int nl = min(p.nlc, p.n_light - l0), nb = a.n_blocks, nc = a.n_centroids;
    const int hsel = a.cent_sh == 0 ? 0 : kv;

    float2* cb = reinterpret_cast<float2*>(smem);                          // [nl][256]
    float* cn = reinterpret_cast<float*>(cb + nl * 256);                   // [nl][256]
    float4* hd = reinterpret_cast<float4*>(cn + nl * 256);                 // [nl]: lo0, lo1, inv_h0, inv_h1
    int* poff = reinterpret_cast<int*>(hd + nl);                           // [nl]: perm0, perm1, block id, 0
    // [heavy blocks]: the block's two dims in the key row, its id, its passthrough slot (chunk 0)
    int4* hinfo = reinterpret_cast<int4*>(poff + 4 * nl);
    uint8_t* cs = reinterpret_cast<uint8_t*>(hinfo + nb) + wave * 64 * nb;  // this wave's code rows

    const int keys_wg = waves * 64;
    const int key = blockIdx.x * keys_wg + wave * 64 + lane;  // this lane's key index
    const bool live = key < km.n_keys;
    const int64_t krow = km.krow(a, live ? key : km.n_keys - 1);
    // this lane's key's output rows (code row, passthrough row), resolved before the staging so
    // that a slot-mapping load is not a round trip at the end
    int64_t crow_k, prow_k;
    {
        int b, ss;
        km.bs(a, live ? key : km.n_keys - 1, b, ss);
        if (a.slot_mapping) {
            const int64_t slot = a.slot_mapping[(int64_t)b * a.sm_sb + ss];
            const int64_t page = slot / a.page_size, off = slot - page * a.page_size;
            crow_k = page * a.c_sb + (int64_t)kv * a.c_sh + off * a.c_st;
            prow_k = page * a.pt_sb + (int64_t)kv * a.pt_sh + off * a.pt_st;
        } else {
            crow_k = (int64_t)b * a.c_sb + (int64_t)kv * a.c_sh + (int64_t)ss * a.c_st;
            prow_k = (int64_t)b * a.pt_sb + (int64_t)kv * a.pt_sh + (int64_t)ss * a.pt_st;
        }
    }

    const int kdt = a.k_dtype;
    // ---- the key's permuted elements, issued before the staging below (they do not depend on
    // it; issued after its barrier they would add a memory round trip to the chain).  ROWREG: the
    // whole row (at most 128 bytes, 16-byte aligned) is loaded once with 16-byte loads into
    // registers, and each block's two elements are picked out by a wave-uniform register index:
    // one memory access per 16 bytes of key instead of one per element.  Otherwise each element
    // is a load of its own, issued one block ahead of its use.
    uint32_t row[32];
    if constexpr (ROWREG) {
        const uint4* src = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.keys) +
                                                          krow * (kdt == SSQ_F32 ? 4 : 2));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 v = i < p.row_q ? src[i] : make_uint4(0u, 0u, 0u, 0u);
            row[4 * i] = v.x; row[4 * i + 1] = v.y; row[4 * i + 2] = v.z; row[4 * i + 3] = v.w;
        }
    }
    // ---- stage the light blocks, one wave per block: codewords, |c|^2 (rounded squares summed
    // left to right), the header, and the codebook fingerprint check (a grid built for another
    // codebook leaves the block without cells: every key scans all codewords)
    const float* cent = a.cent + (int64_t)kv * a.cent_sh;
    const int64_t* perm = a.perm + (int64_t)kv * a.perm_sh;
    for (int li = wave; li < nl; li += waves) {
        const int blk = p.light[l0 + li];
        const float* c = cent + (int64_t)blk * nc * 2;
        // every load of the block first (codewords, header, permutation entries), then arithmetic
        const float4* h4 = reinterpret_cast<const float4*>(p.grid + (size_t)hsel * grid_head_bytes(nb)) +
                           (int64_t)blk * (kHdr / 4);
        const float4 hA = h4[0], hB = h4[1];  // mid0, mid1, inv0, inv1 | Rc, valid, fingerprint, -
        const int64_t pe0 = perm[blk * 2], pe1 = perm[blk * 2 + 1];
        float v0[4], v1[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = lane + 64 * q;
            v0[q] = j < nc ? c[2 * j] : 0.f;
            v1[q] = j < nc ? c[2 * j + 1] : 0.f;
        }
        uint32_t f = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = lane + 64 * q;
            if (j < nc) {
                cb[li * 256 + j] = make_float2(v0[q], v1[q]);
                const float t0 = v0[q] * v0[q], t1 = v1[q] * v1[q];
                cn[li * 256 + j] = t0 + t1;
                f ^= cw_mix(v0[q], v1[q], j);
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) f ^= __shfl_xor(f, o);
        if (lane == 0) {
            const bool ok = hB.y != 0.f && (f ^ cw_count_mix(nc)) == __float_as_uint(hB.z);
            hd[li] = ok ? hA : make_float4(0.f, 0.f, 0.f, 0.f);
            poff[4 * li] = (int)pe0;
            poff[4 * li + 1] = (int)pe1;
            poff[4 * li + 2] = blk;  // kept in LDS: a kernel-argument array indexed in the loop
            poff[4 * li + 3] = 0;    // would be a memory load that waits for every pending load
        }
    }
    if (blockIdx.z == 0 && (a.heavy_mask[0] | a.heavy_mask[1])) {  // chunk 0 copies the heavy blocks
        const uint64_t h0 = a.heavy_mask[0], h1 = a.heavy_mask[1];
        for (int blk = threadIdx.x; blk < nb; blk += blockDim.x) {
            if (!ssq_is_heavy(h0, h1, blk)) continue;
            const int h = blk < 64 ? __popcll(h0 & ((1ull << blk) - 1ull))  // heavy blocks before blk
                                   : __popcll(h0) + __popcll(h1 & ((1ull << (blk - 64)) - 1ull));
            hinfo[h] = make_int4((int)perm[2 * blk], (int)perm[2 * blk + 1], blk, a.pt_dense ? blk : h);
        }
    }
    for (int i = lane; i < 16 * nb; i += 64) reinterpret_cast<uint32_t*>(cs)[i] = 0u;  // heavy blocks: code 0
    __syncthreads();

    const uint64_t hm0 = a.heavy_mask[0], hm1 = a.heavy_mask[1];
    const uint8_t* cells = p.grid + (size_t)hsel * grid_head_bytes(nb) + grid_head_hdr_bytes(nb);
    // element e (wave-uniform) of the register row, as raw bits
    auto row_bits = [&](int e) -> uint32_t {
        if (kdt == SSQ_F32) return row[e & 31];
        const uint32_t w = row[(e >> 1) & 31];
        return (e & 1) ? (w >> 16) : (w & 0xffffu);
    };
    // light block li's permuted element positions and block id, wave-uniform
    auto block_info = [&](int li, int& e0, int& e1, int& blk) {
        const int4 v = reinterpret_cast<const int4*>(poff)[li];
        e0 = __builtin_amdgcn_readfirstlane(v.x);
        e1 = __builtin_amdgcn_readfirstlane(v.y);
        blk = __builtin_amdgcn_readfirstlane(v.z);
    };
    // the byte offset of (x0, x1)'s cell record in block blk of this head's table; inside =
    // false means "scan all" (the offset is then cell (0, 0)'s, a valid record)
    auto cell_off = [&](int li, int blk, float x0, float x1, bool& inside) -> uint32_t {
        const float4 h = hd[li];  // mid0, mid1, inv0, inv1 (inv 0: no grid)
        const float u0 = (x0 - h.x) * h.z, u1 = (x1 - h.y) * h.w;
        const float t0 = u0 * __builtin_amdgcn_rcpf(1.0f + fabsf(u0));
        const float t1 = u1 * __builtin_amdgcn_rcpf(1.0f + fabsf(u1));
        const float f0 = floorf((t0 + 1.0f) * (0.5f * kG)), f1 = floorf((t1 + 1.0f) * (0.5f * kG));
        // t within rounding of +-1 may land one past the ends: the end cells take it.  NaN
        // (a non-finite key element) has no cell
        inside = h.z > 0.f && f0 >= -1.f && f0 <= (float)kG && f1 >= -1.f && f1 <= (float)kG;
        const int c0 = inside ? min(max((int)f0, 0), kG - 1) : 0, c1 = inside ? min(max((int)f1, 0), kG - 1) : 0;
        return (uint32_t)((blk * kG * kG + c0 * kG + c1) * kRec);
    };
    auto rec_lo = [&](uint32_t off) { return *reinterpret_cast<const uint4*>(cells + off); };
    auto rec_hi = [&](uint32_t off) { return *reinterpret_cast<const uint4*>(cells + off + 16); };
    // lists of 16 to 31 candidates continue in the record's second 16 bytes
    auto needs_hi = [](const uint4& r, bool inside) {
        const uint32_t c = r.x & 255u;
        return inside && c > 15u && c != 255u;
    };
    const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);

    // Software pipeline over the light blocks, one block apart: at trip li the loads of trip
    // li - 1 have landed; the trip issues the second half of block li + 1's record (lanes
    // with long lists only) and the first half of block li + 2's, then evaluates block li.
    // Indices past the last block are clamped to it.  Stage names: *0 = block li, *1 = li + 1.
    float xa0 = 0.f, xb0 = 0.f, xa1 = 0.f, xb1 = 0.f;
    uint4 lo0 = zero4, lo1 = zero4, hi0 = zero4;
    uint32_t off1 = 0;
    bool in0 = false, in1 = false;
    uint32_t ua = 0, ub = 0;  // element path: raw bits of block li + 2
    auto elems = [&](int li, float& x0, float& x1, int& blk) {
        int e0, e1;
        block_info(li, e0, e1, blk);
        if constexpr (ROWREG) {
            x0 = ssq_bits_to_f32(row_bits(e0), kdt);
            x1 = ssq_bits_to_f32(row_bits(e1), kdt);
        } else {
            x0 = ssq_load_elem(a.keys, kdt, krow + e0);
            x1 = ssq_load_elem(a.keys, kdt, krow + e1);
        }
    };
    auto issue_bits = [&](int li) {
        if constexpr (!ROWREG) {
            const int4 v = reinterpret_cast<const int4*>(poff)[li];
            ua = ssq_load_bits(a.keys, kdt, krow + __builtin_amdgcn_readfirstlane(v.x));
            ub = ssq_load_bits(a.keys, kdt, krow + __builtin_amdgcn_readfirstlane(v.y));
        }
    };
    if (nl > 0) {
        int blk;
        elems(0, xa0, xb0, blk);
        const uint32_t off0 = cell_off(0, blk, xa0, xb0, in0);
        lo0 = rec_lo(off0);
        elems(min(1, nl - 1), xa1, xb1, blk);
        off1 = cell_off(min(1, nl - 1), blk, xa1, xb1, in1);
        lo1 = rec_lo(off1);
        issue_bits(min(2, nl - 1));
        if (needs_hi(lo0, in0)) {
            hi0 = rec_hi(off0);
        } else {
            const uint32_t pad = (lo0.w >> 24) * 0x01010101u;
            hi0 = make_uint4(pad, pad, pad, pad);
        }
    }
    for (int li = 0; li < nl; ++li) {
        // ---- block li + 1: the record's second half where the list needs it
        uint4 hi1;
        if (needs_hi(lo1, in1)) {
            hi1 = rec_hi(off1);
        } else {  // the list ends in the first half: its padding continues
            const uint32_t pad = (lo1.w >> 24) * 0x01010101u;
            hi1 = make_uint4(pad, pad, pad, pad);
        }
        // ---- block li + 2: key elements, cell, the record's first half
        const int l2 = min(li + 2, nl - 1);
        float xa2, xb2;
        int blk2;
        if constexpr (ROWREG) {
            elems(l2, xa2, xb2, blk2);
        } else {
            int e0, e1;
            block_info(l2, e0, e1, blk2);
            xa2 = ssq_bits_to_f32(ua, kdt);
            xb2 = ssq_bits_to_f32(ub, kdt);
            issue_bits(min(li + 3, nl - 1));
        }
        bool in2;
        const uint32_t off2 = cell_off(l2, blk2, xa2, xb2, in2);
        const uint4 lo2 = rec_lo(off2);

        // ---- candidates of block li
        const float m0 = -2.0f * xa0, m1 = -2.0f * xb0;
        const float xn = xa0 * xa0 + xb0 * xb0;
        const float2* cbl = cb + li * 256;
        const float* cnl = cn + li * 256;
        const uint32_t w[8] = {lo0.x, lo0.y, lo0.z, lo0.w, hi0.x, hi0.y, hi0.z, hi0.w};
        const int cnt = (int)(w[0] & 255u);
        const bool full = !in0 || cnt == 255;
        const int lcnt = full ? 0 : cnt;
        Cand st{INFINITY, -1};
        // Record word g holds bytes 4g .. 4g+3, candidates 4g-1 .. 4g+2 (byte 0 is the count).
        // The codewords of word g + 1 are read while word g is evaluated, so each word costs one
        // LDS latency, not four.  The first candidate starts the running minimum; bytes past a
        // lane's count repeat its last candidate and cannot win.  Lanes that scan all codewords
        // start over below.
        float2 cc[4];
        float cq[4];
        auto fetch = [&](uint32_t wd, int i0, float2 (&c)[4], float (&q)[4]) {
#pragma unroll
            for (int i = i0; i < 4; ++i) {
                const int j = (int)((wd >> (8 * i)) & 255u);
                c[i] = cbl[j];
                q[i] = cnl[j];
            }
        };
        fetch(w[0], 1, cc, cq);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            if (!__builtin_amdgcn_ballot_w64((g == 0 ? 0 : 4 * g - 1) < lcnt)) break;  // the wave's lists are done
            float2 nc2[4];
            float nq[4];
            if (g < 7) fetch(w[g + 1], 0, nc2, nq);
#pragma unroll
            for (int i = (g == 0 ? 1 : 0); i < 4; ++i) {
                const int j = (int)((w[g] >> (8 * i)) & 255u);
                if (g == 0 && i == 1) {
                    st.bd = chain_val(cc[i], cq[i], m0, m1, xn);
                    st.bj = j;
                } else {
                    next_val(cc[i], cq[i], j, m0, m1, xn, st);
                }
            }
            if (g < 7) {
#pragma unroll
                for (int i = 0; i < 4; ++i) { cc[i] = nc2[i]; cq[i] = nq[i]; }
            }
        }
        if (__builtin_amdgcn_ballot_w64(full)) {  // rare: every codeword, 8 read ahead of their use
            if (full) st = Cand{INFINITY, -1};
            for (int j0 = 0; j0 < nc; j0 += 8) {
                float2 c8[8];
                float q8[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int j = min(j0 + u, nc - 1);
                    c8[u] = cbl[j];
                    q8[u] = cnl[j];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) eval_val(c8[u], q8[u], j0 + u, m0, m1, xn, full && j0 + u < nc, st);
            }
        }
        cs[lane * nb + __builtin_amdgcn_readfirstlane(poff[4 * li + 2])] = (uint8_t)(st.bj < 0 ? 0 : st.bj);

        // ---- rotate the stages
        xa0 = xa1; xb0 = xb1; lo0 = lo1; hi0 = hi1; in0 = in1;
        xa1 = xa2; xb1 = xb2; lo1 = lo2; off1 = off2; in1 = in2;
    }

    // ---- outputs: code rows, heavy blocks' passthrough values
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int s_wave = blockIdx.x * keys_wg + wave * 64;
    if (p.row_codes) {
        const int pieces = nb >> 4;
        for (int e = lane; e < 64 * pieces; e += 64) {
            const int m = e / pieces, q = e - m * pieces;
            const int i = s_wave + m;
            // key m's code row, from lane m
            const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)crow_k, m);
            const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)((uint64_t)crow_k >> 32), m);
            const int64_t crow = (int64_t)(((uint64_t)hi << 32) | lo);
            if (i < km.n_keys) {
                const uint32_t* src = reinterpret_cast<const uint32_t*>(cs + m * nb + 16 * q);
                *reinterpret_cast<uint4*>(a.codes + crow + 16 * q) = make_uint4(src[0], src[1], src[2], src[3]);
            }
        }
    } else if (live && gridDim.z == 1) {  // every block's code (heavy blocks' 0 included)
        const int64_t crow = crow_k;
        for (int blk = 0; blk < nb; ++blk) a.codes[crow + blk] = cs[lane * nb + blk];
    } else if (live) {  // one chunk of several: its blocks' codes; chunk 0 also the heavy blocks' 0
        const int64_t crow = crow_k;
        for (int li = 0; li < nl; ++li) {
            const int blk = __builtin_amdgcn_readfirstlane(poff[4 * li + 2]);
            a.codes[crow + blk] = cs[lane * nb + blk];
        }
    }
    // chunk 0: the heavy blocks' values as the key holds them, and (with several chunks, whose
    // stores are per block) their code 0.  One pass over the heavy blocks listed in LDS, the
    // stored dtype's branch taken once.
    if ((hm0 | hm1) && live && blockIdx.z == 0) {
        const int nh = __popcll(hm0) + __popcll(hm1);
        const bool zero_codes = gridDim.z > 1;
        auto heavy_pair = [&](int h, int& blk, int& slot, float& x0, float& x1) {
            const int4 hi = hinfo[h];
            const int e0 = __builtin_amdgcn_readfirstlane(hi.x), e1 = __builtin_amdgcn_readfirstlane(hi.y);
            blk = __builtin_amdgcn_readfirstlane(hi.z);
            slot = __builtin_amdgcn_readfirstlane(hi.w);
            if constexpr (ROWREG) {
                x0 = ssq_bits_to_f32(row_bits(e0), kdt);
                x1 = ssq_bits_to_f32(row_bits(e1), kdt);
            } else {
                x0 = ssq_load_elem(a.keys, kdt, krow + e0);
                x1 = ssq_load_elem(a.keys, kdt, krow + e1);
            }
        };
        if (a.pt_dtype == SSQ_F32) {
            float* dst = reinterpret_cast<float*>(a.pt) + prow_k;
            for (int h = 0; h < nh; ++h) {
                int blk, slot;
                float x0, x1;
                heavy_pair(h, blk, slot, x0, x1);
                if (zero_codes) a.codes[crow_k + blk] = 0;
                dst[2 * slot] = x0;
                dst[2 * slot + 1] = x1;
            }
        } else {
            const bool bf = a.pt_dtype == SSQ_BF16;
            uint16_t* dst = reinterpret_cast<uint16_t*>(a.pt) + prow_k;
            for (int h = 0; h < nh; ++h) {
                int blk, slot;
                float x0, x1;
                heavy_pair(h, blk, slot, x0, x1);
                if (zero_codes) a.codes[crow_k + blk] = 0;
                dst[2 * slot] = (uint16_t)(bf ? ssq_f32_to_bf16(x0) : ssq_f32_to_f16(x0));
                dst[2 * slot + 1] = (uint16_t)(bf ? ssq_f32_to_bf16(x1) : ssq_f32_to_f16(x1));
            }
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
bool ssq_encode_grid_supported(const ssq_encode_args* a) {
    return a->block_dim == 2 && !a->metric && a->n_centroids >= 1 && a->n_centroids <= 256 && a->n_blocks <= 128;
}


extern "C" uint64_t ssq_encode_grid_bytes(const ssq_encode_args* a) {
    if (!a || a->struct_size != sizeof(ssq_encode_args) || !ssq_encode_grid_supported(a) || a->n_blocks < 1 ||
        a->num_kv_heads < 1)
        return 0;
    return grid_total_bytes(*a);
}

extern "C" int ssq_encode_grid_build(const ssq_encode_args* a, void* grid, uint64_t grid_bytes, void* stream) {
    if (!a) return ssq_fail(SSQ_ERR_INVALID, "args is NULL");
    if (a->struct_size != sizeof(ssq_encode_args))
        return ssq_fail(SSQ_ERR_ABI, "ssq_encode_args size %u != library's %zu", a->struct_size, sizeof(ssq_encode_args));
    SSQ_REQUIRE(a->cent && grid, "cent and grid must be non-NULL");
    SSQ_REQUIRE((uintptr_t)grid % 16 == 0, "the grid must be 16-byte aligned");
    SSQ_REQUIRE(a->n_blocks >= 1 && a->num_kv_heads >= 1, "bad n_blocks/num_kv_heads");
    SSQ_UNSUPPORTED(ssq_encode_grid_supported(a), "the encode grid serves block_dim 2 without a block metric");
    SSQ_REQUIRE(grid_bytes >= grid_total_bytes(*a), "grid buffer too small (%llu < %zu bytes)",
                (unsigned long long)grid_bytes, grid_total_bytes(*a));
    hipStream_t st = (hipStream_t)stream;
    const int nh = grid_heads(*a), nb = a->n_blocks, nc = a->n_centroids;
    uint8_t* g = static_cast<uint8_t*>(grid);
    hipLaunchKernelGGL(k_grid_header, dim3(nb, nh), dim3(64), 0, st, a->cent, a->cent_sh, nb, nc, g);
    int rc = ssq_check_hip(hipGetLastError(), "k_grid_header launch");
    if (rc) return rc;
    hipLaunchKernelGGL(k_grid_cells, dim3(kG * kG / kThreads, nb, nh), dim3(kThreads), 0, st, a->cent, a->cent_sh, nb,
                       nc, g);
    return ssq_check_hip(hipGetLastError(), "k_grid_cells launch");
}

// called by ssq_encode (arguments already validated); SSQ_ERR_UNSUPPORTED when the grid path
// cannot serve the call
int ssq_encode_grid_run(const ssq_encode_args* a, hipStream_t st) {
    SSQ_UNSUPPORTED(ssq_encode_grid_supported(a), "the grid encode serves block_dim 2 without a block metric");
    SSQ_REQUIRE(a->grid, "the grid encode needs a grid from ssq_encode_grid_build");
    SSQ_REQUIRE((uintptr_t)a->grid % 16 == 0, "the grid must be 16-byte aligned");
    SSQ_REQUIRE(a->grid_bytes >= grid_total_bytes(*a), "grid too small for this codebook (%llu < %zu bytes)",
                (unsigned long long)a->grid_bytes, grid_total_bytes(*a));
    GridParams gp;
    memset(&gp, 0, sizeof(gp));
    gp.a = *a;
    gp.grid = static_cast<const uint8_t*>(a->grid);
    for (int blk = 0; blk < a->n_blocks; ++blk) {
        const bool heavy = blk < 64 ? ((a->heavy_mask[0] >> blk) & 1) : ((a->heavy_mask[1] >> (blk - 64)) & 1);
        if (!heavy) gp.light[gp.n_light++] = (uint8_t)blk;
    }
    // Launch shape.  Short sequences fold into one key range per KV head; a short launch runs only
    // the waves that have keys, and splits the light blocks into chunks (blockIdx.z) until the
    // workgroups fill the chip.  Chunks also keep a workgroup's codewords within the LDS.
    const int nl = gp.n_light, nb = a->n_blocks;
    gp.fold = ssq_encode_fold(a, 16 * 64);
    const int64_t n_keys = gp.fold ? (int64_t)a->batch * a->seq_len : a->seq_len;
    const int64_t gy = gp.fold ? a->num_kv_heads : (int64_t)a->batch * a->num_kv_heads;
    const int waves = n_keys < 16 * 64 ? (int)((n_keys + 63) / 64) : 16;
    const int keys_wg = waves * 64;
    const int64_t groups = ((n_keys + keys_wg - 1) / keys_wg) * gy;
    int nlc = nl > 0 ? nl : 1;
    if (nl > 1 && groups < ssq_device_cus()) {
        const int64_t want = (ssq_device_cus() + groups - 1) / groups;
        const int64_t chunks0 = want < nl ? want : nl;
        nlc = (int)((nl + chunks0 - 1) / chunks0);
    }
    while (nlc > 1 && grid_smem(nlc, nb, waves) > 160 * 1024) --nlc;
    const size_t smem = grid_smem(nlc, nb, waves);
    SSQ_UNSUPPORTED(smem <= 160 * 1024, "too many blocks for the grid encode's LDS");
    const int chunks = nl > 0 ? (nl + nlc - 1) / nlc : 1;
    gp.nlc = nlc;
    gp.row_codes = chunks == 1 && nb % 16 == 0 && (uintptr_t)a->codes % 16 == 0 && a->c_sb % 16 == 0 &&
                   a->c_sh % 16 == 0 && a->c_st % 16 == 0;
    // key rows of at most 128 bytes at 16-byte aligned addresses are read whole, into registers
    const int esz = a->k_dtype == SSQ_F32 ? 4 : 2;
    const int64_t row_bytes = (int64_t)a->head_dim * esz;
    const bool rowreg = row_bytes % 16 == 0 && row_bytes <= 128 && (uintptr_t)a->keys % 16 == 0 &&
                        (a->k_sb * esz) % 16 == 0 && (a->k_sh * esz) % 16 == 0 && (a->k_ss * esz) % 16 == 0;
    gp.row_q = rowreg ? (int)(row_bytes / 16) : 0;
    const void* fn = rowreg ? reinterpret_cast<const void*>(k_encode_grid<true>)
                            : reinterpret_cast<const void*>(k_encode_grid<false>);
    const int rc = ssq_allow_lds(fn, 160 * 1024, "hipFuncSetAttribute(k_encode_grid)");
    if (rc) return rc;
    dim3 grid((unsigned)((n_keys + keys_wg - 1) / keys_wg), (unsigned)gy, chunks);
    if (rowreg)
        hipLaunchKernelGGL(k_encode_grid<true>, grid, dim3(waves * 64), smem, st, gp);
    else
        hipLaunchKernelGGL(k_encode_grid<false>, grid, dim3(waves * 64), smem, st, gp);
    return ssq_check_hip(hipGetLastError(), "k_encode_grid launch");
}
