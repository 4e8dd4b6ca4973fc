// Grid-search encode for block_dim 2 (no block metric): exact nearest codeword with the
// reference's rounding, evaluating only the codewords a cell grid certifies as possible winners.
//
// Reference semantics (sunshape/codec.py:362-385): code = first argmin_c sqrt(clamp_min(
// [-2x, |x|^2, 1] . [c, 1, |c|^2], 0)), the dot product a k-ascending FMA chain from the first
// product and the norms left-to-right sums of rounded squares (torch.cdist's mm formulation).
//
//  * k_grid_header / k_grid_cells (built once per codebook, ssq_encode_grid_build): per block, a
//    kG x kG grid of cells under a per-dimension map that is finest where the codewords crowd and
//    whose end cells reach to infinity (cell_edge).  Cell C lists, ascending, every codeword j whose
//    Voronoi region, widened by the rounding terms below, meets C: the part of C where
//    |x - c_j|^2 <= |x - c_k|^2 + M_jk for every competitor k (each condition a half-plane) is
//    clipped out of C, and j is listed when it is not empty.  Competitors are the codewords with
//    dmin(C, c_k)^2 <= min_i dmax(C, c_i)^2 + M (a necessary condition for a winner, which also
//    pre-selects the j tried); a j that one competitor's half-plane misses on all four corners of C
//    is dropped before any clipping.  A cell's record is a 32-bit word with the count and the first
//    three indices, and 16 bytes with up to twelve more (read only for longer lists); more than 15
//    codewords, an unbounded cell or a codebook with non-finite values mark it "scan all" (count 0).
//  * k_encode_grid: lane = key.  Per light block: the key's two permuted elements, its cell, the
//    cell's first word (and, for the rare list longer than 3, its second), then the reference chain
//    on each listed candidate in ascending order, keeping the first minimum of the correctly
//    rounded sqrt.  Non-finite keys and "scan all" cells evaluate every codeword.
//
// Why the list holds the winner.  Let r_j be the reference's value for codeword j, D_j the exact
// value of the same expression on the same (rounded) norms, d_j = |x - c_j|.  Then |r_j - D_j| <=
// e_j = g (|x| + |c_j|)^2 (1 + 2.001u) with g = 1.001 K 2^-23, K = bd + 2 (any rounding order),
// and D_j = d_j^2 + alpha + beta_j with |alpha| <= 2.001u|x|^2, |beta_j| <= 2.001u|c_j|^2, u = 2^-24.
// The winner j* has sqrt(max(r_j*, 0)) <= sqrt(max(r_k, 0)) for every k, so max(r_j*, 0) <=
// max(r_k, 0)(1 + 2^-21) (correctly rounded sqrt).  Chaining the bounds, for every k:
//   d_j*^2 <= d_k^2 + 2|alpha| + |beta_j*| + |beta_k| + e_j* + e_k + (d_k^2 + |alpha| + |beta_k| + e_k) 2^-21.
// For x in C (R = max |x| over C, Rc = max |c|) and d_k^2 <= dmax(C, c_k)^2 =: D_k this is at most
//   M_jk = 1.01 (4.002u (R^2 + Rc^2) + 2.0002 g (R + Rc)^2 + (D_k + 2.001u (R^2 + Rc^2) + g (R + Rc)^2) 2^-21),
// so the key x itself lies in j*'s clipped polygon (and no corner test drops j*); with k the
// codeword minimising D_k it gives dmin(C, c_j*)^2 <= min D + M, the pre-selection.  At x every
// condition holds with a slack of 1 % of M_jk and x lies 0.001 of a cell inside the widened cell,
// so the polygon around x is far wider than the fp64 rounding of the clipping.  Cells are widened
// by 0.001 of a cell on each side, far more than the fp32 rounding of the search kernel's cell map,
// so a key always lies in the cell it is looked up in.  The build runs in fp64.
#include "ssq_common.h"

#include <math.h>
#include <string.h>

namespace {

constexpr int kG = 128;        // cells per dimension
constexpr int kMaxCand = 15;   // listed codewords per cell: 3 in the first word, 12 in the rest
constexpr int kHdr = 8;        // floats per block header: mid0, mid1, inv0, inv1, Rc, valid, fingerprint
constexpr int kBuildThreads = 64;  // cells per build workgroup (one wave: per-lane polygons in LDS)
constexpr int kPoly = 16;      // vertex capacity of a clipped cell polygon

// Layout, head-major: per codebook head, its block headers (padded to 256 bytes), the cells' first
// words [nb][kG * kG] (uint32: count, three indices) and then the rest of their lists
// [nb][kG * kG] (16 bytes: twelve indices, padded), so one head's part of a per-KV-head grid is
// itself the grid of that head's codebook, and the words nearly every lookup reads (1 MiB per head
// at 16 blocks) are contiguous; the rest is read only for lists longer than 3.
inline int grid_heads(const ssq_encode_args& a) { return a.cent_sh == 0 ? 1 : a.num_kv_heads; }
__host__ __device__ inline size_t grid_head_hdr_bytes(int nb) { return ((size_t)nb * kHdr * 4 + 255) & ~(size_t)255; }
__host__ __device__ inline size_t grid_head_bytes(int nb) { return grid_head_hdr_bytes(nb) + (size_t)nb * kG * kG * 20; }
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
    // a block whose codewords are all one point (a SunShape-Mixed codec's passthrough blocks hold
    // zeros) gets no grid: every key ties every codeword, and the search scans them all
    bool valid = finite && (lo[0] < hi[0] || lo[1] < hi[1]);
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
        // finite cells reach |x| <= |mid| + 65 sc; beyond 2^40 the reference's fp32 chain could
        // overflow on keys there, which the list bound does not model: no grid
        valid = valid && isfinite(mid[d]) && isfinite(inv[d]) && inv[d] > 0.f && fabs(m) + 65.0 * sc < 0x1.0p40;
    }
    float* out = reinterpret_cast<float*>(grid + (size_t)h * grid_head_bytes(nb)) + (int64_t)blk * kHdr;
    out[0] = mid[0]; out[1] = mid[1]; out[2] = inv[0]; out[3] = inv[1];
    uint32_t fp = cw_count_mix(nc);
    for (int j = 0; j < nc; ++j) fp ^= cw_mix(c[2 * j], c[2 * j + 1], j);
    out[4] = finite ? (float)(sqrt(nrm) * (1.0 + 0x1.0p-20)) : INFINITY;
    valid = valid && out[4] < 0x1.0p40f;  // codewords up to 2^40: no fp32 overflow in the chain
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

// one thread per cell, one wave per workgroup
__global__ __launch_bounds__(kBuildThreads) void k_grid_cells(const float* cent, int64_t cent_sh, int nb, int nc,
                                                              uint8_t* grid) {
    __shared__ double cw[256][2];
    // per-lane clipping polygons, two buffers: vertex v of buffer b of lane l at [b][v][l]
    __shared__ double2 poly[2][kPoly][kBuildThreads];
    const int blk = blockIdx.y, h = blockIdx.z, lane = threadIdx.x;
    const int cell = blockIdx.x * kBuildThreads + lane;
    const float* c = cent + (int64_t)h * cent_sh + (int64_t)blk * nc * 2;
    for (int j = lane; j < nc; j += kBuildThreads) { cw[j][0] = c[2 * j]; cw[j][1] = c[2 * j + 1]; }
    __syncthreads();
    uint8_t* head = grid + (size_t)h * grid_head_bytes(nb);
    const float* hd = reinterpret_cast<const float*>(head) + (int64_t)blk * kHdr;
    uint32_t list[4] = {0u, 0u, 0u, 0u};  // byte i + 1: listed codeword i (byte 0: the count)
    int found = 0;
    bool scan_all = true;
    const int i0 = cell / kG, i1 = cell - (cell / kG) * kG;
    const double w = 2.0 / kG, sc0 = 1.0 / (double)hd[2], sc1 = 1.0 / (double)hd[3];
    const double a0 = cell_edge(-1.0 + w * (i0 - 0.001), hd[0], sc0);
    const double b0 = cell_edge(-1.0 + w * (i0 + 1.001), hd[0], sc0);
    const double a1 = cell_edge(-1.0 + w * (i1 - 0.001), hd[1], sc1);
    const double b1 = cell_edge(-1.0 + w * (i1 + 1.001), hd[1], sc1);
    // end cells (unbounded) and codebooks with non-finite values: scan all
    if (hd[5] != 0.f && isfinite(a0) && isfinite(b0) && isfinite(a1) && isfinite(b1)) {
        scan_all = false;
        const double R2 = fmax(a0 * a0, b0 * b0) + fmax(a1 * a1, b1 * b1);
        const double R = sqrt(R2), Rc = hd[4];
        auto dmax2 = [&](int j) {
            const double dx = fmax(fabs(a0 - cw[j][0]), fabs(b0 - cw[j][0]));
            const double dy = fmax(fabs(a1 - cw[j][1]), fabs(b1 - cw[j][1]));
            return dx * dx + dy * dy;
        };
        auto dmin2 = [&](int j) {
            const double dx = fmax(fmax(a0 - cw[j][0], cw[j][0] - b0), 0.0);
            const double dy = fmax(fmax(a1 - cw[j][1], cw[j][1] - b1), 0.0);
            return dx * dx + dy * dy;
        };
        double dmm = INFINITY;
        int kstar = 0;
        for (int j = 0; j < nc; ++j) {
            const double d = dmax2(j);
            if (d < dmm) { dmm = d; kstar = j; }
        }
        const double u = 0x1.0p-24, g = 1.001 * 4 * 0x1.0p-23;  // K = bd + 2 = 4
        const double S = (R + Rc) * (R + Rc), N2 = R2 + Rc * Rc;
        const double M0 = 1.01 * (4.002 * u * N2 + 2.0002 * g * S + (2.001 * u * N2 + g * S) * 0x1.0p-21);
        const double Mk = 1.01 * 0x1.0p-21;  // M_jk = M0 + Mk D_k
        const double bound = dmm + M0 + Mk * dmm;
        // the pre-selected codewords as a bit set (j is the same for every lane: a uniform
        // register index)
        uint32_t pre[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
        for (int j = 0; j < nc; ++j)
            if (dmin2(j) <= bound) pre[j >> 5] |= 1u << (j & 31);
        auto is_pre = [&](int j) { return (pre[j >> 5] >> (j & 31)) & 1u; };
        // the codewords pre-selected in any cell of the wave: the only j and k worth a trip
        uint32_t any_pre[8];
#pragma unroll
        for (int w8 = 0; w8 < 8; ++w8) {
            uint32_t v = pre[w8];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v |= (uint32_t)__shfl_xor((int)v, o);
            any_pre[w8] = __builtin_amdgcn_readfirstlane(v);
        }
        // calls body(k) for every k of any_pre, ascending (a wave-uniform loop); body returns
        // false to stop early
        auto for_any_pre = [&](auto&& body) {
            for (int w8 = 0; w8 < 8; ++w8)
                for (uint32_t bits = any_pre[w8]; bits; bits &= bits - 1u)
                    if (!body(w8 * 32 + __builtin_ctz(bits))) return;
        };
        // half-plane of j against k: |x - c_j|^2 - |x - c_k|^2 <= M_jk, i.e.
        // 2 (c_k - c_j) . x <= M_jk + |c_k|^2 - |c_j|^2 =: rhs
        auto halfplane = [&](int j, int k, double& nx, double& ny, double& rhs) {
            nx = 2.0 * (cw[k][0] - cw[j][0]);
            ny = 2.0 * (cw[k][1] - cw[j][1]);
            const double nj = cw[j][0] * cw[j][0] + cw[j][1] * cw[j][1];
            const double nk = cw[k][0] * cw[k][0] + cw[k][1] * cw[k][1];
            rhs = M0 + Mk * dmax2(k) + nk - nj;
        };
        // k drops j outright when the half-plane misses all four corners of the cell
        auto drops = [&](int k, int j) {
            double nx, ny, rhs;
            halfplane(j, k, nx, ny, rhs);
            return fmin(nx * a0, nx * b0) + fmin(ny * a1, ny * b1) > rhs;
        };
        // Sutherland-Hodgman: the polygon in buffer src (n vertices) clipped to the half-plane into
        // buffer 1 - src; returns the new count, 0 when nothing is left, -1 when it would exceed
        // kPoly vertices (the caller then keeps j: listing one too many costs time only)
        auto clip = [&](int src, int n, double nx, double ny, double rhs) {
            int m = 0;
            double2 P = poly[src][0][lane];
            double f = nx * P.x + ny * P.y - rhs;
            for (int i = 0; i < n; ++i) {
                const double2 Q = poly[src][i + 1 == n ? 0 : i + 1][lane];
                const double f2 = nx * Q.x + ny * Q.y - rhs;
                if (f <= 0.0) {
                    if (m < kPoly) poly[1 - src][m][lane] = P;
                    ++m;
                }
                if ((f <= 0.0) != (f2 <= 0.0)) {
                    const double t = f / (f - f2);
                    if (m < kPoly) poly[1 - src][m][lane] = make_double2(P.x + t * (Q.x - P.x), P.y + t * (Q.y - P.y));
                    ++m;
                }
                P = Q;
                f = f2;
            }
            return m > kPoly ? -1 : m;
        };
        auto byte_of = [](const uint32_t (&l)[4], int i) { return (int)((l[i >> 2] >> (8 * (i & 3))) & 255u); };
        // the polygon of j: the cell, clipped by competitor k's half-plane (n vertices in buffer src)
        auto start = [&](int& n, int& src) {
            poly[0][0][lane] = make_double2(a0, a1);
            poly[0][1][lane] = make_double2(b0, a1);
            poly[0][2][lane] = make_double2(b0, b1);
            poly[0][3][lane] = make_double2(a0, b1);
            n = 4;
            src = 0;
        };
        auto cut = [&](int& n, int& src, int j, int k) {
            double nx, ny, rhs;
            halfplane(j, k, nx, ny, rhs);
            n = clip(src, n, nx, ny, rhs);
            src ^= 1;
        };
        // 1. corner tests, the codeword nearest the whole cell first: they drop most candidates.
        // The survivors (up to 16 kept in cand, bytes 0-15) hold every codeword that can win in the
        // cell, so only their half-planes shape the winners' regions inside it.
        uint32_t cand[4] = {0u, 0u, 0u, 0u};
        int n_surv = 0;
        constexpr int kMaxSurv = 64;  // more survivors (a degenerate codebook): the cell scans all
        for_any_pre([&](int j) {
            bool alive = n_surv <= kMaxSurv && is_pre(j) && !(j != kstar && drops(kstar, j));
            if (__builtin_amdgcn_ballot_w64(alive))
                for_any_pre([&](int k) {
                    if (alive && k != j && k != kstar && is_pre(k) && drops(k, j)) alive = false;
                    return __builtin_amdgcn_ballot_w64(alive) != 0;
                });
            if (alive) {
                if (n_surv < 16) cand[n_surv >> 2] |= (uint32_t)j << (8 * (n_surv & 3));
                ++n_surv;
            }
            return __builtin_amdgcn_ballot_w64(n_surv <= kMaxSurv) != 0;
        });
        auto keep = [&](int j) {
            if (found < kMaxCand) list[(found + 1) >> 2] |= (uint32_t)j << (8 * ((found + 1) & 3));
            ++found;
        };
        // 2. each survivor's polygon clipped by the other survivors' half-planes (kstar first)
        for (int si = 0; si < 16 && __builtin_amdgcn_ballot_w64(si < n_surv && n_surv <= 16); ++si) {
            const bool act = si < n_surv && n_surv <= 16;
            const int j = byte_of(cand, si);
            int n = 0, src = 0;
            if (act) start(n, src);
            if (act && n_surv > 1 && j != kstar) cut(n, src, j, kstar);
            for (int ti = 0; ti < 16 && __builtin_amdgcn_ballot_w64(n > 0 && n_surv > 1 && ti < n_surv); ++ti) {
                const int k = byte_of(cand, ti);
                if (n > 0 && n_surv > 1 && ti < n_surv && k != j && k != kstar) cut(n, src, j, k);
            }
            if (act && n != 0) keep(j);  // left over, or out of vertex room (n < 0): listed
        }
        // 17 to 64 survivors (rare): every pre-selected codeword against every pre-selected one,
        // until the list overflows
        const bool wide = n_surv > 16 && n_surv <= kMaxSurv;
        if (__builtin_amdgcn_ballot_w64(wide)) {
            for_any_pre([&](int j) {
                const bool act = wide && is_pre(j) && found <= kMaxCand;
                int n = 0, src = 0;
                if (act) start(n, src);
                if (act && j != kstar) cut(n, src, j, kstar);
                if (__builtin_amdgcn_ballot_w64(n > 0))
                    for_any_pre([&](int k) {
                        if (n > 0 && k != j && k != kstar && is_pre(k)) cut(n, src, j, k);
                        return __builtin_amdgcn_ballot_w64(n > 0) != 0;
                    });
                if (act && n != 0) keep(j);
                return __builtin_amdgcn_ballot_w64(wide && found <= kMaxCand) != 0;
            });
        }
        if (found == 0 || found > kMaxCand || n_surv > kMaxSurv) scan_all = true;  // every codeword
    }
    // count and indices, bytes past the list repeating its last index (evaluating a codeword again
    // cannot change the search's result); scan-all cells hold zeros
    uint32_t wd[4] = {0u, 0u, 0u, 0u};
    if (!scan_all) {
        wd[0] = list[0] | (uint32_t)found;
        wd[1] = list[1]; wd[2] = list[2]; wd[3] = list[3];
        const uint32_t last = (wd[found >> 2] >> (8 * (found & 3))) & 255u;
        for (int b = found + 1; b < 16; ++b) wd[b >> 2] |= last << (8 * (b & 3));
    }
    uint32_t* first = reinterpret_cast<uint32_t*>(head + grid_head_hdr_bytes(nb));
    first[(int64_t)blk * kG * kG + cell] = wd[0];
    uint4* rest = reinterpret_cast<uint4*>(head + grid_head_hdr_bytes(nb) + (size_t)nb * kG * kG * 4);
    rest[(int64_t)blk * kG * kG + cell] = make_uint4(wd[1], wd[2], wd[3], 0u);
}

// ---------------------------------------------------------------------------
// search
// ---------------------------------------------------------------------------
constexpr int kMaxLight = 128;

struct GridParams {
    ssq_encode_args a;
    const uint8_t* grid;       // head-major: headers, first words, second words per codebook head
    int n_light;
    int row_codes;             // whole code rows in 16-byte stores
    int row_q;                 // 16-byte pieces of a key row when rows are read whole (else 0)
    int fold;                  // short sequences: all sequences of a KV head share one key range
    int nlc;                   // light blocks per workgroup chunk (blockIdx.z picks the chunk)
    int xcd_order;             // workgroup ids regrouped so each XCD takes a contiguous range
    uint8_t light[kMaxLight];  // light block ids, ascending
};

// A lane's staged code row: nb bytes padded to an odd number of 32-bit words, so the 64 lanes'
// one-byte writes of a block land in 64 different LDS banks
__host__ __device__ inline int code_row_bytes(int nb) {
    const int w = (nb + 3) >> 2;
    return 4 * (w | 1);
}
// LDS layout (bytes): cb [nl][256] float2 | cn [nl][256] float | hd [nl] float4 | poff [nl][4] int |
// hinfo [nb] int4 | codes [waves][64][code_row_bytes(nb)]
inline size_t grid_smem(int nl, int nb, int waves) {
    return (size_t)nl * 256 * 12 + (size_t)nl * 16 + (size_t)nl * 16 + (size_t)nb * 16 +
           (size_t)waves * 64 * code_row_bytes(nb);
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

template <bool ROWREG, int KDT>
__global__ __launch_bounds__(1024) void k_encode_grid(const GridParams p) {
    extern __shared__ __align__(16) float smem[];
    const ssq_encode_args& a = p.a;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int waves = blockDim.x >> 6;
    // Workgroup order.  The hardware deals consecutive workgroup ids to the 8 XCDs in turn; with
    // xcd_order each XCD's ids are regrouped into one contiguous range of (KV head, sequence, key
    // range) in KV-head-major order, so an XCD's L2 holds the cell words of one codebook head
    // (per-KV-head codebooks) instead of all of them.
    const uint32_t gx = gridDim.x, n_wg = gx * gridDim.y;
    uint32_t id = blockIdx.x + gx * blockIdx.y;
    if (p.xcd_order) id = (id & 7u) * (n_wg >> 3) + (id >> 3);
    const int gxi = (int)(id % gx), gyi = (int)(id / gx);
    const int nbat = p.fold ? 1 : a.batch;
    const SsqKeyMap km(a, p.fold, gyi / nbat, gyi % nbat);
    const int kv = km.kv;
    const int l0 = blockIdx.z * p.nlc;  // this chunk's first light block
    const int nl = min(p.nlc, p.n_light - l0), nb = a.n_blocks, nc = a.n_centroids;
    const int hsel = a.cent_sh == 0 ? 0 : kv;

    float2* cb = reinterpret_cast<float2*>(smem);                          // [nl][256]
    float* cn = reinterpret_cast<float*>(cb + nl * 256);                   // [nl][256]
    float4* hd = reinterpret_cast<float4*>(cn + nl * 256);                 // [nl]: mid0, mid1, inv0, inv1
    int* poff = reinterpret_cast<int*>(hd + nl);                           // [nl]: perm0, perm1, block id, 0
    // [heavy blocks]: the block's two dims in the key row, its id, its passthrough slot (chunk 0)
    int4* hinfo = reinterpret_cast<int4*>(poff + 4 * nl);
    const int crb = code_row_bytes(nb);
    uint8_t* cs = reinterpret_cast<uint8_t*>(hinfo + nb) + wave * 64 * crb;  // this wave's code rows

    const int keys_wg = waves * 64;
    const int key = gxi * keys_wg + wave * 64 + lane;  // this lane's key index
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

    constexpr int kdt = KDT;
    // ---- the key's permuted elements, issued before the staging below (they do not depend on
    // it; issued after its barrier they would add a memory round trip to the chain).  ROWREG: the
    // whole row (at most 128 bytes, 16-byte aligned) is loaded once with 16-byte loads into
    // registers, and each block's two elements are picked out by a wave-uniform register index
    // (non-temporal loads were measured 20 % slower here).  Otherwise each element is a load of
    // its own, issued one block ahead of its use.
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
            // no grid (or one built for another codebook): a NaN centre sends every key to cell
            // (0, 0), an end cell, which scans all codewords
            const bool ok = hB.y != 0.f && (f ^ cw_count_mix(nc)) == __float_as_uint(hB.z);
            hd[li] = ok ? hA : make_float4(__builtin_nanf(""), __builtin_nanf(""), 0.f, 0.f);
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
    for (int i = lane; i < 16 * crb; i += 64) reinterpret_cast<uint32_t*>(cs)[i] = 0u;  // heavy blocks: code 0
    __syncthreads();

    const uint64_t hm0 = a.heavy_mask[0], hm1 = a.heavy_mask[1];
    // the cells' first words of this head's table, and the rest of their lists
    const uint32_t* words = reinterpret_cast<const uint32_t*>(p.grid + (size_t)hsel * grid_head_bytes(nb) +
                                                              grid_head_hdr_bytes(nb));
    const uint4* rest = reinterpret_cast<const uint4*>(words + (size_t)nb * kG * kG);
    // element e (wave-uniform) of the register row, as raw bits
    auto row_bits = [&](int e) -> uint32_t {
        if constexpr (KDT == SSQ_F32) {
            return row[e & 31];
        } else {
            const uint32_t w = row[(e >> 1) & 31];
            return (e & 1) ? (w >> 16) : (w & 0xffffu);
        }
    };
    // the word index of (x0, x1)'s cell in block blk of this head's table under the block's map h
    // (mid0, mid1, inv0, inv1).  t within rounding of +-1 may land one past the ends: the end cells
    // take it.  |u| of 2^100 or more (whose reciprocal would leave the normal range) is +-1
    // outright; a non-finite key element, or a block without a grid (NaN centre), gives NaN, and
    // t = -1.  Either way the key lands in an end cell, whose record says "scan all".
    auto map_t = [](float u) {
        return fabsf(u) < 0x1.0p100f ? u * __builtin_amdgcn_rcpf(1.0f + fabsf(u)) : (u > 0.f ? 1.f : -1.f);
    };
    auto cell_of = [&](const float4& h, int blk, float x0, float x1) -> uint32_t {
        const float u0 = (x0 - h.x) * h.z, u1 = (x1 - h.y) * h.w;
        const float t0 = map_t(u0), t1 = map_t(u1);
        const float f0 = floorf((t0 + 1.0f) * (0.5f * kG)), f1 = floorf((t1 + 1.0f) * (0.5f * kG));
        const int c0 = (int)fminf(fmaxf(f0, 0.f), (float)(kG - 1));  // fmaxf(NaN, 0) = 0
        const int c1 = (int)fminf(fmaxf(f1, 0.f), (float)(kG - 1));
        return (uint32_t)(blk * kG * kG + c0 * kG + c1);
    };
    // a key row's element (element path), as raw bits
    auto key_bits = [&](int e) { return ssq_load_bits(a.keys, KDT, krow + e); };
    // the rest of a cell's list, loaded by every lane: lanes whose list ends in the first word read
    // one 16-byte dummy that every such lane shares (an exact count of loads in flight lets each
    // wait name the load it needs); the evaluation picks the padding for them
    auto rest_raw = [&](uint32_t w0, uint32_t cell) -> uint4 { return rest[(w0 & 255u) > 3u ? cell : 0u]; };

    // Software pipeline over the light blocks.  Trip li evaluates block li while blocks li + 1 ..
    // li + 3 are in flight:
    //   1. block li + 3: its elements, cell, and the cell's first word (a load);
    //   2. element path: the raw key elements of block li + 4 (loads);
    //   3. block li + 2: its first word (loaded a trip ago) gives its count, and the rest of its
    //      list is loaded: two trips before its use, since it is rarely in the L2;
    //   4. block li is evaluated;
    //   5. the LDS entries (element positions, block id, cell map) that the next trip's steps 1
    //      and 2 use are read ahead.
    // Loads are issued unconditionally, so each wait names the load it needs.  Indices past the
    // last block are clamped to it.  Stage S holds block li + S.
    const int4* pinfo = reinterpret_cast<const int4*>(poff);
    auto clampb = [&](int l) { return min(l, nl - 1); };
    float x0a = 0.f, x0b = 0.f, x1a = 0.f, x1b = 0.f, x2a = 0.f, x2b = 0.f;
    uint32_t w0s = 0u, w1s = 0u, w2s = 0u, cell1 = 0u, cell2 = 0u;
    uint4 r0s = make_uint4(0u, 0u, 0u, 0u), r1s = r0s;  // raw rests of stages 0 and 1
    int blk0 = 0, blk1 = 0, blk2 = 0;
    int4 pi3 = make_int4(0, 0, 0, 0), pi4 = pi3;  // LDS entries of blocks li + 3 (and li + 4: element path)
    float4 hi3 = make_float4(0.f, 0.f, 0.f, 0.f);
    uint32_t ua3 = 0u, ub3 = 0u;                  // element path: raw elements of block li + 3
    if (nl > 0) {
        float xa[3], xb[3];
        uint32_t wv[3], cv[3];
        int bv[3];
#pragma unroll
        for (int s3 = 0; s3 < 3; ++s3) {
            const int l = clampb(s3);
            const int4 v = pinfo[l];
            const int e0 = __builtin_amdgcn_readfirstlane(v.x), e1 = __builtin_amdgcn_readfirstlane(v.y);
            bv[s3] = __builtin_amdgcn_readfirstlane(v.z);
            if constexpr (ROWREG) {
                xa[s3] = ssq_bits_to_f32(row_bits(e0), KDT);
                xb[s3] = ssq_bits_to_f32(row_bits(e1), KDT);
            } else {
                xa[s3] = ssq_bits_to_f32(key_bits(e0), KDT);
                xb[s3] = ssq_bits_to_f32(key_bits(e1), KDT);
            }
            cv[s3] = cell_of(hd[l], bv[s3], xa[s3], xb[s3]);
            wv[s3] = words[cv[s3]];
        }
        x0a = xa[0]; x0b = xb[0]; w0s = wv[0]; blk0 = bv[0];
        x1a = xa[1]; x1b = xb[1]; w1s = wv[1]; blk1 = bv[1]; cell1 = cv[1];
        x2a = xa[2]; x2b = xb[2]; w2s = wv[2]; blk2 = bv[2]; cell2 = cv[2];
        r0s = rest_raw(w0s, cv[0]);
        r1s = rest_raw(w1s, cell1);
        pi3 = pinfo[clampb(3)];
        hi3 = hd[clampb(3)];
        if constexpr (!ROWREG) {
            ua3 = key_bits(__builtin_amdgcn_readfirstlane(pi3.x));
            ub3 = key_bits(__builtin_amdgcn_readfirstlane(pi3.y));
            pi4 = pinfo[clampb(4)];
        }
    }
    for (int li = 0; li < nl; ++li) {
        // ---- 1. block li + 3: elements, cell, first word
        const int blk3 = __builtin_amdgcn_readfirstlane(pi3.z);
        float x3a, x3b;
        if constexpr (ROWREG) {
            x3a = ssq_bits_to_f32(row_bits(__builtin_amdgcn_readfirstlane(pi3.x)), KDT);
            x3b = ssq_bits_to_f32(row_bits(__builtin_amdgcn_readfirstlane(pi3.y)), KDT);
        } else {
            x3a = ssq_bits_to_f32(ua3, KDT);
            x3b = ssq_bits_to_f32(ub3, KDT);
        }
        const uint32_t cell3 = cell_of(hi3, blk3, x3a, x3b);
        const uint32_t w3s = words[cell3];
        // ---- 2. element path: block li + 4's raw elements
        if constexpr (!ROWREG) {
            ua3 = key_bits(__builtin_amdgcn_readfirstlane(pi4.x));
            ub3 = key_bits(__builtin_amdgcn_readfirstlane(pi4.y));
        }
        // ---- 3. block li + 2: the rest of its list
        const uint4 r2s = rest_raw(w2s, cell2);

        // ---- 4. block li: candidates 0-2 in bytes 1-3 of the first word, 3-14 in the rest
        const float m0 = -2.0f * x0a, m1 = -2.0f * x0b;
        const float xn = x0a * x0a + x0b * x0b;
        const float2* cbl = cb + li * 256;
        const float* cnl = cn + li * 256;
        const int cnt = (int)(w0s & 255u);  // 0: every codeword
        const uint32_t pad = (w0s >> 24) * 0x01010101u;
        const uint32_t rw[3] = {cnt > 3 ? r0s.x : pad, cnt > 3 ? r0s.y : pad, cnt > 3 ? r0s.z : pad};
        auto cand = [&](int i) {  // i is a compile-time constant in the unrolled loop below
            return (int)(i < 3 ? (w0s >> (8 * (i + 1))) & 255u : (rw[(i - 3) >> 2] >> (8 * ((i - 3) & 3))) & 255u);
        };
        // The first candidate starts the running minimum; each trip reads the next candidate's
        // codeword while it evaluates its own.  Bytes past a lane's count repeat its last
        // candidate and cannot win.  Lanes that scan all codewords start over below.
        float2 cc = cbl[cand(0)];
        float cq = cnl[cand(0)];
        float2 nc2 = cbl[cand(1)];
        float nq = cnl[cand(1)];
        Cand st{chain_val(cc, cq, m0, m1, xn), cand(0)};
#pragma unroll
        for (int i = 1; i < kMaxCand; ++i) {
            if (!__builtin_amdgcn_ballot_w64(i < cnt)) break;  // the wave's lists are done
            cc = nc2;
            cq = nq;
            if (i + 1 < kMaxCand) {
                nc2 = cbl[cand(i + 1)];
                nq = cnl[cand(i + 1)];
            }
            next_val(cc, cq, cand(i), m0, m1, xn, st);
        }
        const bool full = cnt == 0;
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
        cs[lane * crb + blk0] = (uint8_t)(st.bj < 0 ? 0 : st.bj);

        // ---- 5. the next trip's LDS entries
        if constexpr (ROWREG) {
            pi3 = pinfo[clampb(li + 4)];
        } else {
            pi3 = pi4;
            pi4 = pinfo[clampb(li + 5)];
        }
        hi3 = hd[clampb(li + 4)];

        // ---- rotate the stages
        x0a = x1a; x0b = x1b; w0s = w1s; r0s = r1s; blk0 = blk1;
        x1a = x2a; x1b = x2b; w1s = w2s; r1s = r2s; blk1 = blk2; cell1 = cell2;
        x2a = x3a; x2b = x3b; w2s = w3s; blk2 = blk3; cell2 = cell3;
    }

    // ---- outputs: code rows, heavy blocks' passthrough values
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int s_wave = gxi * keys_wg + wave * 64;
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
                const uint32_t* src = reinterpret_cast<const uint32_t*>(cs + m * crb + 16 * q);
                *reinterpret_cast<uint4*>(a.codes + crow + 16 * q) = make_uint4(src[0], src[1], src[2], src[3]);
            }
        }
    } else if (live && gridDim.z == 1) {  // every block's code (heavy blocks' 0 included)
        const int64_t crow = crow_k;
        for (int blk = 0; blk < nb; ++blk) a.codes[crow + blk] = cs[lane * crb + blk];
    } else if (live) {  // one chunk of several: its blocks' codes; chunk 0 also the heavy blocks' 0
        const int64_t crow = crow_k;
        for (int li = 0; li < nl; ++li) {
            const int blk = __builtin_amdgcn_readfirstlane(poff[4 * li + 2]);
            a.codes[crow + blk] = cs[lane * crb + blk];
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
    hipLaunchKernelGGL(k_grid_cells, dim3(kG * kG / kBuildThreads, nb, nh), dim3(kBuildThreads), 0, st, a->cent,
                       a->cent_sh, nb,
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
    // one instantiation per (row path, key dtype)
    using Kern = void (*)(const GridParams);
    const int dsel = a->k_dtype == SSQ_F32 ? 0 : a->k_dtype == SSQ_BF16 ? 1 : 2;
    static const Kern kerns[2][3] = {
        {k_encode_grid<false, SSQ_F32>, k_encode_grid<false, SSQ_BF16>, k_encode_grid<false, SSQ_F16>},
        {k_encode_grid<true, SSQ_F32>, k_encode_grid<true, SSQ_BF16>, k_encode_grid<true, SSQ_F16>}};
    const Kern fn = kerns[rowreg ? 1 : 0][dsel];
    const int rc = ssq_allow_lds(reinterpret_cast<const void*>(fn), 160 * 1024, "hipFuncSetAttribute(k_encode_grid)");
    if (rc) return rc;
    dim3 grid((unsigned)((n_keys + keys_wg - 1) / keys_wg), (unsigned)gy, chunks);
    gp.xcd_order = ((uint64_t)grid.x * grid.y) % 8 == 0;
    hipLaunchKernelGGL(fn, grid, dim3(waves * 64), smem, st, gp);
    return ssq_check_hip(hipGetLastError(), "k_encode_grid launch");
}
