// matmul.hip — weight x activation products on gfx950: y[c*rows + r] = W[r] . x[c] for c < ncols.
//
// K-quant weights (Q4_K, Q5_K, Q6_K) go to the matrix-core kernel (kq_mfma.h); this file holds the Q8_0 / Q4_0
// and F32 products, the weight repacking into planes, and the dispatch by weight type.
#include "aq_common.h"

#include <map>
#include <mutex>
#include <tuple>

namespace aq {
namespace {

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    _Float16 f;
    __builtin_memcpy(&f, &h, 2);
    return (float)f;
}

// --------------------------------------------------------------------------------- Q8_0 / Q4_0 / F32 rows
// dot.rs:29-66 (Q8_0, Q4_0 x Q8_0) and dot.rs:180-200 (F32 x f32): per 32-block an exact i32 sum (or a
// left-to-right f32 partial for F32), then ONE f32 accumulator over the blocks left to right. The block
// products are independent, so a work-group computes them in parallel into LDS, then one lane per
// (row, column) adds them in block order: the reference's chain, bit for bit.
// One matrix of a grouped wave-kernel launch (matrices sharing the activations, the type and K): its planes, its
// output, its rows, and the first work-group of the launch that computes it.
struct Q8Seg {
    const uint8_t *qa, *dm;
    float *y;
    int rows, wg0;
};

struct Q8Args {
    int type;
    const uint8_t *qa, *dm; // codes plane, f16 scales (F32: qa = rows)
    int rows, nb32;
    const int8_t *xq; // ncols x n
    const float *xd;  // ncols x nb32
    const int32_t *xs; // ncols x nb32
    const float *xf;  // ncols x n (F32 weights)
    size_t n;
    float *y;
    const float *resid;
    int ncols; // columns of the launch (the F32 kernel: groups of NC along grid y)
};

// The matrices of a grouped wave-kernel launch (its own kernel argument, so single launches keep Q8Args alone).
struct Q8Group {
    Q8Seg seg[Q8_MAXSEG];
    int nseg;
};

template <int NC, int RPB>
__global__ void __launch_bounds__(256) q8_matmul_kernel(Q8Args a) {
    extern __shared__ float prods[]; // RPB x nb32 x NC
    constexpr int TPR = 256 / RPB;   // threads per row
    const int r_loc = threadIdx.x / TPR, j = threadIdx.x % TPR;
    const int row = (int)blockIdx.x * RPB + r_loc;
    const int nb = a.nb32;
    if (row < a.rows) {
        for (int b = j; b < nb; b += TPR) {
            const size_t wb = (size_t)row * nb + b;
            if (a.type == AQ_TYPE_F32) { // the last block may be the reference's short tail
                const float *w = reinterpret_cast<const float *>(a.qa) + (size_t)row * a.n + (size_t)b * 32;
                const int ne = a.n - (size_t)b * 32 < 32 ? (int)(a.n - (size_t)b * 32) : 32;
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const float *x = a.xf + (size_t)c * a.n + (size_t)b * 32;
                    float part = 0.0f;
                    for (int e = 0; e < ne; e++) part += w[e] * x[e];
                    prods[(r_loc * nb + b) * NC + c] = part;
                }
                continue;
            }
            const float dw = half_bits_to_float(*reinterpret_cast<const uint16_t *>(a.dm + wb * 2));
            uint32_t wq[8];
            if (a.type == AQ_TYPE_Q8_0) {
                const uint4 w0 = *reinterpret_cast<const uint4 *>(a.qa + wb * 32);
                const uint4 w1 = *reinterpret_cast<const uint4 *>(a.qa + wb * 32 + 16);
                wq[0] = w0.x; wq[1] = w0.y; wq[2] = w0.z; wq[3] = w0.w;
                wq[4] = w1.x; wq[5] = w1.y; wq[6] = w1.z; wq[7] = w1.w;
            } else { // Q4_0: low nibbles are elements 0..15, high nibbles 16..31, each q - 8
                const uint4 w0 = *reinterpret_cast<const uint4 *>(a.qa + wb * 16);
                const uint32_t ws[4] = {w0.x, w0.y, w0.z, w0.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    wq[i] = ws[i] & 0x0F0F0F0Fu;
                    wq[i + 4] = (ws[i] >> 4) & 0x0F0F0F0Fu;
                }
            }
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int8_t *xp = a.xq + (size_t)c * a.n + (size_t)b * 32;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xp);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xp + 16);
                const uint32_t xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                int isum = 0;
#pragma unroll
                for (int i = 0; i < 8; i++) isum = dot4(wq[i], xs[i], isum);
                const size_t xm = (size_t)c * nb + b;
                if (a.type == AQ_TYPE_Q4_0) isum -= 8 * a.xs[xm];
                prods[(r_loc * nb + b) * NC + c] = (dw * a.xd[xm]) * (float)isum;
            }
        }
    }
    __syncthreads();
    // the chain: one lane per (row, column), blocks in order
    if (threadIdx.x < RPB * NC) {
        const int rr = threadIdx.x / NC, c = threadIdx.x % NC;
        const int orow = (int)blockIdx.x * RPB + rr;
        if (orow < a.rows) {
            float acc = 0.0f;
            const float *pc = prods + (size_t)rr * nb * NC + c;
            int b = 0;
            for (; b + 16 <= nb; b += 16) { // 16 reads in flight, the sum still in block order
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = pc[(b + u) * NC];
#pragma unroll
                for (int u = 0; u < 16; u++) acc += v[u];
            }
            for (; b < nb; b++) acc += pc[b * NC];
            // dot.rs:180-200 (F32): full blocks, then `acc + part` with the tail's partial (0.0f when there is none)
            if (a.type == AQ_TYPE_F32 && a.n % 32 == 0) acc = acc + 0.0f;
            const size_t o = (size_t)c * a.rows + orow;
            a.y[o] = a.resid ? a.resid[o] + acc : acc;
        }
    }
}

// ------------------------------------------------------------------------------------ Q8_0 / Q4_0 by waves
// dot.rs:29-66 per 32-block: isum = the exact integer dot of the codes (Q4_0: codes q - 8, taken as
// sum(q*x) - 8*sum(x)), then acc += (dw * dx) * float(isum) block after block: one chain per (row, column).
// A wave owns RPW rows; lane (r, ks) = KS*r + ks (KS = 64 / RPW) computes, in round rd, block KS*rd + ks of row r
// for every column. The KS products of a (row, column) go through the wave's LDS slot to its chain owner, lane
// RPW*c + r, which adds them in block order (no work-group barrier: one wave's LDS accesses execute in order).
// Weights stream through a register ring Q8W_PF rounds deep; the activations (codes, f32 scales, Q4_0 code sums)
// are staged in LDS once per work-group (4 to 16 waves: the most that still let the whole grid be resident at once),
// so the staging (~31 KB at K = 6144, 4 columns) is shared by up to 16 * RPW rows. Few rows per wave keep short
// matrices (5120 rows) at several waves per SIMD.
constexpr int Q8W_PF = 4;
// the block record of the staged codes: NC columns of 32 bytes plus 16, so the 16 blocks that one LDS access of
// 16 lanes reads start in 16 different 4-bank groups
constexpr int q8w_xs(int nc) { return nc * 32 + 16; }

template <int TYPE>
struct Q8Regs {
    uint4 c0, c1; // Q8_0: 32 codes; Q4_0: c0 = 16 bytes of nibbles
    uint32_t d;   // f16 scale bits
};

template <int TYPE, int NC, int RPW>
__device__ __forceinline__ void q8_wave_body(const Q8Args &a, int wg, const uint8_t *wqa, const uint8_t *wdm, float *wy,
                                             const float *wres, const int rows) {
    extern __shared__ __align__(16) uint8_t q8_lds[];
    constexpr bool Q4 = TYPE == AQ_TYPE_Q4_0;
    constexpr int KS = 64 / RPW;
    const int nb = a.nb32;
    constexpr int XS = q8w_xs(NC);                                    // bytes per block record (NC columns)
    int8_t *sx = reinterpret_cast<int8_t *>(q8_lds);                   // [nb][XS]: column c at c * 32
    float *sxd = reinterpret_cast<float *>(q8_lds + (size_t)nb * XS);  // [NC][nb]
    int32_t *sxs = reinterpret_cast<int32_t *>(sxd + (size_t)nb * NC); // [NC][nb]
    float *xch = reinterpret_cast<float *>(sxs + (size_t)nb * NC);     // [waves][NC][RPW rows][KS + 1]
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int r = lane / KS, ks = lane % KS;
    const int nwv = (int)(blockDim.x >> 6); // waves per work-group
    const int row0 = (wg * nwv + wid) * RPW;
    int row = row0 + r;
    if (row >= rows) row = rows - 1;
    const size_t rowb = (size_t)row * nb;
    auto load = [&](Q8Regs<TYPE> &w, int blk) {
        const size_t wb = rowb + (blk < nb ? blk : nb - 1);
        if constexpr (Q4) {
            w.c0 = ld_nt4(wqa + wb * 16);
        } else {
            w.c0 = ld_nt4(wqa + wb * 32);
            w.c1 = ld_nt4(wqa + wb * 32 + 16);
        }
        w.d = ld_nth(wdm + wb * 2);
    };
    Q8Regs<TYPE> wr[Q8W_PF];
    const int NT = (int)blockDim.x;
    const int nh = nb * NC * 2; // 16-byte halves of the activation code blocks
    auto half_src = [&](int e) {
        const int rec = e >> 1, c = rec / nb, blk = rec - c * nb;
        return reinterpret_cast<const uint4 *>(a.xq + (size_t)c * a.n + (size_t)blk * 32 + (e & 1) * 16);
    };
    auto half_dst = [&](int e) {
        const int rec = e >> 1, c = rec / nb, blk = rec - c * nb;
        return reinterpret_cast<uint4 *>(sx + (size_t)blk * XS + c * 32 + (e & 1) * 16);
    };
    const int ns = nb * NC; // block scales (and Q4_0 code sums) of the activations
    if (nh <= 3 * NT && ns <= 2 * NT) { // uniform: the activations fit a few registers per thread
        // loaded ahead of the first weights (every load issued, clamped), written after them: the LDS writes wait
        // only for the activations
        const int e0 = min((int)threadIdx.x, nh - 1), e1 = min((int)threadIdx.x + NT, nh - 1),
                  e2 = min((int)threadIdx.x + 2 * NT, nh - 1);
        const int s0 = min((int)threadIdx.x, ns - 1), s1 = min((int)threadIdx.x + NT, ns - 1);
        const uint4 h0 = *half_src(e0), h1 = *half_src(e1), h2 = *half_src(e2);
        const float xd0 = a.xd[s0], xd1 = a.xd[s1];
        const int32_t xs0 = Q4 ? a.xs[s0] : 0, xs1 = Q4 ? a.xs[s1] : 0;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < Q8W_PF; p++) load(wr[p], p * KS + ks);
        __builtin_amdgcn_sched_barrier(0);
        *half_dst(e0) = h0; // past the end: the last entry again, with its own bytes
        *half_dst(e1) = h1;
        *half_dst(e2) = h2;
        sxd[s0] = xd0; // same [column][block] order as the activations
        sxd[s1] = xd1;
        if constexpr (Q4) {
            sxs[s0] = xs0;
            sxs[s1] = xs1;
        }
    } else {
#pragma unroll
        for (int p = 0; p < Q8W_PF; p++) load(wr[p], p * KS + ks);
        for (int e = (int)threadIdx.x; e < nh; e += NT) *half_dst(e) = *half_src(e);
        for (int e = (int)threadIdx.x; e < nb * NC; e += NT) {
            sxd[e] = a.xd[e];
            if constexpr (Q4) sxs[e] = a.xs[e];
        }
    }
    __syncthreads();
    if (row0 >= rows) return; // no barrier follows
    // one float of padding per (column, row) record: the chain owners' reads fall in different banks
    constexpr int KP = KS + 1;
    float *xw = xch + (size_t)wid * NC * RPW * KP;
    const int oc = lane / RPW, orr = lane % RPW; // as a chain owner (lane < RPW * NC): column oc, row orr
    float acc = 0.0f;
    const int nr = (nb + KS - 1) / KS;

    auto round_body = [&](Q8Regs<TYPE> &w, const int rd, const bool prefetch) {
        const int blk = rd * KS + ks, blkc = blk < nb ? blk : nb - 1;
        uint32_t wq[8];
        if constexpr (Q4) {
            const uint32_t c4[4] = {w.c0.x, w.c0.y, w.c0.z, w.c0.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                wq[i] = c4[i] & 0x0F0F0F0Fu;            // elements 4i .. 4i+3
                wq[i + 4] = (c4[i] >> 4) & 0x0F0F0F0Fu; // elements 16 + 4i ..
            }
        } else {
            wq[0] = w.c0.x, wq[1] = w.c0.y, wq[2] = w.c0.z, wq[3] = w.c0.w;
            wq[4] = w.c1.x, wq[5] = w.c1.y, wq[6] = w.c1.z, wq[7] = w.c1.w;
        }
        const float dw = half_bits_to_float((uint16_t)w.d);
        float pr[NC];
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const uint4 *xp = reinterpret_cast<const uint4 *>(sx + (size_t)blkc * XS + c * 32);
            const uint4 x0 = xp[0], x1 = xp[1];
            const uint32_t xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            int isum = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) isum = dot4(wq[i], xs[i], isum);
            if constexpr (Q4) isum -= 8 * sxs[c * nb + blkc];
            pr[c] = (dw * sxd[c * nb + blkc]) * (float)isum;
        }
        if (prefetch) {
            __builtin_amdgcn_sched_barrier(0);
            load(w, blk + Q8W_PF * KS);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int c = 0; c < NC; c++) xw[(c * RPW + r) * KP + ks] = pr[c];
        __asm__ volatile("" ::: "memory");
        if (lane < RPW * NC) {
            const int live = nb - rd * KS < KS ? nb - rd * KS : KS;
            const float *pv = xw + (oc * RPW + orr) * KP;
#pragma unroll
            for (int u0 = 0; u0 < KS; u0 += 16) { // 16 reads in flight, the sum in block order
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = pv[u0 + u];
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if (u0 + u < live) acc += v[u];
            }
        }
        __asm__ volatile("" ::: "memory");
    };
    const int nfull = nr / Q8W_PF * Q8W_PF;
    for (int rd = 0; rd < nfull; rd += Q8W_PF) {
#pragma unroll
        for (int p = 0; p < Q8W_PF; p++) round_body(wr[p], rd + p, true);
    }
#pragma unroll
    for (int p = 0; p < Q8W_PF; p++)
        if (nfull + p < nr) round_body(wr[p], nfull + p, false);
    if (lane < RPW * NC && row0 + orr < rows) {
        const size_t o = (size_t)oc * rows + row0 + orr;
        wy[o] = wres ? wres[o] + acc : acc;
    }
}

template <int TYPE, int NC, int RPW>
__global__ void __launch_bounds__(1024) q8_wave_kernel(Q8Args a) {
    q8_wave_body<TYPE, NC, RPW>(a, (int)blockIdx.x, a.qa, a.dm, a.y, a.resid, a.rows);
}

// A grouped launch: the matrix of this work-group is the segment its index falls in (uniform), found with fixed
// indices only, so the table stays in the argument segment (no private copy); no residual.
template <int TYPE, int NC, int RPW>
__global__ void __launch_bounds__(1024) q8_wave_group_kernel(Q8Args a, Q8Group g) {
    const int wg = (int)blockIdx.x;
    int base = 0, rows = g.seg[0].rows;
    const uint8_t *wqa = g.seg[0].qa, *wdm = g.seg[0].dm;
    float *wy = g.seg[0].y;
#pragma unroll
    for (int i = 1; i < Q8_MAXSEG; i++)
        if (i < g.nseg && wg >= g.seg[i].wg0) { // wg0 increases: the last one reached is this one's
            base = g.seg[i].wg0;
            wqa = g.seg[i].qa;
            wdm = g.seg[i].dm;
            wy = g.seg[i].y;
            rows = g.seg[i].rows;
        }
    q8_wave_body<TYPE, NC, RPW>(a, wg - base, wqa, wdm, wy, nullptr, rows);
}

// ---------------------------------------------------------------------------------------------- repack
// One thread per block: ggml bytes <-> planes (to_planes selects the direction).
__global__ void repack_kernel(int type, size_t nblocks, size_t nb, uint8_t *ggml, uint8_t *qa, uint8_t *qb,
                              uint8_t *sc, uint8_t *dm, bool to_planes) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const size_t row = i / nb, sb = i % nb; // ggml block i = row * nb + sb
    auto mv = [&](uint8_t *plane_byte, uint8_t *ggml_byte) {
        if (to_planes)
            *plane_byte = *ggml_byte;
        else
            *ggml_byte = *plane_byte;
    };
    switch (type) {
    case AQ_TYPE_Q4_K:
    case AQ_TYPE_Q5_K: {
        const bool q5 = type == AQ_TYPE_Q5_K;
        uint8_t *g = ggml + i * (q5 ? 176 : 144);
        for (int b = 0; b < 16; b++) mv(sc + kq_sc_off(row, sb, nb) + b, g + b); // d, dmin, 12 scale bytes
        if (q5)
            for (int l = 0; l < 8; l++)
                for (int b = 0; b < 4; b++) mv(qb + kq_qb5_off(row, sb, nb, l) + b, g + 16 + 4 * l + b);
        uint8_t *qs = g + (q5 ? 48 : 16);
        for (int l = 0; l < 8; l++)
            for (int j = 0; j < 4; j++)
                for (int b = 0; b < 4; b++) mv(qa + kq_qa_off(row, sb, nb, l) + j * 4 + b, qs + 32 * j + 4 * l + b);
        break;
    }
    case AQ_TYPE_Q6_K: {
        uint8_t *g = ggml + i * 210;
        for (int l = 0; l < 8; l++)
            for (int h = 0; h < 2; h++) {
                for (int jj = 0; jj < 2; jj++)
                    for (int b = 0; b < 4; b++)
                        mv(qa + kq_qa_off(row, sb, nb, l) + (h * 2 + jj) * 4 + b, g + h * 64 + jj * 32 + 4 * l + b);
                for (int b = 0; b < 4; b++) mv(qb + kq_qb6_off(row, sb, nb, l) + h * 4 + b, g + 128 + h * 32 + 4 * l + b);
            }
        for (int b = 0; b < 16; b++) mv(sc + kq_sc_off(row, sb, nb) + b, g + 192 + b);
        for (int b = 0; b < 2; b++) mv(dm + kq_dm_off(row, sb, nb) + b, g + 208 + b);
        break;
    }
    case AQ_TYPE_Q8_0: {
        uint8_t *g = ggml + i * 34;
        for (int b = 0; b < 2; b++) mv(dm + i * 2 + b, g + b);
        for (int b = 0; b < 32; b++) mv(qa + i * 32 + b, g + 2 + b);
        break;
    }
    case AQ_TYPE_Q4_0: {
        uint8_t *g = ggml + i * 18;
        for (int b = 0; b < 2; b++) mv(dm + i * 2 + b, g + b);
        for (int b = 0; b < 16; b++) mv(qa + i * 16 + b, g + 2 + b);
        break;
    }
    default: {
        uint8_t *g = ggml + i * 4;
        for (int b = 0; b < 4; b++) mv(qa + i * 4 + b, g + b);
    }
    }
}

// dot.rs:180-200 for F32 weights (ssm_alpha / ssm_beta: few rows, long columns): one work-group per row;
// thread b computes block b's 32-element partial left to right for every column, then one thread per column
// adds the partials in block order (acc += part), and `acc + 0.0f` when the row has no short tail.
template <int NC>
__global__ void __launch_bounds__(256) f32_matmul_kernel(Q8Args a) {
    extern __shared__ float prods[]; // nb32 x NC
    const int row = blockIdx.x, nb = a.nb32;
    const size_t n = a.n;
    const int c0 = (int)blockIdx.y * NC, nc = a.ncols - c0 < NC ? a.ncols - c0 : NC; // this work-group's columns
    const float *w = reinterpret_cast<const float *>(a.qa) + (size_t)row * n;
    for (int b = threadIdx.x; b < nb; b += 256) {
        const size_t e0 = (size_t)b * 32;
        const int ne = n - e0 < 32 ? (int)(n - e0) : 32;
        float wv[32];
        if (ne == 32 && n % 4 == 0) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 t = *reinterpret_cast<const float4 *>(w + e0 + 4 * i);
                wv[4 * i] = t.x;
                wv[4 * i + 1] = t.y;
                wv[4 * i + 2] = t.z;
                wv[4 * i + 3] = t.w;
            }
        } else {
            for (int i = 0; i < 32; i++) wv[i] = i < ne ? w[e0 + i] : 0.0f;
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            if (c >= nc) break; // uniform
            const float *x = a.xf + (size_t)(c0 + c) * n + e0;
            float part = 0.0f;
            if (ne == 32 && n % 4 == 0) {
                float xv[32];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float4 t = *reinterpret_cast<const float4 *>(x + 4 * i);
                    xv[4 * i] = t.x;
                    xv[4 * i + 1] = t.y;
                    xv[4 * i + 2] = t.z;
                    xv[4 * i + 3] = t.w;
                }
#pragma unroll
                for (int i = 0; i < 32; i++) part += wv[i] * xv[i];
            } else {
                for (int i = 0; i < ne; i++) part += wv[i] * x[i];
            }
            prods[b * NC + c] = part;
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < nc) {
        const int c = threadIdx.x;
        float acc = 0.0f;
        int b = 0;
        for (; b + 8 <= nb; b += 8) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = prods[(b + i) * NC + c];
#pragma unroll
            for (int i = 0; i < 8; i++) acc += v[i];
        }
        for (; b < nb; b++) acc += prods[b * NC + c];
        if (n % 32 == 0) acc = acc + 0.0f;
        const size_t o = (size_t)(c0 + c) * a.rows + row;
        a.y[o] = a.resid ? a.resid[o] + acc : acc;
    }
}

// Work-groups of `fn` (`threads` threads, `lds` dynamic bytes) resident on the whole device at once.
inline long q8_capacity(const void *fn, int threads, size_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<const void *, int, size_t>, long> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_tuple(fn, threads, lds);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds) != hipSuccess)
        return 0;
    return cache[key] = (long)per_cu * cus;
}

// Compute units of the current device (0 if the query fails).
inline long q8_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 1;
    return cus > 0 ? cus : 1;
}

template <int NC>
int launch_q8_nc(const Q8Args &args, hipStream_t stream, const Q8Group *grp = nullptr) {
    if (args.type == AQ_TYPE_F32) {
        const size_t lds = (size_t)args.nb32 * NC * sizeof(float);
        if (lds > 64 * 1024) return fail(AQ_EUNSUP, "f32 matmul: row too long for the LDS chain");
        // NC columns per work-group, the column groups along grid y (ncols past NC: a prompt chunk's rows)
        const dim3 grid((unsigned)args.rows, (unsigned)((args.ncols + NC - 1) / NC));
        hipLaunchKernelGGL((f32_matmul_kernel<NC>), grid, dim3(256), lds, stream, args);
        return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "f32_matmul launch");
    }
    {
        // the wave kernel: activations staged in LDS
        // per wave: NC x RPW records of 64 / RPW + 1 floats (at most NC * 68)
        const size_t stage = (size_t)args.nb32 * (q8w_xs(NC) + NC * 8), xw = (size_t)NC * 68 * 4;
        if (grp && (stage + 4 * xw > 64 * 1024 || NC > 4)) return fail(AQ_EUNSUP, "q8 group: not this launch shape");
        if (stage + 4 * xw <= 64 * 1024) {
            // rows per wave: the most that still give the grid about four waves per SIMD (one column: two rows
            // from 4096, measured faster for the MTP's Q4_0 matrices)
            long all_rows = args.rows;
            if (grp) {
                all_rows = 0;
                for (int i = 0; i < grp->nseg; i++) all_rows += grp->seg[i].rows;
            }
            const int rpw = all_rows >= 16384 ? 4 : (all_rows >= 8192 || (NC == 1 && all_rows >= 4096) ? 2 : 1);
            const bool q4 = args.type == AQ_TYPE_Q4_0;
            const void *k4[2] = {(const void *)&q8_wave_kernel<AQ_TYPE_Q8_0, NC, 4>,
                                 (const void *)&q8_wave_kernel<AQ_TYPE_Q4_0, NC, 4>};
            const void *k2[2] = {(const void *)&q8_wave_kernel<AQ_TYPE_Q8_0, NC, 2>,
                                 (const void *)&q8_wave_kernel<AQ_TYPE_Q4_0, NC, 2>};
            const void *k1[2] = {(const void *)&q8_wave_kernel<AQ_TYPE_Q8_0, NC, 1>,
                                 (const void *)&q8_wave_kernel<AQ_TYPE_Q4_0, NC, 1>};
            const void *fn = (rpw == 4 ? k4 : rpw == 2 ? k2 : k1)[q4 ? 1 : 0];
            // waves per work-group: of 16, 8, 4 (grids resident in one pass), the one whose busiest CU holds the
            // fewest waves (work-groups are dealt to the CUs in turn), the larger on a tie (less staging)
            int nwv = 4;
            long best = -1;
            const long cus = q8_cus();
            for (int w : {16, 8, 4}) {
                const size_t lds = stage + w * xw;
                const long grid = (all_rows + (long)w * rpw - 1) / ((long)w * rpw);
                if (lds > 64 * 1024 || grid > q8_capacity(fn, 64 * w, lds)) continue;
                const long busiest = (grid + cus - 1) / cus * w;
                if (best < 0 || busiest < best) {
                    best = busiest;
                    nwv = w;
                }
            }
            const size_t lds = stage + nwv * xw;
            const int rpg = nwv * rpw; // rows per work-group
            long nwg = (args.rows + rpg - 1) / rpg;
            Q8Group g{};
            if (grp) { // each matrix its own whole work-groups, in order
                g = *grp;
                nwg = 0;
                for (int i = 0; i < g.nseg; i++) {
                    g.seg[i].wg0 = (int)nwg;
                    nwg += (g.seg[i].rows + rpg - 1) / rpg;
                }
            }
            const dim3 grid((unsigned)nwg), block(64 * nwv);
#define AQ_Q8W(R)                                                                                             \
    if constexpr (NC <= 4) {                                                                                  \
        if (grp) {                                                                                            \
            if (q4)                                                                                           \
                hipLaunchKernelGGL((q8_wave_group_kernel<AQ_TYPE_Q4_0, NC, R>), grid, block, lds, stream, args, g); \
            else                                                                                              \
                hipLaunchKernelGGL((q8_wave_group_kernel<AQ_TYPE_Q8_0, NC, R>), grid, block, lds, stream, args, g); \
            return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "q8_wave group launch");              \
        }                                                                                                     \
    }                                                                                                         \
    if (q4)                                                                                                   \
        hipLaunchKernelGGL((q8_wave_kernel<AQ_TYPE_Q4_0, NC, R>), grid, block, lds, stream, args);             \
    else                                                                                                      \
        hipLaunchKernelGGL((q8_wave_kernel<AQ_TYPE_Q8_0, NC, R>), grid, block, lds, stream, args);
            if (rpw == 4) {
                AQ_Q8W(4)
            } else if (rpw == 2) {
                AQ_Q8W(2)
            } else {
                AQ_Q8W(1)
            }
#undef AQ_Q8W
            return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "q8_wave launch");
        }
    }
    // longer rows: rows per block chosen so the LDS products fit in 64 KiB
    const size_t per_row = (size_t)args.nb32 * NC * sizeof(float);
    int rpb = 16;
    while (rpb > 1 && per_row * rpb > 64 * 1024) rpb /= 2;
    if (per_row * rpb > 64 * 1024) return fail(AQ_EUNSUP, "q8 matmul: row too long for the LDS chain");
    const size_t lds = per_row * rpb;
    const dim3 block(256);
    switch (rpb) {
#define CASE(R)                                                                                               \
    case R:                                                                                                   \
        hipLaunchKernelGGL((q8_matmul_kernel<NC, R>), dim3((unsigned)((args.rows + R - 1) / R)), block, lds, stream, \
                           args);                                                                             \
        break;
        CASE(16) CASE(8) CASE(4) CASE(2) CASE(1)
#undef CASE
    }
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "q8_matmul launch");
}

} // namespace

int launch_matmul_many(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream) {
    if (ncols <= 8) return launch_matmul(w, x, ncols, y, resid, stream);
    if ((is_kquant(w.type) && !q8_fine()) || ((w.type == AQ_TYPE_Q8_0 || w.type == AQ_TYPE_Q4_0) && w.cols % 256 == 0))
        return launch_gemm(w, x, ncols, y, resid, stream);
    if (w.type == AQ_TYPE_F32) return launch_matmul(w, x, ncols, y, resid, stream); // one launch, column groups
    // K-quants under the q8-fine switch, Q8_0 / Q4_0 rows not a multiple of 256 long
    for (size_t c0 = 0; c0 < ncols; c0 += 8) {
        const size_t tc = ncols - c0 < 8 ? ncols - c0 : 8;
        Act v = x;
        v.ncols = x.ncols - c0;
        v.f32 = x.f32 + c0 * x.n;
        v.qs = x.qs + c0 * x.n;
        v.d = x.d + c0 * x.nb;
        v.bs = x.bs + c0 * x.nb * 16;
        v.q8s = x.q8s + c0 * x.nb * 8;
        v.q0 = x.q0 + c0 * x.n;
        v.d0 = x.d0 + c0 * x.nb32;
        v.h0 = x.h0 + c0 * x.nb32;
        v.s0 = x.s0 + c0 * x.nb32;
        const int rc = launch_matmul(w, v, tc, y + c0 * w.rows, resid ? resid + c0 * w.rows : nullptr, stream);
        if (rc) return rc;
    }
    return 0;
}

int launch_matmul(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream) {
    if (is_kquant(w.type))
        return q8_fine() ? launch_kq_q8f(w, x, ncols, y, resid, stream) : launch_kq_mfma(w, x, ncols, y, resid, stream);
    Q8Args args{};
    args.type = w.type;
    args.qa = w.qa;
    args.dm = w.dm;
    args.rows = (int)w.rows;
    args.nb32 = (int)(w.type == AQ_TYPE_F32 ? (w.cols + 31) / 32 : w.nb);
    args.xq = x.q0;
    args.xd = x.d0;
    args.xs = x.s0;
    args.xf = x.f32;
    args.n = x.n;
    args.y = y;
    args.resid = resid;
    args.ncols = (int)ncols;
    if (w.type == AQ_TYPE_F32 && ncols > 8) return launch_q8_nc<8>(args, stream); // groups of 8 along grid y
    switch (ncols) {
    case 1: return launch_q8_nc<1>(args, stream);
    case 2: return launch_q8_nc<2>(args, stream);
    case 3: return launch_q8_nc<3>(args, stream);
    case 4: return launch_q8_nc<4>(args, stream);
    case 5: return launch_q8_nc<5>(args, stream);
    case 6: return launch_q8_nc<6>(args, stream);
    case 7: return launch_q8_nc<7>(args, stream);
    case 8: return launch_q8_nc<8>(args, stream);
    default: return fail(AQ_EINVAL, "matmul: ncols must be 1..8 for Q8_0/Q4_0/F32 weights in this build");
    }
}

int launch_q8_group(const Weight *const *ws, float *const *ys, int n, const Act &x, size_t ncols, hipStream_t stream) {
    const int t = ws[0]->type;
    bool one = n >= 2 && n <= Q8_MAXSEG && ncols >= 1 && ncols <= 4 && (t == AQ_TYPE_Q8_0 || t == AQ_TYPE_Q4_0);
    for (int i = 1; i < n && one; i++) one = ws[i]->type == t && ws[i]->nb == ws[0]->nb && ws[i]->cols == ws[0]->cols;
    // the wave kernel's staging for ncols columns (the condition launch_q8_nc applies)
    const size_t stage = ws[0]->nb * ((size_t)q8w_xs((int)ncols) + ncols * 8), xw = ncols * 68 * 4;
    if (!one || stage + 4 * xw > 64 * 1024) {
        for (int i = 0; i < n; i++) {
            const int rc = launch_matmul(*ws[i], x, ncols, ys[i], nullptr, stream);
            if (rc) return rc;
        }
        return 0;
    }
    Q8Args args{};
    args.type = t;
    args.qa = ws[0]->qa;
    args.dm = ws[0]->dm;
    args.rows = (int)ws[0]->rows;
    args.nb32 = (int)ws[0]->nb;
    args.xq = x.q0;
    args.xd = x.d0;
    args.xs = x.s0;
    args.xf = x.f32;
    args.n = x.n;
    args.y = ys[0];
    args.resid = nullptr;
    args.ncols = (int)ncols;
    Q8Group g{};
    g.nseg = n;
    for (int i = 0; i < n; i++) g.seg[i] = Q8Seg{ws[i]->qa, ws[i]->dm, ys[i], (int)ws[i]->rows, 0};
    switch (ncols) {
    case 1: return launch_q8_nc<1>(args, stream, &g);
    case 2: return launch_q8_nc<2>(args, stream, &g);
    case 3: return launch_q8_nc<3>(args, stream, &g);
    default: return launch_q8_nc<4>(args, stream, &g);
    }
}

int launch_repack(Weight &w, const uint8_t *ggml_dev, bool to_planes, hipStream_t stream) {
    const size_t nblocks = w.rows * w.nb;
    const unsigned grid = (unsigned)((nblocks + 255) / 256);
    hipLaunchKernelGGL(repack_kernel, dim3(grid), dim3(256), 0, stream, w.type, nblocks, w.nb,
                       const_cast<uint8_t *>(ggml_dev), w.qa, w.qb, w.sc, w.dm, to_planes);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "repack launch");
}

} // namespace aq
