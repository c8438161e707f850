// Fused NOVA F(6,3) forward for gfx950: input transform, the 64 Winograd-domain
// MFMA products and the output transform in one launch.
//
// Replaces the reference's fused kernel
// (/root/reference/csrc/nova_winograd_fused.hip:283-440: one workgroup per
// 16 tiles x 64 output channels x all 64 positions, the input transform
// recomputed per output-channel chunk, 16x16x16 MFMA) with a decomposition
// built for MI355X's 256 CUs:
//   * grid = tile blocks x output-channel blocks (16, 32 or 64 channels) x 8
//     position rows. Workgroup (tb, kb, i) computes row i of V = B^T d B (8 of
//     the 64 positions) for its tile block. The filter U, the largest operand
//     at small batch, is then streamed by every CU at once, each reading a
//     disjoint slice, and no workgroup holds more than one row of V;
//   * input staging: per 32-channel chunk the tile block's input rows are
//     copied into LDS with 16-byte buffer loads of whole aligned row spans
//     (image borders, channel tails and row wrap-around are masked when the
//     patch is read back);
//   * products: v_mfma_f32_16x16x32_f16 with V from LDS and U from global/L2,
//     U issued before the chunk's transform so its latency is hidden;
//   * M, rounded to fp16 (the reference's rounding point,
//     nova_winograd_fused.hip:405), goes to a scratch buffer. The last of the
//     8 row workgroups of a (tile block, channel block) to finish -- found
//     with an agent-scope counter after a release fence, nobody waits -- reads
//     the 64 positions back and runs the output transform. It also resets the
//     counter, so every launch finds the counters at zero.
// Both transforms use the shared tile arithmetic (bit-identical to the
// standalone kernels); MFMA accumulation runs over 32-channel steps in
// ascending order.
#include <algorithm>

#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

constexpr int kFThreads = 256;
constexpr int kFCC = 32;                        // channels per chunk = one MFMA k-step
constexpr int kFVBytes = 8 * 4 * 16 * 16;       // one V row: [8 q][4 octets][16 tiles][8 h]
constexpr int kFXBytes = 69632;                 // staged input rows of one chunk
constexpr int kFMaxPieces = 16;                 // 16-byte staging loads per thread per chunk
constexpr int kFOob = (int)0x80000000;          // buffer offset that reads 0 / drops stores

struct FusedArgs {
    const void* x_al;  // x rounded down to 16 bytes
    const _Float16* U;
    _Float16* y;
    _Float16* Ms;
    unsigned* cnt;
    int x_bytes;  // bytes from x_al to the end of x
    int xd;       // x - x_al in bytes
    int u_bytes;
    int C, K, Cp, H, W, pad, nh, nw, Ho, Wo;
    int tbh, tbw, nbh, nbw, n_kb;
    int rr, rp, cp, nj;  // staging geometry: rows, row pitch, channel pitch (bytes), loads/row
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// Row I of V for one (channel, tile) patch. rb[ii] is the LDS byte address of
// d[ii][0]; bit ii of rmask / bit j of cmask say whether input row ii /
// column j lies inside the image (else d = 0, the reference's zero padding).
// Same chains as input_tile_rows: t[j] over ii ascending, V[I][s] over j.
template <int I>
__device__ __forceinline__ void v_row(const unsigned char* xs, const int rb[8], unsigned rmask,
                                      unsigned cmask, float out[8]) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float acc = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 8; ii++) {
            if (kBh[ii][I] != 0.0f) {
                const unsigned short raw =
                    *reinterpret_cast<const unsigned short*>(xs + rb[ii] + 2 * j);
                const unsigned keep = (rmask >> ii) & (cmask >> j) & 1u;
                const _Float16 d = __builtin_bit_cast(_Float16, (unsigned short)(keep ? raw : 0));
                acc = __builtin_fmaf(kBh[ii][I], (float)d, acc);
            }
        }
        t[j] = acc;
    }
#pragma unroll
    for (int s = 0; s < 8; s++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (kBh[j][s] != 0.0f) acc = __builtin_fmaf(t[j], kBh[j][s], acc);
        out[s] = acc;
    }
}

template <int NM>
__global__ __launch_bounds__(kFThreads, 2) void fused_kernel(FusedArgs a) {
    constexpr int KB = 16 * NM;  // output channels per workgroup
    __shared__ __align__(16) unsigned char lds[kFVBytes + kFXBytes];
    __shared__ unsigned s_last;
    unsigned char* vs = lds;
    unsigned char* xs = lds + kFVBytes;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // ---- which (image, tile block, channel block, position row) ----
    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int i = L & 7;
    const int blk = L >> 3;  // ((b*nbh + bh)*nbw + bw)*n_kb + kb
    int r = blk;
    const int kb = r % a.n_kb;
    r /= a.n_kb;
    const int bw = r % a.nbw;
    r /= a.nbw;
    const int bh = r % a.nbh;
    const int b = r / a.nbh;

    const int H = a.H, W = a.W, HW = H * W;
    const int h0 = bh * a.tbh * 6 - a.pad;
    const int w0 = bw * a.tbw * 6 - a.pad;
    const int ws_lo = w0 > 0 ? w0 : 0;
    // byte offset (from x_al) of element (b, c=0, h=0, w=ws_lo)
    const int xrow0 = a.xd + 2 * (b * a.C * HW + ws_lo);
    const __amdgpu_buffer_rsrc_t xrs = rsrc(a.x_al, a.x_bytes);
    const __amdgpu_buffer_rsrc_t urs = rsrc(a.U, a.u_bytes);

    // ---- staging pieces of this thread (chunk-invariant part) ----
    // piece e -> (channel c, region row rr, 16-byte column j16); rows outside
    // the image are not loaded (their LDS bytes are masked on read).
    const int NP = kFCC * a.rr * a.nj;
    int goff[kFMaxPieces], lofc[kFMaxPieces];  // lofc = c << 20 | LDS byte offset; -1: none
#pragma unroll
    for (int u = 0; u < kFMaxPieces; u++) {
        const int e = tid + u * kFThreads;
        goff[u] = 0;
        lofc[u] = -1;
        if (e < NP) {
            const int j16 = e % a.nj;
            const int rest = e / a.nj;
            const int rr = rest % a.rr;
            const int c = rest / a.rr;
            const int h = h0 + rr;
            if (h >= 0 && h < H) {
                const int o = xrow0 + 2 * (c * HW + h * W);
                goff[u] = (o & ~15) + 16 * j16;
                lofc[u] = (c << 20) | (c * a.cp + rr * a.rp + 16 * j16);
            }
        }
    }

    // ---- transform pairs of this thread: (channel c, tile slot t) ----
    const int tb_tiles = a.tbh * a.tbw;
    int prb[2][8];
    unsigned prm[2], pcm[2];
    int pc[2], pt[2];
#pragma unroll
    for (int v = 0; v < 2; v++) {
        const int e = tid + v * kFThreads;
        const int t = e & 15, c = e >> 4;
        pc[v] = c;
        pt[v] = t;
        const int ta = t / a.tbw, tc = t - (t / a.tbw) * a.tbw;
        const bool tile_ok =
            t < tb_tiles && bh * a.tbh + ta < a.nh && bw * a.tbw + tc < a.nw;
        unsigned rm = 0, cm = 0;
#pragma unroll
        for (int ii = 0; ii < 8; ii++) {
            const int h = h0 + 6 * ta + ii;
            const bool ok = tile_ok && h >= 0 && h < H;
            rm |= ok ? (1u << ii) : 0u;
            const int rho = (xrow0 + 2 * (c * HW + h * W)) & 15;
            // padded tile slots read a fixed in-range address (masked anyway)
            prb[v][ii] = tile_ok ? c * a.cp + (6 * ta + ii) * a.rp + rho +
                                       2 * (w0 + 6 * tc - ws_lo)
                                 : 0;
            const int w = w0 + 6 * tc + ii;
            cm |= (w >= 0 && w < W) ? (1u << ii) : 0u;
        }
        prm[v] = rm;
        pcm[v] = cm;
    }

    f4 acc[2][NM];
#pragma unroll
    for (int qq = 0; qq < 2; qq++)
#pragma unroll
        for (int m = 0; m < NM; m++) acc[qq][m] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    const int kbase = kb * KB;
    for (int c0 = 0; c0 < a.Cp; c0 += kFCC) {
        // -- U fragments of this chunk (A operands), issued first --
        h8 ua[2][NM];
        {
            const int cA = c0 + 8 * (lane >> 4);
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                const int p = 8 * i + 2 * wave + qq;
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    const int k = kbase + 16 * m + (lane & 15);
                    const int off =
                        (k < a.K && cA < a.Cp) ? 2 * ((p * a.K + k) * a.Cp + cA) : kFOob;
                    ua[qq][m] = __builtin_bit_cast(
                        h8, __builtin_amdgcn_raw_buffer_load_b128(urs, off, 0, 0));
                }
            }
        }
        // -- stage the chunk's input rows --
        __syncthreads();  // previous chunk finished reading xs and vs
        {
            const int shift = 2 * c0 * HW;
#pragma unroll
            for (int g = 0; g < kFMaxPieces; g += 8) {
                u4 val[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int lc = lofc[g + u];
                    const bool ok = lc >= 0 && c0 + (lc >> 20) < a.C;
                    val[u] = ok ? __builtin_amdgcn_raw_buffer_load_b128(xrs, goff[g + u] + shift,
                                                                         0, 0)
                                : u4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int lc = lofc[g + u];
                    if (lc >= 0 && c0 + (lc >> 20) < a.C)
                        *reinterpret_cast<u4*>(xs + (lc & 0xfffff)) = val[u];
                }
            }
        }
        __syncthreads();
        // -- row i of V for this thread's two (channel, tile) pairs --
#pragma unroll
        for (int v = 0; v < 2; v++) {
            const bool cok = c0 + pc[v] < a.C;
            const unsigned rm = cok ? prm[v] : 0u;
            float out[8];
            switch (i) {
                case 0: v_row<0>(xs, prb[v], rm, pcm[v], out); break;
                case 1: v_row<1>(xs, prb[v], rm, pcm[v], out); break;
                case 2: v_row<2>(xs, prb[v], rm, pcm[v], out); break;
                case 3: v_row<3>(xs, prb[v], rm, pcm[v], out); break;
                case 4: v_row<4>(xs, prb[v], rm, pcm[v], out); break;
                case 5: v_row<5>(xs, prb[v], rm, pcm[v], out); break;
                case 6: v_row<6>(xs, prb[v], rm, pcm[v], out); break;
                default: v_row<7>(xs, prb[v], rm, pcm[v], out); break;
            }
            _Float16* vh = reinterpret_cast<_Float16*>(vs);
            const int c = pc[v];
#pragma unroll
            for (int q = 0; q < 8; q++)
                vh[((q * 4 + (c >> 3)) * 16 + pt[v]) * 8 + (c & 7)] = to_f16(out[q]);
        }
        __syncthreads();
        // -- products: this wave's two positions x NM row blocks --
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int q = 2 * wave + qq;
            const h8 bv = *reinterpret_cast<const h8*>(
                vs + (((q * 4 + (lane >> 4)) * 16 + (lane & 15)) * 16));
#pragma unroll
            for (int m = 0; m < NM; m++)
                acc[qq][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ua[qq][m], bv, acc[qq][m], 0,
                                                                    0, 0);
        }
    }

    // ---- M (fp16) of positions 8i + 2*wave + {0,1} to the scratch buffer:
    // Ms[blk][i][kk][t][q], one 4-byte store per (kk, t) ----
    {
        const int t = lane & 15;
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
                const int kk = 16 * m + 4 * (lane >> 4) + rr;
                const h2 val = {to_f16(acc[0][m][rr]), to_f16(acc[1][m][rr])};
                const int64_t o = ((((int64_t)blk * 8 + i) * KB + kk) * 16 + t) * 8 + 2 * wave;
                *reinterpret_cast<h2*>(a.Ms + o) = val;
            }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0) {
        const unsigned old =
            __hip_atomic_fetch_add(a.cnt + blk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == 7u ? 1u : 0u;
    }
    __syncthreads();
    if (s_last == 0u) return;
    if (tid == 0) __hip_atomic_store(a.cnt + blk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

    // ---- last arriver: output transform of (kk, tile) pairs ----
    for (int e = tid; e < KB * 16; e += kFThreads) {
        const int t = e & 15, kk = e >> 4;
        const int k = kbase + kk;
        const int ta = t / a.tbw, tc = t - (t / a.tbw) * a.tbw;
        const int th = bh * a.tbh + ta, tw = bw * a.tbw + tc;
        if (t >= tb_tiles || th >= a.nh || tw >= a.nw || k >= a.K) continue;
        const _Float16* src = a.Ms + ((((int64_t)blk * 8) * KB + kk) * 16 + t) * 8;
        h8 mv[8];
#pragma unroll
        for (int ii = 0; ii < 8; ii++)
            mv[ii] = *reinterpret_cast<const h8*>(src + (int64_t)ii * KB * 16 * 8);
        float out[6][6];
        output_tile([&](int ii, int j) { return (float)mv[ii][j]; }, out);
        const int oh = th * 6, ow = tw * 6;
        _Float16* yb = a.y + ((int64_t)b * a.K + k) * a.Ho * a.Wo;
#pragma unroll
        for (int rr = 0; rr < 6; rr++) {
            if (oh + rr >= a.Ho) break;
#pragma unroll
            for (int ss = 0; ss < 6; ss++)
                if (ow + ss < a.Wo) yb[(oh + rr) * a.Wo + ow + ss] = to_f16(out[rr][ss]);
        }
    }
}

// ---------------------------------------------------------------------------
// Host side: plan and launch.
// ---------------------------------------------------------------------------
static int round16(int v) { return (v + 15) & ~15; }

bool fused_plan(int B, int C, int K, int Cp, int H, int W, int nh, int nw, FusedPlan* p) {
    (void)C;
    (void)H;
    (void)W;
    if (B < 1 || K < 1 || Cp < 1) return false;
    // Tile block: fewest blocks, then fewest padded tile slots, then the
    // smallest LDS footprint, within the staging budget.
    int best_nb = 0, best_waste = 0, best_cp = 0, best_h = 0, best_w = 0;
    for (int th = 1; th <= 16; th++) {
        for (int tw = 1; th * tw <= 16; tw++) {
            if ((th > nh && th > 1) || (tw > nw && tw > 1)) continue;
            const int rr = 6 * th + 2;
            const int rp = round16(2 * (6 * tw + 2) + 14);
            const int cp = rr * rp + 16;
            if (kFCC * cp > kFXBytes || kFCC * rr * (rp / 16) > kFMaxPieces * kFThreads) continue;
            const int nb = ((nh + th - 1) / th) * ((nw + tw - 1) / tw);
            const int waste = nb * th * tw - nh * nw;
            const bool better = best_nb == 0 || nb < best_nb ||
                                (nb == best_nb && (waste < best_waste ||
                                                   (waste == best_waste && cp < best_cp)));
            if (better) {
                best_nb = nb;
                best_waste = waste;
                best_cp = cp;
                best_h = th;
                best_w = tw;
            }
        }
    }
    if (best_nb == 0) return false;
    p->tbh = best_h;
    p->tbw = best_w;
    p->nbh = (nh + best_h - 1) / best_h;
    p->nbw = (nw + best_w - 1) / best_w;
    p->rr = 6 * best_h + 2;
    p->rp = round16(2 * (6 * best_w + 2) + 14);
    p->cp = best_cp;
    p->nj = p->rp / 16;
    p->n_tb = (int64_t)B * p->nbh * p->nbw;
    // Output-channel block: the largest (least recomputation of V) that
    // still gives the grid enough workgroups to cover the chip.
    p->nm = 4;
    while (p->nm > 1 && p->n_tb * ((K + 16 * p->nm - 1) / (16 * p->nm)) * 8 < 1024) p->nm /= 2;
    const int KB = 16 * p->nm;
    p->n_kb = (K + KB - 1) / KB;
    p->grid = p->n_tb * p->n_kb * 8;
    p->ms_bytes = p->n_tb * p->n_kb * (int64_t)8 * KB * 16 * 8 * 2;
    p->cnt_count = p->n_tb * p->n_kb;
    return p->grid < ((int64_t)1 << 31) && p->ms_bytes < ((int64_t)1 << 40);
}

bool fused_fits(int64_t x_elems, int64_t u_elems, int64_t y_elems) {
    const int64_t lim = ((int64_t)1 << 31) - 64;
    return 2 * x_elems < lim && 2 * u_elems < lim && y_elems < lim;
}

const char* fused_name(const FusedPlan& p) {
    switch (p.nm) {
        case 1: return "fused_kernel<1>";
        case 2: return "fused_kernel<2>";
        default: return "fused_kernel<4>";
    }
}

hipError_t launch_fused(const uint16_t* x, const uint16_t* U, uint16_t* y, uint16_t* Ms,
                        unsigned* cnt, int B, int C, int K, int Cp, int H, int W, int pad,
                        int nh, int nw, int Ho, int Wo, const FusedPlan& p, hipStream_t s) {
    FusedArgs a;
    const uintptr_t xp = reinterpret_cast<uintptr_t>(x);
    a.x_al = reinterpret_cast<const void*>(xp & ~(uintptr_t)15);
    a.xd = (int)(xp & 15);
    a.x_bytes = (int)(2 * (int64_t)B * C * H * W + a.xd);
    a.U = reinterpret_cast<const _Float16*>(U);
    a.u_bytes = (int)(2 * (int64_t)64 * K * Cp);
    a.y = reinterpret_cast<_Float16*>(y);
    a.Ms = reinterpret_cast<_Float16*>(Ms);
    a.cnt = cnt;
    a.C = C;
    a.K = K;
    a.Cp = Cp;
    a.H = H;
    a.W = W;
    a.pad = pad;
    a.nh = nh;
    a.nw = nw;
    a.Ho = Ho;
    a.Wo = Wo;
    a.tbh = p.tbh;
    a.tbw = p.tbw;
    a.nbh = p.nbh;
    a.nbw = p.nbw;
    a.n_kb = p.n_kb;
    a.rr = p.rr;
    a.rp = p.rp;
    a.cp = p.cp;
    a.nj = p.nj;
    const dim3 grid((unsigned)p.grid), block(kFThreads);
    switch (p.nm) {
        case 1: fused_kernel<1><<<grid, block, 0, s>>>(a); break;
        case 2: fused_kernel<2><<<grid, block, 0, s>>>(a); break;
        default: fused_kernel<4><<<grid, block, 0, s>>>(a); break;
    }
    return hipGetLastError();
}

}  // namespace nova
