// Fused NOVA F(6,3) forward for gfx950, position-row variant, built for small
// batches: input transform, the 64 Winograd-domain MFMA products and the
// output transform in one launch.
//
// Replaces the reference's fused kernel
// (/root/reference/csrc/nova_winograd_fused.hip:283-440: one workgroup per
// 16 tiles x 64 output channels x all 64 positions, the input transform
// recomputed per output-channel chunk, 16x16x16 MFMA) with a decomposition
// that spreads one small-batch layer over all of MI355X's 256 CUs:
//   * grid = tile blocks x output-channel blocks (16, 32 or 64 channels) x 8
//     position rows. Workgroup (tb, kb, i) computes row i of V = B^T d B (8 of
//     the 64 positions) for its tile block, so the filter U -- the largest
//     operand at small batch -- is streamed by every CU at once, each reading
//     a disjoint slice, and no workgroup holds more than one row of V;
//   * input staging: per 32-channel chunk the tile block's input rows are
//     copied into LDS as 16-byte-aligned row spans (anchored at the block's
//     first column, image borders masked on read); the next chunk's loads are
//     issued before the current chunk's arithmetic;
//   * products: one v_mfma_f32_16x16x32_f16 per chunk, position and row
//     tile, V from LDS and U from its fragment-ordered copy (1 KB contiguous
//     per wave load);
//   * M, rounded to fp16 (the reference's rounding point,
//     nova_winograd_fused.hip:405), goes to a scratch buffer with agent-scope
//     (write-through) stores; each workgroup waits for its stores to complete
//     before it counts itself done on an agent-scope counter. The last of the
//     8 row workgroups of a (tile block, channel block) to arrive reads the 64
//     positions back with agent-scope loads and runs the output transform;
//     it also returns the counter to zero, so every launch finds the counters
//     at zero. Nobody waits on another workgroup.
// Both transforms use the shared tile arithmetic (bit-identical to the
// standalone kernels); products accumulate over 32-channel chunks in order.
#include <algorithm>

#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

constexpr int kFThreads = 256;
constexpr int kFCC = 32;                        // channels per chunk (two 16-channel k-steps)
constexpr int kFVBytes = 8 * kFCC * 16 * 2;     // one V row: 8 positions x 32 ch x 16 tiles
constexpr int kFXBytes = 69632;                 // staged input rows of one chunk
constexpr int kFMaxPieces = 16;                 // 16-byte staging loads per thread per chunk
constexpr int kFOob = (int)0x80000000;          // buffer offset that reads 0 / drops stores

struct FusedArgs {
    const void* x_al;  // x rounded down to 16 bytes
    const _Float16* Uf;  // fragment-ordered U
    _Float16* y;
    _Float16* Ms;
    unsigned* cnt;
    int x_bytes;  // bytes from x_al through the dword holding the last element of x
    int xd;       // x - x_al in bytes
    int u_bytes, y_bytes;
    int C, K, Cp, H, W, pad, nh, nw, Ho, Wo;
    int tbh, tbw, nbh, nbw, n_kb;
    int rr, rp, cp, nj;  // staging geometry: rows, row pitch, channel pitch (bytes), loads/row
    int nkt, nkp;        // 16-row tiles / 32-channel chunks of the fragment-ordered U
    const _Float16* bias;  // output epilogue (null: none)
    int relu;
    const _Float16* residual;  // added after the bias, y's layout (null: none)
    int nwg;                   // workgroups in the grid (gridDim.x; a kernel that reads gridDim gets hidden arguments)
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// V row layout (halves): [position q][channel group][tile][16-channel half of
// the chunk][4 channels]: the B operand of lane l (tile l % 16, channels
// 4*(l/16)..+3 of both halves, paired like the fragment-ordered U) is one
// 16-byte read.
__device__ __forceinline__ int v_slot(int q, int c, int t) {
    return (((q * 4 + ((c >> 2) & 3)) * 16 + t) * 2 + ((c >> 4) & 1)) * 4 + (c & 3);
}

// Row I of V for one (channel, tile) patch out of the staged rows. rb: LDS
// byte of (patch row 0, column 0) before the per-row alignment shift rho[ii];
// bit ii of rmask / bit j of cmask: input row / column inside the image.
template <int I>
__device__ __forceinline__ void v_row(const unsigned char* xs, int rb, int rp, unsigned rho_pack,
                                      unsigned rmask, unsigned cmask, float out[8]) {
    unsigned dd[8][4];
#pragma unroll
    for (int ii = 0; ii < 8; ii++) {
        if (input_row_uses(I, ii)) {
            const int rho = (int)((rho_pack >> (4 * ii)) & 15u);
            const unsigned* src = reinterpret_cast<const unsigned*>(xs + rb + ii * rp + (rho & ~3));
            unsigned w5[5];
#pragma unroll
            for (int q = 0; q < 5; q++) w5[q] = src[q];
#pragma unroll
            for (int q = 0; q < 4; q++)
                dd[ii][q] = __builtin_amdgcn_alignbyte(w5[q + 1], w5[q], (unsigned)(rho & 3));
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) dd[ii][q] = 0u;
        }
    }
    input_row<I>(
        [&](int ii, int j) {
            const unsigned pr = dd[ii][j >> 1];
            const unsigned short bits = (unsigned short)((j & 1) ? (pr >> 16) : (pr & 0xffffu));
            return ((rmask >> ii) & (cmask >> j) & 1u) ? (float)__builtin_bit_cast(_Float16, bits)
                                                        : 0.0f;
        },
        out);
}

__device__ __forceinline__ void v_row_dispatch(int I, const unsigned char* xs, int rb, int rp,
                                               unsigned rho_pack, unsigned rmask, unsigned cmask,
                                               float out[8]) {
    switch (I) {
        case 0: v_row<0>(xs, rb, rp, rho_pack, rmask, cmask, out); break;
        case 1: v_row<1>(xs, rb, rp, rho_pack, rmask, cmask, out); break;
        case 2: v_row<2>(xs, rb, rp, rho_pack, rmask, cmask, out); break;
        case 3: v_row<3>(xs, rb, rp, rho_pack, rmask, cmask, out); break;
        case 4: v_row<4>(xs, rb, rp, rho_pack, rmask, cmask, out); break;
        case 5: v_row<5>(xs, rb, rp, rho_pack, rmask, cmask, out); break;
        case 6: v_row<6>(xs, rb, rp, rho_pack, rmask, cmask, out); break;
        default: v_row<7>(xs, rb, rp, rho_pack, rmask, cmask, out); break;
    }
}

template <int NM>
__global__ __launch_bounds__(kFThreads, 1) void fused_kernel(FusedArgs a) {
    constexpr int KB = 16 * NM;  // output channels per workgroup
    __shared__ __align__(16) unsigned char lds[kFVBytes + kFXBytes];
    __shared__ unsigned s_last;
    _Float16* vs = reinterpret_cast<_Float16*>(lds);
    unsigned char* xs = lds + kFVBytes;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // ---- which (image, tile block, channel block, position row) ----
    const int L = xcd_remap(blockIdx.x, a.nwg);
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
    // byte offset (from x_al) of element (b, c=0, h=0, w=w0); may be negative
    const int xrow0 = a.xd + 2 * (b * a.C * HW + w0);
    const int chan2 = (2 * HW) & 15;
    const __amdgpu_buffer_rsrc_t xrs = rsrc(a.x_al, a.x_bytes);
    const __amdgpu_buffer_rsrc_t urs = rsrc(a.Uf, a.u_bytes);
    const __amdgpu_buffer_rsrc_t yrs = rsrc(a.y, a.y_bytes);

    // ---- staging pieces: e = (channel c, region row rr, 16-byte column j),
    // decoded once and stepped by carries ----
    const int per_c = a.rr * a.nj;
    const int total = kFCC * per_c;
    const int e_c = tid / per_c;
    const int e_rem = tid - e_c * per_c;
    const int e_r = e_rem / a.nj;
    const int e_j = e_rem - e_r * a.nj;
    const int dc = kFThreads / per_c, drem = kFThreads - dc * per_c;
    const int dr = drem / a.nj, dj = drem - dr * a.nj;

    // Piece u of this thread: its (c, rr, j) is re-derived by the same carry
    // walk at load and at store time (no per-piece offsets kept in registers).
    u4 pre[kFMaxPieces];
    auto walk = [&](int u, int& c, int& rr, int& j) {
        (void)u;
        j += dj;
        rr += dr;
        c += dc;
        if (j >= a.nj) {
            j -= a.nj;
            rr++;
        }
        if (rr >= a.rr) {
            rr -= a.rr;
            c++;
        }
    };
    auto stage_load = [&](int c0) {
        int c = e_c, rr = e_r, j = e_j;
#pragma unroll
        for (int u = 0; u < kFMaxPieces; u++) {
            const int h = h0 + rr;
            const bool ok = tid + u * kFThreads < total && h >= 0 && h < H && c0 + c < a.C;
            const int o = xrow0 + 2 * ((c0 + c) * HW + h * W);
            pre[u] = ok ? __builtin_amdgcn_raw_buffer_load_b128(xrs, (o & ~15) + 16 * j, 0, 0)
                        : u4{0u, 0u, 0u, 0u};
            walk(u, c, rr, j);
        }
    };
    auto stage_store = [&](int c0) {
        int c = e_c, rr = e_r, j = e_j;
#pragma unroll
        for (int u = 0; u < kFMaxPieces; u++) {
            const int h = h0 + rr;
            if (tid + u * kFThreads < total && h >= 0 && h < H && c0 + c < a.C)
                *reinterpret_cast<u4*>(xs + c * a.cp + rr * a.rp + 16 * j) = pre[u];
            walk(u, c, rr, j);
        }
    };

    // ---- transform pairs of this thread: (channel c, tile slot t) over the
    // tb_tiles real slots ----
    const int tb_tiles = a.tbh * a.tbw;
    const int npairs = kFCC * tb_tiles;
    int prb[2], pc[2], pt[2];
    unsigned prm[2], pcm[2], prho[2];
#pragma unroll
    for (int v = 0; v < 2; v++) {
        const int e = tid + v * kFThreads;
        const int c = e / tb_tiles, t = e - (e / tb_tiles) * tb_tiles;
        const int ta = t / a.tbw, tc = t - (t / a.tbw) * a.tbw;
        const bool ok = e < npairs && bh * a.tbh + ta < a.nh && bw * a.tbw + tc < a.nw;
        pc[v] = e < npairs ? c : -1;
        pt[v] = t;
        unsigned rm = 0, cm = 0, rh = 0;
#pragma unroll
        for (int ii = 0; ii < 8; ii++) {
            const int h = h0 + 6 * ta + ii;
            rm |= (ok && h >= 0 && h < H) ? (1u << ii) : 0u;
            rh |= (unsigned)((xrow0 + 2 * (c * HW + h * W)) & 15) << (4 * ii);
            const int w = w0 + 6 * tc + ii;
            cm |= (w >= 0 && w < W) ? (1u << ii) : 0u;
        }
        prb[v] = ok ? c * a.cp + 6 * ta * a.rp + 12 * tc : 0;
        prm[v] = rm;
        pcm[v] = cm;
        prho[v] = rh;
    }

    f4 acc[2][NM];
#pragma unroll
    for (int qq = 0; qq < 2; qq++)
#pragma unroll
        for (int m = 0; m < NM; m++) acc[qq][m] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    const int kt0 = kb * NM;  // first 16-row tile of this channel block
    stage_load(0);
    for (int c0 = 0; c0 < a.Cp; c0 += kFCC) {
        __syncthreads();  // previous chunk is done with xs and vs
        stage_store(c0);
        // -- U operands of this chunk: 2 positions x NM row tiles --
        h8 ua[2][NM];
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int p = 8 * i + 2 * wave + qq;
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const int kt = kt0 + m;
                const int soff = kt < a.nkt ? ((p * a.nkt + kt) * a.nkp + (c0 >> 5)) * 1024 : kFOob;
                ua[qq][m] = __builtin_bit_cast(
                    h8, __builtin_amdgcn_raw_buffer_load_b128(urs, lane * 16, soff, 0));
            }
        }
        __syncthreads();
        if (c0 + kFCC < a.Cp) stage_load(c0 + kFCC);  // next chunk's rows, in flight
        // -- row i of V for this thread's pairs --
#pragma unroll
        for (int v = 0; v < 2; v++) {
            if (pc[v] < 0) continue;
            const int cg = c0 + pc[v];
            const unsigned rm = cg < a.C ? prm[v] : 0u;
            // alignment shift of each patch row for this chunk's channel
            unsigned rho_pack = 0;
#pragma unroll
            for (int ii = 0; ii < 8; ii++)
                rho_pack |= (((prho[v] >> (4 * ii)) + (unsigned)(c0 * chan2)) & 15u) << (4 * ii);
            float out[8];
            v_row_dispatch(i, xs, prb[v], a.rp, rho_pack, rm, pcm[v], out);
#pragma unroll
            for (int q = 0; q < 8; q++) vs[v_slot(q, pc[v], pt[v])] = to_f16(out[q]);
        }
        __syncthreads();
        // -- products: this wave's two positions x NM row tiles --
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int q = 2 * wave + qq;
            const h8 bv = *reinterpret_cast<const h8*>(vs + (q * 64 + lane) * 8);
#pragma unroll
            for (int m = 0; m < NM; m++)
                acc[qq][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ua[qq][m], bv, acc[qq][m], 0,
                                                                    0, 0);
        }
    }

    // ---- M (fp16) of positions 8i + 2*wave + {0,1} to the scratch buffer,
    // Ms[blk][i][kk][t][q], one 4-byte agent-scope store per (kk, t) ----
    {
        const int t = lane & 15;
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
                const int kk = 16 * m + 4 * (lane >> 4) + rr;
                const unsigned lo = __builtin_bit_cast(uint16_t, to_f16(acc[0][m][rr]));
                const unsigned hi = __builtin_bit_cast(uint16_t, to_f16(acc[1][m][rr]));
                const int64_t o = ((((int64_t)blk * 8 + i) * KB + kk) * 16 + t) * 8 + 2 * wave;
                __hip_atomic_store(reinterpret_cast<unsigned*>(a.Ms + o), lo | (hi << 16),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
    }
    // Hand-off under the memory model: every thread's M stores are released
    // at agent scope, the workgroup barrier orders them before thread 0's
    // acquire-release increment of the block's counter, and the workgroup
    // that observes the count 7 (the last of the block's 8 position rows)
    // acquires at agent scope in every thread before it reads the other
    // workgroups' M.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0) {
        const unsigned old =
            __hip_atomic_fetch_add(a.cnt + blk, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == 7u ? 1u : 0u;
    }
    __syncthreads();
    if (s_last == 0u) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // every other workgroup of the block has arrived: none touches the counter
    // again in this launch, so it is returned to zero for the next one
    if (tid == 0) __hip_atomic_store(a.cnt + blk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- last arriver: output transform of (kk, tile) pairs ----
    for (int e = tid; e < KB * 16; e += kFThreads) {
        const int t = e & 15, kk = e >> 4;
        const int k = kb * KB + kk;
        const int ta = t / a.tbw, tc = t - (t / a.tbw) * a.tbw;
        const int th = bh * a.tbh + ta, tw = bw * a.tbw + tc;
        if (t >= tb_tiles || th >= a.nh || tw >= a.nw || k >= a.K) continue;
        const unsigned long long* src = reinterpret_cast<const unsigned long long*>(
            a.Ms + ((((int64_t)blk * 8) * KB + kk) * 16 + t) * 8);
        typedef unsigned long long ull2 __attribute__((ext_vector_type(2)));
        h8 mv[8];
#pragma unroll
        for (int ii = 0; ii < 8; ii++) {
            const unsigned long long* q = src + (int64_t)ii * KB * 16 * 2;
            const unsigned long long lo =
                __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned long long hi =
                __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            mv[ii] = __builtin_bit_cast(h8, ull2{lo, hi});
        }
        float out[6][6];
        output_tile([&](int ii, int j) { return (float)mv[ii][j]; }, out);
        const int oh = th * 6, ow = tw * 6;
        const int ybase = 2 * (((b * a.K + k) * a.Ho + oh) * a.Wo + ow);
        const __amdgpu_buffer_rsrc_t rrs = rsrc(a.residual, a.residual ? a.y_bytes : 0);
#pragma unroll
        for (int rr = 0; rr < 6; rr++) {
            if (oh + rr >= a.Ho) break;
#pragma unroll
            for (int ss = 0; ss < 6; ss++)
                if (ow + ss < a.Wo) {
                    const int off = ybase + 2 * (rr * a.Wo + ss);
                    _Float16 v = epilogue(out[rr][ss], a.bias, k, a.residual ? 0 : a.relu);
                    if (a.residual)
                        v = add_residual(v,
                                         __builtin_bit_cast(_Float16,
                                                            __builtin_amdgcn_raw_buffer_load_b16(
                                                                rrs, off, 0, 0)),
                                         a.relu);
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs, off,
                                                          0, 0);
                }
        }
    }
}

int round16(int v) { return (v + 15) & ~15; }

}  // namespace

// ---------------------------------------------------------------------------
// Host side: plan and launch.
// ---------------------------------------------------------------------------
bool fused_plan(int B, int C, int K, int Cp, int H, int W, int nh, int nw, FusedPlan* p) {
    (void)C;
    (void)H;
    (void)W;
    if (B < 1 || K < 1 || Cp < 1) return false;
    // Tile block: fewest blocks, then fewest padded tile slots, then the
    // smallest LDS footprint, within the staging budget. Row spans hold the
    // block's 6*tbw+2 columns plus 16-byte alignment slack and one dword of
    // read-ahead.
    int best_nb = 0, best_waste = 0, best_cp = 0, best_h = 0, best_w = 0;
    for (int th = 1; th <= 16; th++) {
        for (int tw = 1; th * tw <= 16; tw++) {
            if ((th > nh && th > 1) || (tw > nw && tw > 1)) continue;
            const int rr = 6 * th + 2;
            const int rp = round16(2 * (6 * tw + 2) + 18);
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
    p->rp = round16(2 * (6 * best_w + 2) + 18);
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
    return 2 * x_elems < lim && 2 * u_elems < lim && 2 * y_elems < lim;
}

const char* fused_name(const FusedPlan& p) {
    switch (p.nm) {
        case 1: return "fused_kernel<1>";
        case 2: return "fused_kernel<2>";
        default: return "fused_kernel<4>";
    }
}

hipError_t launch_fused(const uint16_t* x, const uint16_t* Uf, uint16_t* y, uint16_t* Ms,
                        unsigned* cnt, int B, int C, int K, int Cp, int H, int W, int pad,
                        int nh, int nw, int Ho, int Wo, const FusedPlan& p, hipStream_t s,
                        Epilogue ep) {
    FusedArgs a;
    a.bias = reinterpret_cast<const _Float16*>(ep.bias);
    a.relu = ep.relu;
    a.residual = reinterpret_cast<const _Float16*>(ep.residual);
    const uintptr_t xp = reinterpret_cast<uintptr_t>(x);
    a.x_al = reinterpret_cast<const void*>(xp & ~(uintptr_t)15);
    a.xd = (int)(xp & 15);
    a.x_bytes = (int)dword_ceil(2 * (int64_t)B * C * H * W + a.xd);
    a.Uf = reinterpret_cast<const _Float16*>(Uf);
    a.u_bytes = (int)(2 * u_frag_elems(K, Cp));
    a.y = reinterpret_cast<_Float16*>(y);
    a.y_bytes = (int)(2 * (int64_t)B * K * Ho * Wo);
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
    a.nkt = (K + 15) / 16;
    a.nkp = (Cp + 31) / 32;
    const dim3 grid((unsigned)p.grid), block(kFThreads);
    a.nwg = (int)grid.x;
    switch (p.nm) {
        case 1: launch(fused_kernel<1>, grid, block, s, a); break;
        case 2: launch(fused_kernel<2>, grid, block, s, a); break;
        default: launch(fused_kernel<4>, grid, block, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace nova
