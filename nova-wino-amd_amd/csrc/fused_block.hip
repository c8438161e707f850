// Fused NOVA F(6,3) forward, block variant, for layers with few channels at
// batch > 1: input transform, the 64 Winograd-domain MFMA products and the
// output transform in one launch: V and M stay in LDS, the products'
// accumulators in registers.
//
// The reference's fused kernel (/root/reference/csrc/nova_winograd_fused.hip:
// 283-440) stages V for 16 tiles in LDS, multiplies with 16x16x16 MFMA and
// keeps fp32 accumulators for 64 output channels; this kernel keeps that
// output-stationary shape and re-plans the rest for gfx950 (160 KB LDS, one
// workgroup of 8 waves per CU):
//   * workgroup = 16 consecutive tiles of one image (row-major, so runs cross
//     tile rows and no tile slot is wasted inside an image) x 64 output
//     channels x all 64 positions; 8 waves (two per SIMD), wave w owns
//     position row w (8 positions) and keeps its 128 fp32 accumulators in
//     registers for the whole channel loop;
//   * per 32-channel chunk the input rows that the run touches are staged in
//     LDS as 16-byte-aligned row spans; every thread transforms one (channel,
//     tile) patch (the full 8x8, 40 aligned LDS reads) and writes its 64
//     positions into a V buffer laid out as v_mfma_f32_16x16x32_f16 B
//     operands (one 16-byte read per lane and position);
//   * each wave then multiplies its 8 positions: U fragments (A operands)
//     straight from global/L2, the chunk's two 16-channel fragments paired
//     into one v_mfma_f32_16x16x32_f16 per (position, row tile);
//   * after the channel loop, M (rounded to fp16, the reference's rounding
//     point, nova_winograd_fused.hip:405) goes to LDS as [k][tile][position],
//     and every thread runs the output transform for 2 (k, tile) pairs.
// The transforms are the shared tile arithmetic (bit-identical to the
// standalone kernels); products accumulate over 32-channel chunks in order.
// That staged form (fused_block_kernel) serves layers above 64 input
// channels, when forced; layers with at most 64, NCHW and channels-last,
// take fused_block_kernel_direct below: the same workgroup and arithmetic,
// no staging (patch rows loaded straight into registers, V of both chunks
// built in one pass), so y is the same bit for bit.
#include <algorithm>
#include <type_traits>

#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

constexpr int kBT = 512;                            // threads per workgroup (8 waves)
constexpr int kBCC = 32;                            // channels per chunk
constexpr int kPre = 4;                             // positions of U operands prefetched
constexpr int kBMPitch = 72;                        // halves per (k, tile) row of M
constexpr int kBLdsBytes = 160 * 1024;              // whole LDS: staging + V, later M
constexpr int kBVBytes = 64 * kBCC * 16 * 2;        // 65536: V of one chunk
constexpr int kBXBytes = kBLdsBytes - kBVBytes;     // 98304: staged input rows
constexpr int kBOob = (int)0x80000000;

struct BlockArgs {
    const void* x_al;  // x rounded down to 16 bytes
    const _Float16* U;  // fragment-ordered U
    _Float16* y;
    int x_bytes, xd, u_bytes, y_bytes;
    int C, K, Cp, H, W, pad, nh, nw, Ho, Wo;
    int P;        // tiles per image
    int nruns;    // 16-tile runs per image
    int n_kblk;   // 64-channel output blocks
    int rp;       // bytes per staged row span
    int cp;       // bytes per staged channel
    int nj;       // 16-byte loads per row span
    int chan2;    // (2*H*W) mod 16: span-alignment step per channel
    int nkt, nkp; // 16-row output tiles and 32-channel chunks of the fragment-ordered U
    int y_pairs;  // 1: store output pairs as 4-byte words (even Wo, 4-byte aligned y)
    const _Float16* bias;  // output epilogue (null: none)
    int relu;
    const _Float16* residual;  // added after the bias, y's layout (null: none)
    int cols;                  // NHWC: staged pixels per row (6*nw + 2)
    int nwg;                   // workgroups in the grid (gridDim.x; a kernel that reads gridDim gets hidden arguments)
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// V layout in LDS (halves): [position][channel group of 4][tile][16-channel
// half of the chunk][4 channels] -- the B operand of lane l (tile l % 16,
// channels 4*(l/16) .. +3 of both halves, paired like the A operands of the
// fragment-ordered U) is one 16-byte read, 1 KB contiguous per wave.
__device__ __forceinline__ int v_index(int pos, int c, int t) {
    return (((pos * 4 + ((c >> 2) & 3)) * 16 + t) * 2 + ((c >> 4) & 1)) * 4 + (c & 3);
}

// v_index with the tile slot swizzled by the channel group (slot t ^ 4g for
// group g = (c >> 2) & 3): the unstaged kernel's channels-last threads write
// 32 channels of 2 tiles per instruction, whose 4 groups would otherwise
// share banks (lanes over 16 tiles of one group, the NCHW threads, stay
// conflict-free). Lane l reads its B operand at slot l ^ ((l >> 4) << 2).
__device__ __forceinline__ int v_index_sw(int pos, int c, int t) {
    return v_index(pos, c, t ^ (((c >> 2) & 3) << 2));
}

// Byte offset of the A operand of (position p, row tile kt, chunk j) in the
// fragment-ordered U; out of range (reads zero) past the last row tile.
__device__ __forceinline__ int u_off(const BlockArgs& a, int p, int kt, int j) {
    return kt < a.nkt ? ((p * a.nkt + kt) * a.nkp + j) * 1024 : kBOob;
}

// kNhwc: x and y channels-last. The chunk is then staged as [row][pixel]
// [channel] (kNhwcPix halves per pixel: 16-byte loads of 8 channels, zero for
// pixels outside the image), the transform reads its patch with 2-byte LDS
// reads, and the output phase runs with lanes over channels (128-byte NHWC
// stores). NJ is unused (0) in that form.
constexpr int kNhwcPix = 36;  // 72 bytes: tiles 6 pixels apart fall in distinct banks
// NHWC keeps M as [tile][kk][position] (tile pitch padded by 16 bytes): the
// output phase then reads consecutive channels per lane at a 144-byte stride,
// and the MFMA write, with lanes over tiles, at a 16-byte offset per tile.
constexpr int kNhwcTileP = 64 * 72 + 8;
static_assert(16 * kNhwcTileP * 2 <= 160 * 1024, "NHWC M fits in LDS");

// Output phase of the NCHW forms: thread (kk, tile t) pairs e = tid + 512 i,
// M read as 8 16-byte rows of [kk][tile][position], the output transform,
// epilogue and residual, 4-byte pair stores where y allows them.
template <bool kEpi>
__device__ __forceinline__ void output_phase_nchw(const BlockArgs& a, const _Float16* ms, int tid,
                                                  int t, bool tile_ok, int th, int tw, int b,
                                                  int k0, __amdgpu_buffer_rsrc_t yrs) {
    const bool pairs_w = a.y_pairs != 0;
    const _Float16* res = a.residual;
    const int relu0 = res ? 0 : a.relu;  // with a residual the ReLU comes after it
    const __amdgpu_buffer_rsrc_t rrs = rsrc(res, res ? a.y_bytes : 0);
    for (int e = tid; e < 64 * 16; e += kBT) {
        const int kk = e >> 4;
        const int k = k0 + kk;
        if (!tile_ok || k >= a.K) continue;
        h8 mv[8];
#pragma unroll
        for (int ii = 0; ii < 8; ii++)
            mv[ii] = *reinterpret_cast<const h8*>(ms + (kk * 16 + t) * kBMPitch + 8 * ii);
        float out[6][6];
        output_tile([&](int ii, int j) { return (float)mv[ii][j]; }, out);
        const int oh = th * 6, ow = tw * 6;
        const int ybase = 2 * ((b * a.K + k) * a.Ho * a.Wo + ow);
        const ChannelEpilogue<kEpi> epi(a.bias, k, relu0);
#pragma unroll
        for (int r = 0; r < 6; r++) {
            const int row = ybase + 2 * (oh + r) * a.Wo;
            if (oh + r >= a.Ho) break;
            if (pairs_w) {
#pragma unroll
                for (int s = 0; s < 6; s += 2) {
                    if (ow + s < a.Wo) {
                        const unsigned lo = __builtin_bit_cast(uint16_t, epi(out[r][s]));
                        const unsigned hi = __builtin_bit_cast(uint16_t, epi(out[r][s + 1]));
                        unsigned v = lo | (hi << 16);
                        if (res)
                            v = add_residual2(
                                v, __builtin_amdgcn_raw_buffer_load_b32(rrs, row + 2 * s, 0, 0),
                                a.relu);
                        __builtin_amdgcn_raw_buffer_store_b32(v, yrs, row + 2 * s, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int s = 0; s < 6; s++)
                    if (ow + s < a.Wo) {
                        _Float16 v = epi(out[r][s]);
                        if (res)
                            v = add_residual(
                                v,
                                __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(
                                                                 rrs, row + 2 * s, 0, 0)),
                                a.relu);
                        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs,
                                                              row + 2 * s, 0, 0);
                    }
            }
        }
    }
}

// Output phase of the channels-last forms: lanes over 64 consecutive output
// channels (pair e = (tile e / 64, channel e % 64)), M read as 8 16-byte rows
// of [tile][kk][position], 2-byte NHWC stores (128 bytes per wave and pixel).
template <bool kEpi>
__device__ __forceinline__ void output_phase_nhwc(const BlockArgs& a, const _Float16* ms, int tid,
                                                  int ntiles, int t0, int b, int k0,
                                                  __amdgpu_buffer_rsrc_t yrs) {
    const _Float16* res = a.residual;
    const int relu0 = res ? 0 : a.relu;  // with a residual the ReLU comes after it
    const __amdgpu_buffer_rsrc_t rrs = rsrc(res, res ? a.y_bytes : 0);
    // lanes over channels: pair e = (tile e / 64, channel e % 64)
    for (int e = tid; e < 64 * 16; e += kBT) {
        const int kk = e & 63, to = e >> 6;
        const int k = k0 + kk;
        if (to >= ntiles || k >= a.K) continue;
        h8 mv[8];
#pragma unroll
        for (int ii = 0; ii < 8; ii++)
            mv[ii] = *reinterpret_cast<const h8*>(ms + to * kNhwcTileP + kk * kBMPitch + 8 * ii);
        float out[6][6];
        output_tile([&](int ii, int j) { return (float)mv[ii][j]; }, out);
        const int tlo = t0 + to;
        const int oh = (tlo / a.nw) * 6, ow = (tlo - (tlo / a.nw) * a.nw) * 6;
        const ChannelEpilogue<kEpi> epi(a.bias, k, relu0);
#pragma unroll
        for (int r = 0; r < 6; r++) {
            if (oh + r >= a.Ho) break;
#pragma unroll
            for (int s = 0; s < 6; s++)
                if (ow + s < a.Wo) {
                    const int off = 2 * (((b * a.Ho + oh + r) * a.Wo + ow + s) * a.K + k);
                    _Float16 v = epi(out[r][s]);
                    if (res)
                        v = add_residual(
                            v,
                            __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(
                                                             rrs, off, 0, 0)),
                            a.relu);
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs,
                                                          off, 0, 0);
                }
        }
    }
}

template <int NJ, bool kNhwc, bool kEpi>
__global__ __launch_bounds__(kBT, 1) void fused_block_kernel(BlockArgs a) {
    __shared__ __align__(16) unsigned char lds[kBLdsBytes];
    unsigned char* xs = lds;
    _Float16* vs = reinterpret_cast<_Float16*>(lds + kBXBytes);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // = position row

    // ---- work item: (image b, 16-tile run, 64-channel output block) ----
    const int L = xcd_remap(blockIdx.x, a.nwg);
    const int kblk = L % a.n_kblk;
    const int rest = L / a.n_kblk;
    const int run = rest % a.nruns;
    const int b = rest / a.nruns;
    const int k0 = kblk * 64;
    const int t0 = run * 16;
    const int ntiles = min(16, a.P - t0);
    const int th_first = t0 / a.nw;
    const int nrows = (t0 + ntiles - 1) / a.nw - th_first + 1;
    const int rows_st = 6 * nrows + 2;       // staged input rows
    const int h_first = 6 * th_first - a.pad;
    const int HW = a.H * a.W;
    const __amdgpu_buffer_rsrc_t xrs = rsrc(a.x_al, a.x_bytes);
    const __amdgpu_buffer_rsrc_t urs = rsrc(a.U, a.u_bytes);
    const __amdgpu_buffer_rsrc_t yrs = rsrc(a.y, a.y_bytes);

    // ---- transform role: channel ct = tid / 16 of the chunk, tile t ----
    const int t = tid & 15;
    const int ct = tid >> 4;
    const bool tile_ok = t < ntiles;
    const int tl = t0 + (tile_ok ? t : 0);
    const int th = tl / a.nw, tw = tl - (tl / a.nw) * a.nw;
    const int rb0 = 6 * (th - th_first) * a.rp + 12 * tw;
    unsigned rr0 = 0, cmask = 0;
#pragma unroll
    for (int ii = 0; ii < 8; ii++) {
        const int h = 6 * th - a.pad + ii;
        rr0 |= (unsigned)((a.xd + 2 * (b * a.C * HW + h * a.W - a.pad)) & 15) << (4 * ii);
        const int w = 6 * tw - a.pad + ii;
        cmask |= (w >= 0 && w < a.W) ? (1u << ii) : 0u;
    }
    // column mask as four dword masks over the packed halves
    unsigned dm[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
        dm[q] = (((cmask >> (2 * q)) & 1u) ? 0xffffu : 0u) |
                (((cmask >> (2 * q + 1)) & 1u) ? 0xffff0000u : 0u);

    // ---- staging spans: (channel c, staged row r), kSpr per thread per round ----
    // Each span is NJ 16-byte loads at immediate offsets, all of a round in
    // flight at once (one span per thread and round: two would need spill
    // registers beside the accumulators); rows outside the image and
    // channels past C get an out-of-range offset, so zeros are staged for
    // them.
    constexpr int kSpr = 1;
    const int nspans = kBCC * rows_st;

    f4 acc[8][4];
#pragma unroll
    for (int s = 0; s < 8; s++)
#pragma unroll
        for (int kb = 0; kb < 4; kb++) acc[s][kb] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int c0 = 0; c0 < a.Cp; c0 += kBCC) {
        __syncthreads();  // the previous chunk is done with the staging area and V
        // -- stage the chunk's input rows --
        if constexpr (kNhwc) {
            // units (row r, pixel pc, 8-channel group g), 4 loads in flight per
            // thread (8 spill registers beside the accumulators: 5 % slower)
            const int nunits = rows_st * a.cols * 4;
            _Float16* xh = reinterpret_cast<_Float16*>(xs);
            for (int e0 = 0; e0 < nunits; e0 += 4 * kBT) {
                u4 v[4];
                int dst[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int e = e0 + tid + u * kBT;
                    const int g = e & 3, rp = e >> 2;
                    const int r = rp / a.cols, pc = rp - (rp / a.cols) * a.cols;
                    const int h = h_first + r, w = pc - a.pad, cg = c0 + 8 * g;
                    const bool live = e < nunits;
                    const bool ok = live && h >= 0 && h < a.H && w >= 0 && w < a.W && cg < a.C;
                    v[u] = __builtin_amdgcn_raw_buffer_load_b128(
                        xrs, ok ? 2 * (((b * a.H + h) * a.W + w) * a.C + cg) : kBOob, 0, 0);
                    dst[u] = live ? (r * a.cols + pc) * kNhwcPix + 8 * g : -1;
                }
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (dst[u] >= 0) {  // 8-byte aligned: two 8-byte writes
                        *reinterpret_cast<u2*>(xh + dst[u]) = u2{v[u][0], v[u][1]};
                        *reinterpret_cast<u2*>(xh + dst[u] + 4) = u2{v[u][2], v[u][3]};
                    }
            }
        } else
        for (int sp0 = 0; sp0 < nspans; sp0 += kSpr * kBT) {
            u4 v[kSpr][NJ];
            int dst[kSpr];
#pragma unroll
            for (int u = 0; u < kSpr; u++) {
                const int sp = sp0 + tid + u * kBT;
                const int c = sp / rows_st, r = sp - (sp / rows_st) * rows_st;
                const int h = h_first + r;
                const int cg = c0 + c;
                const bool live = sp < nspans;
                const int o = a.xd + 2 * ((b * a.C + cg) * HW + h * a.W - a.pad);
                const int base = (live && h >= 0 && h < a.H && cg < a.C) ? (o & ~15) : kBOob;
                dst[u] = live ? c * a.cp + r * a.rp : -1;
#pragma unroll
                for (int q = 0; q < NJ; q++)
                    v[u][q] = __builtin_amdgcn_raw_buffer_load_b128(xrs, base + 16 * q, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < kSpr; u++)
                if (dst[u] >= 0) {
#pragma unroll
                    for (int q = 0; q < NJ; q++)
                        *reinterpret_cast<u4*>(xs + dst[u] + 16 * q) = v[u][q];
                }
        }
        __syncthreads();
        // -- input transform of (channel c0 + ct, tile t) into V --
        if constexpr (kNhwc) {
            const _Float16* src = reinterpret_cast<const _Float16*>(xs) +
                                  ((6 * (th - th_first)) * a.cols + 6 * tw) * kNhwcPix + ct;
            const int rstride = a.cols * kNhwcPix;
            // the whole patch into registers first: the V writes below could
            // alias the staging area for the compiler, which would re-read it
            // (packed in pairs, as the NCHW form holds it)
            h2 d[8][4];
#pragma unroll
            for (int ii = 0; ii < 8; ii++) {
#pragma unroll
                for (int q = 0; q < 4; q++)
                    d[ii][q] = h2{src[ii * rstride + 2 * q * kNhwcPix],
                                  src[ii * rstride + (2 * q + 1) * kNhwcPix]};
                if (ii & 1) __builtin_amdgcn_sched_barrier(0);  // 16 reads in flight at most
            }
            input_tile_rows(
                [&](int ii, int j) { return (float)d[ii][j >> 1][j & 1]; },
                [&](int r, int s2, float v) { vs[v_index(r * 8 + s2, ct, t)] = to_f16(v); });
        } else {
            const int cg = c0 + ct;
            const unsigned char* cbase = xs + ct * a.cp + rb0;
            unsigned d4[8][4];
#pragma unroll
            for (int ii = 0; ii < 8; ii++) {
                const int rho = ((int)((rr0 >> (4 * ii)) & 15u) + cg * a.chan2) & 15;
                const unsigned* src =
                    reinterpret_cast<const unsigned*>(cbase + ii * a.rp + (rho & ~3));
                unsigned w5[5];
#pragma unroll
                for (int q = 0; q < 5; q++) w5[q] = src[q];
#pragma unroll
                for (int q = 0; q < 4; q++)
                    d4[ii][q] = __builtin_amdgcn_alignbyte(w5[q + 1], w5[q], (unsigned)(rho & 3));
            }
            // edge tiles: zero the columns outside the image (rows outside it
            // and channels past C were staged as zeros)
            if (cmask != 0xffu) {
#pragma unroll
                for (int ii = 0; ii < 8; ii++)
#pragma unroll
                    for (int q = 0; q < 4; q++) d4[ii][q] &= dm[q];
            }
            input_tile_rows(
                [&](int ii, int j) {
                    const unsigned pr = d4[ii][j >> 1];
                    const unsigned short bits =
                        (unsigned short)((j & 1) ? (pr >> 16) : (pr & 0xffffu));
                    return (float)__builtin_bit_cast(_Float16, bits);
                },
                [&](int r, int s2, float v) { vs[v_index(r * 8 + s2, ct, t)] = to_f16(v); });
        }
        // the U operands of the first half of this wave's row (kPre
        // positions) are requested before the barrier, so their L2 latency
        // overlaps the wait for the slowest wave's transform (more would not
        // fit beside the accumulators without spilling)
        h8 ua0[kPre][4];
#pragma unroll
        for (int s = 0; s < kPre; s++)
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
                ua0[s][kb] = __builtin_bit_cast(
                    h8, __builtin_amdgcn_raw_buffer_load_b128(
                            urs, lane * 16, u_off(a, 8 * wave + s, k0 / 16 + kb, c0 >> 5), 0));
        __syncthreads();
        // -- products: this wave's position row, one v_mfma_f32_16x16x32_f16
        // per (position, row tile) and chunk, positions in two halves of 4
        // (64 registers of U operands beside the accumulators) --
#pragma unroll
        for (int half = 0; half < 2; half++) {
            h8 ua[4][4];
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int kb = 0; kb < 4; kb++) {
                    if (half == 0 && s < kPre) {
                        ua[s][kb] = ua0[s][kb];
                    } else {
                        ua[s][kb] = __builtin_bit_cast(
                            h8, __builtin_amdgcn_raw_buffer_load_b128(
                                    urs, lane * 16,
                                    u_off(a, 8 * wave + 4 * half + s, k0 / 16 + kb, c0 >> 5), 0));
                    }
                }
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int pos = 8 * wave + 4 * half + s;
                const h8 vb = *reinterpret_cast<const h8*>(vs + (pos * 64 + lane) * 8);
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
                    acc[4 * half + s][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        ua[s][kb], vb, acc[4 * half + s][kb], 0, 0, 0);
            }
        }
    }
    __syncthreads();  // staging area and V become M

    // ---- M (fp16) to LDS: [kk][tile][position] ([tile][kk][position] for
    // NHWC), one 16-byte write per (k, position row) of this lane ----
    _Float16* ms = reinterpret_cast<_Float16*>(lds);
    {
        const int g = lane >> 4, tq = lane & 15;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kk = 16 * kb + 4 * g + i;
                h8 v;
#pragma unroll
                for (int s = 0; s < 8; s++) v[s] = to_f16(acc[s][kb][i]);
                const int mo = kNhwc ? tq * kNhwcTileP + kk * kBMPitch : (kk * 16 + tq) * kBMPitch;
                *reinterpret_cast<h8*>(ms + mo + 8 * wave) = v;
            }
    }
    __syncthreads();

    // ---- output transform: (kk, tile) pairs, tile = tid % 16 ----
    if constexpr (kNhwc) {
        output_phase_nhwc<kEpi>(a, ms, tid, ntiles, t0, b, k0, yrs);
        return;
    }
    output_phase_nchw<kEpi>(a, ms, tid, t, tile_ok, th, tw, b, k0, yrs);
}

// ---------------------------------------------------------------------------
// Unstaged form for Cp <= 64 (NS = 1 or 2 steps of 32 channels), NCHW and
// channels-last (kNhwc: one 2-byte load per pixel, lanes over 32 channels of
// 2 tiles, so a load covers 64 bytes of consecutive channels; any C and any
// alignment of x).
// Same workgroup (16 tiles x 64 output channels x 64 positions, 8 waves)
// and the same arithmetic in the same order, so y equals the staged form's
// bit for bit; the phases are re-planned around the register budget:
//   * every thread loads its NS patches (channel ct + 32 j, tile t)
//     straight from global memory -- NCHW each row as a 16-byte and a
//     4-byte load from the dword at or below its start, all NS*16 loads in
//     flight at once -- so no LDS holds the input, and V for all NS steps
//     (NS KB per position) fits beside nothing else and is built in one
//     pass;
//   * no accumulator lives during the transform, so the U operands of the
//     wave's first kPreU positions (both steps) are requested before it, and
//     of kMidU more once the first of two patches is transformed (its
//     registers are free then); they arrive during the VALU work;
//   * each wave then finishes one position at a time (both steps, the first
//     MFMA from a zero accumulator), requesting the next position's
//     operands as registers free up;
//   * V is written in the staged form's operand layout with the tile slots
//     swizzled by channel group (v_index_sw); NCHW pairs channels c, c ^ 1
//     across lane rows with one v_permlane16_swap per two positions, so
//     every lane writes whole dwords;
//   * after a barrier, M is written over V (as the staged form lays it out
//     for the layout) and the output phase is the staged form's.
// Rows that start before x_al (only the first row of channel 0 of image 0
// with left padding and a 16-byte aligned x) are loaded from offset 0 and
// shifted into place in a branch that only the wave holding them takes.
// ---------------------------------------------------------------------------
// Positions whose U operands are requested before the transform (one step:
// 6; two steps: 3, and kMidU = 2 more once the first patch is transformed,
// as many as fit beside the transform's registers without spilling).
// Whole forwards, graph of ten, us: conv2_x B=32 22.25 (3 before) -> 21.43
// (3 + 3, before the paired V writes, which leave room for 2); C = 32 B=32
// 12.75 (3) -> 12.49 (6).
template <int NS>
constexpr int kPreU = NS == 1 ? 6 : 3;
constexpr int kMidU = 2;

template <int NS, bool kNhwc, bool kEpi>
__global__ __launch_bounds__(kBT, 1) void fused_block_kernel_direct(BlockArgs a) {
    static_assert(NS == 1 || NS == 2, "one or two 32-channel steps");
    static_assert(64 * kBMPitch * 16 * 2 <= kBLdsBytes && 16 * kNhwcTileP * 2 <= kBLdsBytes,
                  "M fits in LDS");
    __shared__ __align__(16) unsigned char lds[kBLdsBytes];
    _Float16* vs = reinterpret_cast<_Float16*>(lds);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // = position row

    const int L = xcd_remap(blockIdx.x, a.nwg);
    const int kblk = L % a.n_kblk;
    const int rest = L / a.n_kblk;
    const int run = rest % a.nruns;
    const int b = rest / a.nruns;
    const int k0 = kblk * 64;
    const int t0 = run * 16;
    const int ntiles = min(16, a.P - t0);
    const int HW = a.H * a.W;
    const __amdgpu_buffer_rsrc_t xrs = rsrc(a.x_al, a.x_bytes);
    const __amdgpu_buffer_rsrc_t urs = rsrc(a.U, a.u_bytes);
    const __amdgpu_buffer_rsrc_t yrs = rsrc(a.y, a.y_bytes);

    // ---- transform role: channel ct + 32 j (j < NS), tile t. NCHW: a wave
    // holds 16 tiles x 4 channels (a row load spans the 16 tiles of one
    // channel); channels-last: 32 channels x 2 tiles (a pixel load spans 64
    // bytes of consecutive channels) ----
    const int t = kNhwc ? tid >> 5 : tid & 15;
    const int ct = kNhwc ? tid & 31 : tid >> 4;
    const bool tile_ok = t < ntiles;
    const int tl = t0 + (tile_ok ? t : 0);
    const int th = tl / a.nw, tw = tl - (tl / a.nw) * a.nw;
    const int h0 = 6 * th - a.pad, w0 = 6 * tw - a.pad;
    unsigned cmask = 0;
#pragma unroll
    for (int ii = 0; ii < 8; ii++) {
        const int w = w0 + ii;
        cmask |= (w >= 0 && w < a.W) ? (1u << ii) : 0u;
    }
    unsigned dm[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
        dm[q] = (((cmask >> (2 * q)) & 1u) ? 0xffffu : 0u) |
                (((cmask >> (2 * q + 1)) & 1u) ? 0xffff0000u : 0u);

    // ---- patch rows: 20 bytes from the dword at or below the row start ----
    // (rows outside the image, channels past C and empty tile slots read
    // zeros through out-of-range offsets)
    unsigned w5[NS][8][5];      // NCHW: the five dwords of each row
    unsigned px[NS][8][4];      // channels-last: the patch, column pairs packed
    unsigned odd[NS], neg[NS];  // per row: start at a 2-byte offset; start before x_al
#pragma unroll
    for (int j = 0; j < NS; j++) {
        const int c = ct + 32 * j;
        odd[j] = 0;
        neg[j] = 0;
        if constexpr (kNhwc) {
            // one 2-byte load per pixel; pixels outside the image read zero
#pragma unroll
            for (int ii = 0; ii < 8; ii++) {
                const int h = h0 + ii;
                const bool rok = tile_ok && c < a.C && h >= 0 && h < a.H;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    unsigned pr = 0;
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const int w = w0 + 2 * q + e;
                        const bool ok = rok && w >= 0 && w < a.W;
                        const int o = a.xd + 2 * (((b * a.H + h) * a.W + w) * a.C + c);
                        pr |= (unsigned)__builtin_amdgcn_raw_buffer_load_b16(xrs, ok ? o : kBOob,
                                                                             0, 0)
                              << (16 * e);
                    }
                    px[j][ii][q] = pr;
                }
            }
        } else {
#pragma unroll
            for (int ii = 0; ii < 8; ii++) {
                const int h = h0 + ii;
                const bool ok = tile_ok && c < a.C && h >= 0 && h < a.H;
                const int o = a.xd + 2 * ((b * a.C + c) * HW + h * a.W + w0);
                odd[j] |= (unsigned)((o >> 1) & 1) << ii;
                neg[j] |= (ok && o < 0) ? (1u << ii) : 0u;
                const int A = !ok ? kBOob : (o < 0 ? 0 : (o & ~3));
                const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, A, 0, 0);
#pragma unroll
                for (int q = 0; q < 4; q++) w5[j][ii][q] = v[q];
                w5[j][ii][4] = __builtin_amdgcn_raw_buffer_load_b32(xrs, A + 16, 0, 0);
            }
        }
    }

    // ---- U operands of this wave's first kPreU positions, both steps ----
    h8 ua[8][4][NS];
    auto load_u = [&](int s) {
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int j = 0; j < NS; j++)
                ua[s][kb][j] = __builtin_bit_cast(
                    h8, __builtin_amdgcn_raw_buffer_load_b128(
                            urs, lane * 16, u_off(a, 8 * wave + s, k0 / 16 + kb, j), 0));
    };
#pragma unroll
    for (int s = 0; s < kPreU<NS>; s++) load_u(s);

    // a row that starts before x_al was loaded from offset 0: move its dwords
    // up by the missing ones (zeros before the buffer, all in masked columns)
    unsigned any_neg = 0;
#pragma unroll
    for (int j = 0; j < NS; j++) any_neg |= neg[j];
    if (!kNhwc && __builtin_amdgcn_ballot_w64(any_neg != 0) != 0) {
#pragma unroll
        for (int j = 0; j < NS; j++) {
            const int c = ct + 32 * j;
#pragma unroll
            for (int ii = 0; ii < 8; ii++) {
                if (!((neg[j] >> ii) & 1u)) continue;
                const int o = a.xd + 2 * ((b * a.C + c) * HW + (h0 + ii) * a.W + w0);
                const int sh = -(o >> 2);  // dwords before x_al (o >> 2 rounds down)
                unsigned l5[5];
#pragma unroll
                for (int q = 0; q < 5; q++) l5[q] = w5[j][ii][q];
#pragma unroll
                for (int q = 0; q < 5; q++) {
                    unsigned v = 0;
#pragma unroll
                    for (int r = 0; r < 5; r++) v = (q - sh == r) ? l5[r] : v;
                    w5[j][ii][q] = v;
                }
            }
        }
    }

    // ---- input transform of the NS patches into V: [position][step][the
    // staged form's 1 KB operand block] ----
#pragma unroll
    for (int j = 0; j < NS; j++) {
        unsigned d4[8][4];
#pragma unroll
        for (int ii = 0; ii < 8; ii++) {
            const unsigned sb = ((odd[j] >> ii) & 1u) * 2;
#pragma unroll
            for (int q = 0; q < 4; q++)
                d4[ii][q] = kNhwc ? px[j][ii][q]
                                  : __builtin_amdgcn_alignbyte(w5[j][ii][q + 1], w5[j][ii][q], sb);
        }
        if (!kNhwc && cmask != 0xffu) {
#pragma unroll
            for (int ii = 0; ii < 8; ii++)
#pragma unroll
                for (int q = 0; q < 4; q++) d4[ii][q] &= dm[q];
        }
        if (j == 1) {
#pragma unroll
            for (int s = kPreU<NS>; s < kPreU<NS> + kMidU; s++) load_u(s);
        }
        _Float16* vj = vs + j * 512;
        float pend = 0.0f;  // NCHW: the even position of the pair being written
        input_tile_rows(
            [&](int ii, int jj) {
                const unsigned pr = d4[ii][jj >> 1];
                const unsigned short bits =
                    (unsigned short)((jj & 1) ? (pr >> 16) : (pr & 0xffffu));
                return (float)__builtin_bit_cast(_Float16, bits);
            },
            [&](int r, int s2, float v) {
                if constexpr (kNhwc) {
                    vj[(r * 8 + s2) * (NS * 512) + v_index_sw(0, ct, t)] = to_f16(v);
                } else {
                    // Channels c and c ^ 1 share a dword of V and sit 16 lanes
                    // apart (lane row = c % 4). Per pair of positions (p, p + 1)
                    // one row swap gives the even row both channels at p and
                    // the odd row both at p + 1: one 4-byte write per lane
                    // instead of two 2-byte writes into shared dwords.
                    if ((s2 & 1) == 0) {
                        pend = v;
                        return;
                    }
                    const auto sw = __builtin_amdgcn_permlane16_swap(
                        __builtin_bit_cast(unsigned, pend), __builtin_bit_cast(unsigned, v), false,
                        false);
                    const int pos = r * 8 + s2 - 1 + (ct & 1);
                    *reinterpret_cast<unsigned*>(vj + pos * (NS * 512) + v_index_sw(0, ct & ~1, t)) =
                        pack_f16x2(__builtin_bit_cast(float, (unsigned)sw[0]),
                                   __builtin_bit_cast(float, (unsigned)sw[1]));
                }
            });
    }
    __syncthreads();

    // ---- products: one position at a time, both steps in channel order ----
    f4 acc[8][4];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int pos = 8 * wave + s;
        h8 vb[NS];
#pragma unroll
        for (int j = 0; j < NS; j++)
            vb[j] = *reinterpret_cast<const h8*>(vs + pos * (NS * 512) + j * 512 +
                                                 (lane ^ ((lane >> 4) << 2)) * 8);
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            acc[s][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                ua[s][kb][0], vb[0], f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            if constexpr (NS == 2)
                acc[s][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ua[s][kb][1], vb[1],
                                                                    acc[s][kb], 0, 0, 0);
        }
        constexpr int kAhead = kPreU<NS> + (NS == 2 ? kMidU : 0);  // positions already requested
        if (s + kAhead < 8) load_u(s + kAhead);
    }
    __syncthreads();  // V becomes M

    // ---- M (fp16) to LDS: [kk][tile][position] ([tile][kk][position] for
    // channels-last), as the staged form ----
    _Float16* ms = reinterpret_cast<_Float16*>(lds);
    {
        const int g = lane >> 4, tq = lane & 15;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kk = 16 * kb + 4 * g + i;
                h8 v;
#pragma unroll
                for (int s = 0; s < 8; s++) v[s] = to_f16(acc[s][kb][i]);
                const int mo = kNhwc ? tq * kNhwcTileP + kk * kBMPitch : (kk * 16 + tq) * kBMPitch;
                *reinterpret_cast<h8*>(ms + mo + 8 * wave) = v;
            }
    }
    __syncthreads();
    if constexpr (kNhwc)
        output_phase_nhwc<kEpi>(a, ms, tid, ntiles, t0, b, k0, yrs);
    else
        output_phase_nchw<kEpi>(a, ms, tid, t, tile_ok, th, tw, b, k0, yrs);
}

int round16i(int v) { return (v + 15) & ~15; }

}  // namespace

bool fused_block_plan(int B, int C, int K, int Cp, int H, int W, int nh, int nw,
                      FusedBlockPlan* p, bool nhwc) {
    if (B < 1 || C < 1 || K < 1) return false;
    const int P = nh * nw;
    const int nruns = (P + 15) / 16;
    int maxrows = 1;
    for (int r = 0; r < nruns; r++) {
        const int t0 = 16 * r, n = std::min(16, P - t0);
        maxrows = std::max(maxrows, (t0 + n - 1) / nw - t0 / nw + 1);
    }
    const int rows_st = 6 * maxrows + 2;
    p->nhwc = nhwc;
    if (Cp <= 64) {
        // the unstaged form (fused_block_kernel_direct): no limit on the image
        // width, any C and any alignment of x
        p->cols = p->rp = p->cp = p->nj = 0;
    } else if (nhwc) {
        // [row][pixel][channel] staging; 16-byte channel groups need C % 8 == 0
        const int cols = 6 * nw + 2;
        if (C % 8 != 0 || rows_st * cols * kNhwcPix * 2 > kBXBytes) return false;
        p->cols = cols;
        p->rp = p->cp = p->nj = 0;
    } else {
        const int rp = round16i(2 * (6 * nw + 2) + 18);
        const int cp = rows_st * rp + 16;
        if (kBCC * cp > kBXBytes || rp / 16 > 10) return false;
        p->cols = 0;
        p->rp = rp;
        p->cp = cp;
        p->nj = rp / 16;
    }
    p->nruns = nruns;
    p->n_kblk = (K + 63) / 64;
    p->grid = (int64_t)B * nruns * p->n_kblk;
    (void)H;
    (void)W;
    return p->grid < ((int64_t)1 << 31);
}

hipError_t launch_fused_block(const uint16_t* x, const uint16_t* U, uint16_t* y, int B, int C,
                              int K, int Cp, int H, int W, int pad, int nh, int nw, int Ho,
                              int Wo, const FusedBlockPlan& p, hipStream_t s, Epilogue ep) {
    BlockArgs a;
    a.bias = reinterpret_cast<const _Float16*>(ep.bias);
    a.relu = ep.relu;
    a.residual = reinterpret_cast<const _Float16*>(ep.residual);
    const uintptr_t xp = reinterpret_cast<uintptr_t>(x);
    a.x_al = reinterpret_cast<const void*>(xp & ~(uintptr_t)15);
    a.xd = (int)(xp & 15);
    a.x_bytes = (int)dword_ceil(2 * (int64_t)B * C * H * W + a.xd);
    a.U = reinterpret_cast<const _Float16*>(U);
    a.u_bytes = (int)(2 * u_frag_elems(K, Cp));
    a.nkt = (K + 15) / 16;
    a.nkp = (Cp + 31) / 32;
    a.y = reinterpret_cast<_Float16*>(y);
    a.y_bytes = (int)(2 * (int64_t)B * K * Ho * Wo);
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
    a.P = nh * nw;
    a.nruns = p.nruns;
    a.n_kblk = p.n_kblk;
    a.rp = p.rp;
    a.cp = p.cp;
    a.nj = p.nj;
    a.chan2 = (2 * H * W) & 15;
    a.y_pairs = (Wo % 2 == 0 &&
                 ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(ep.residual)) & 3) ==
                     0)
                    ? 1
                    : 0;
    a.cols = p.cols;
    const dim3 grid((unsigned)p.grid), block(kBT);
    a.nwg = (int)grid.x;
    const bool epi = epilogue_needed(ep.bias, ep.relu, ep.residual);
    auto go = [&](auto kernel) { launch(kernel, grid, block, s, a); };
    if (Cp <= 64) {
        auto direct = [&](auto ns, auto nhwc) {
            constexpr int NS = decltype(ns)::value;
            constexpr bool kN = decltype(nhwc)::value;
            epi ? go(fused_block_kernel_direct<NS, kN, true>)
                : go(fused_block_kernel_direct<NS, kN, false>);
        };
        using one = std::integral_constant<int, 1>;
        using two = std::integral_constant<int, 2>;
        if (p.nhwc)
            Cp > 32 ? direct(two(), std::true_type()) : direct(one(), std::true_type());
        else
            Cp > 32 ? direct(two(), std::false_type()) : direct(one(), std::false_type());
        return hipGetLastError();
    }
    if (p.nhwc) {
        if (a.xd != 0) return hipErrorInvalidValue;  // 16-byte loads need an aligned x
        epi ? go(fused_block_kernel<0, true, true>) : go(fused_block_kernel<0, true, false>);
        return hipGetLastError();
    }
    auto go_nj = [&](auto nj) {
        constexpr int NJ = decltype(nj)::value;
        epi ? go(fused_block_kernel<NJ, false, true>) : go(fused_block_kernel<NJ, false, false>);
    };
    switch (p.nj) {
        case 2: go_nj(std::integral_constant<int, 2>()); break;
        case 3: go_nj(std::integral_constant<int, 3>()); break;
        case 4: go_nj(std::integral_constant<int, 4>()); break;
        case 5: go_nj(std::integral_constant<int, 5>()); break;
        case 6: go_nj(std::integral_constant<int, 6>()); break;
        case 7: go_nj(std::integral_constant<int, 7>()); break;
        case 8: go_nj(std::integral_constant<int, 8>()); break;
        case 9: go_nj(std::integral_constant<int, 9>()); break;
        case 10: go_nj(std::integral_constant<int, 10>()); break;
        default: return hipErrorInvalidConfiguration;
    }
    return hipGetLastError();
}

}  // namespace nova
