// Input transform fused into the Winograd-domain products, for GEMV-like
// shapes: few tiles, many channels (batch 1 above 64 channels). Path 7.
//
// The reference runs such layers as three dependent launches
// (/root/reference/csrc/nova_winograd.hip:565-610: input transform, rocBLAS
// batched GEMM, output transform). At batch 1 each of them is a few
// microseconds of latency around very little work, and the transformed input
// V is tiny (64 positions x C channels x a few tiles). This kernel drops the
// first launch: every workgroup builds, in LDS, the slice of V that its own
// products need, from x, and multiplies it straight away; M goes to memory as
// in the three-pass path and the output transform follows as its own launch.
// A hand-off of M to a last-arriving workgroup inside the kernel was measured
// on MI355X and costs more than the launch boundary it would save (agent-scope
// fences ~35 us per call; device-coherent stores and loads ~6-8 us against
// ~6 us for two launches), so two launches remain.
//
// Workgroup = one position row r (positions 8r .. 8r+7) x a group of nt <= 16
// consecutive tiles x KR 16-row output-channel tiles; 8 waves, wave w owns
// position 8r + w. Per workgroup:
//   * each wave requests the U operands of its position (KR row tiles x all
//     32-channel steps, 1 KB blocks of the three-pass GEMM's block copy, one
//     16-byte load per lane) before anything else, so they arrive during the
//     transform;
//   * every thread transforms (channel, tile) patches of the group -- only
//     row r of V = B^T d B, which reads only the input rows i with
//     B[i][r] != 0 (4 or 6 of 8) -- with the shared per-element chains
//     (input_row<r>), and writes the 8 values to LDS as V[position][tile]
//     [channel] (channel pitch Cp + 8 halves: conflict-free 16-byte reads);
//   * after one barrier each wave multiplies its position: B operands are
//     16-byte LDS reads (lane l: tile l % 16, channels 8*(l/16) .. +7 of the
//     step, zero past the group's tiles and past Cp), one
//     v_mfma_f32_16x16x32_f16 per row tile and step, steps in order;
//   * M (fp16) is stored in the product layout M[p][bp][k].
// V is bit-identical to the standalone input transform's (same chains, zero
// for channels C .. Cp-1) and the products use the block GEMM's operand lanes
// and step order, so M -- and y -- equal the three-pass path's bit for bit.
// The row-r-only transform costs 76-92 FMAs per patch (a whole patch: 704),
// but every output-channel group of a row repeats it; the plan keeps that
// work per workgroup near the time its U bytes take to arrive.
#include <algorithm>
#include <type_traits>

#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

constexpr int kIT = 512;  // threads per workgroup: 8 waves, one per position of the row
constexpr int kIOob = (int)0x80000000;
constexpr int kMaxTiles = 16;

struct InGemmArgs {
    const void* x_al;    // NCHW: x rounded down to 16 bytes; NHWC: x
    const _Float16* Uw;  // U blocks (three-pass GEMM lane layout)
    _Float16* M;         // [64][BP][K]
    int x_bytes, xd, u_bytes, m_bytes;
    int C, K, Cp, H, W, pad, nw;
    int P, BP;     // tiles per image, tiles in all
    int nt;        // tiles per workgroup (<= 16)
    int ntg;       // tile groups
    int nkt;       // 16-row output-channel tiles
    int nsteps;    // 32-channel steps (Cp / 32 rounded up)
    int vpitch;    // halves per (position, tile) row of V in LDS: Cp + 8
    int nwg;       // workgroups in the grid (gridDim.x; a kernel that reads gridDim gets hidden arguments)
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// Per-tile part of the patch addresses, one LDS entry per tile of the group:
// the byte offset of the tile's top-left input element in channel 0 (NCHW
// xd + 2*(b*C*H*W + h0*W + w0); channels-last 2*((b*H + h0)*W + w0)*C), and
// which of its 8 input rows (bits 0-7) and columns (bits 8-15) lie inside
// the image.
struct TileOrigin {
    int off;
    unsigned masks;
};

// One (channel, tile) patch of the workgroup, as loaded: the input rows that
// row R of V reads. NCHW: each row is the five dwords from the dword at or
// below its start (shifted into place by 0 or 2 bytes later); channels-last:
// the row's 8 pixels, column pairs packed.
struct PatchRows {
    unsigned w[8][5];
    unsigned odd, neg, cmask;
    int c, tl, off;
    bool valid;
};

template <int R, bool kNhwc>
__device__ __forceinline__ void load_patch(const InGemmArgs& a, const TileOrigin* to,
                                           __amdgpu_buffer_rsrc_t xrs, int c, int tl,
                                           PatchRows& pr) {
    const TileOrigin o = to[tl];
    const unsigned rows = c < a.C ? o.masks & 0xffu : 0u;  // channels past C read zero
    pr.c = c;
    pr.tl = tl;
    pr.odd = 0;
    pr.neg = 0;
    pr.cmask = o.masks >> 8;
    if constexpr (kNhwc) {
        const int ro = o.off + 2 * c;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (!input_row_uses(R, i)) continue;
            const int rio = ro + 2 * i * a.W * a.C;
            const bool rok = (rows >> i) & 1u;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                unsigned v = 0;
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const bool ok = rok && ((pr.cmask >> (2 * q + u)) & 1u);
                    v |= (unsigned)__builtin_amdgcn_raw_buffer_load_b16(
                             xrs, ok ? rio + 2 * (2 * q + u) * a.C : kIOob, 0, 0)
                         << (16 * u);
                }
                pr.w[i][q] = v;
            }
        }
    } else {
        const int oc = o.off + 2 * c * a.H * a.W;
        pr.off = oc;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (!input_row_uses(R, i)) continue;
            const int off = oc + 2 * i * a.W;
            const bool ok = (rows >> i) & 1u;
            pr.odd |= (unsigned)(off & 2) << i;
            pr.neg |= (ok && off < 0) ? (1u << i) : 0u;
            // rows outside the image (and channels past C) read zeros through
            // an out-of-range offset; a row starting before x_al from 0
            const int A = !ok ? kIOob : (off < 0 ? 0 : (off & ~3));
            const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, A, 0, 0);
#pragma unroll
            for (int q = 0; q < 4; q++) pr.w[i][q] = v[q];
            pr.w[i][4] = __builtin_amdgcn_raw_buffer_load_b32(xrs, A + 16, 0, 0);
        }
    }
}

// Row R of V for one loaded patch, into vs[(s * nt + tl) * vpitch + c].
// Columns outside the image are zeroed after the first pass: every term of
// t[j] is B[i][R] * d[i][j], all zero for such a column, and the chain from
// +0 gives +0 -- so t[j] = +0 is what masking the inputs would give, with 8
// selects instead of masks on every input word.
template <int R, bool kNhwc>
__device__ __forceinline__ void transform_patch(const InGemmArgs& a, PatchRows& pr,
                                                _Float16* vs, int nt) {
    unsigned d4[8][4];  // row i: columns 2q, 2q+1 packed
    if constexpr (kNhwc) {
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) d4[i][q] = pr.w[i][q];
    } else {
        // a row that starts before x_al (the first row of channel 0 of image
        // 0 with left padding and a 16-byte aligned x; at most 2 dwords
        // before it, as the plan admits pads up to 2) was loaded from offset
        // 0: move its dwords up by the missing ones (the zeros land in masked
        // columns)
        if (pr.neg != 0) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (!input_row_uses(R, i) || !((pr.neg >> i) & 1u)) continue;
                const int off = pr.off + 2 * i * a.W;
                const bool two = off < -4;  // off >= -8: one or two dwords
#pragma unroll
                for (int q = 4; q >= 0; q--) {
                    const unsigned m1 = q >= 1 ? pr.w[i][q - 1] : 0u;
                    const unsigned m2 = q >= 2 ? pr.w[i][q - 2] : 0u;
                    pr.w[i][q] = two ? m2 : m1;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (!input_row_uses(R, i)) continue;
            const unsigned sb = (pr.odd >> i) & 2u;
#pragma unroll
            for (int q = 0; q < 4; q++)
                d4[i][q] = __builtin_amdgcn_alignbyte(pr.w[i][q + 1], pr.w[i][q], sb);
        }
    }
    float out[8];
    input_row_masked<R>(
        [&](int i, int j) {
            const unsigned v = d4[i][j >> 1];
            const unsigned short bits = (unsigned short)((j & 1) ? (v >> 16) : (v & 0xffffu));
            return (float)__builtin_bit_cast(_Float16, bits);
        },
        kNhwc ? 0xffu : pr.cmask, out);
    _Float16* dst = vs + pr.tl * a.vpitch + pr.c;
#pragma unroll
    for (int s = 0; s < 8; s++) dst[s * nt * a.vpitch] = to_f16(out[s]);
}

// Row R of V for the patches (channel c < Cp, tile t0 + tl, tl < nt) of this
// workgroup, into LDS. Channels C .. Cp-1 and rows/columns outside the image
// read zero (out-of-range offsets, column masks), so their V is +0 as the
// standalone transform writes it. NCHW: tiles run fastest over the lanes
// (neighbouring tiles share input lines); each needed input row is a 16-byte
// and a 4-byte load from the dword at or below its start, shifted by 0 or 2
// bytes. Channels-last: channels run fastest (a 2-byte load per pixel covers
// 128 consecutive bytes per wave). The input rows of the thread's first kPre
// patches are requested before issue_u() requests the U operands: vector
// loads return in order, so patches loaded after U would wait for all of U.
template <int R, bool kNhwc, int kPre, typename IssueU>
__device__ __forceinline__ void v_row_phase(const InGemmArgs& a, const TileOrigin* to,
                                            _Float16* vs, int nt, IssueU issue_u) {
    const int tid = threadIdx.x;
    const int total = a.Cp * nt;
    const __amdgpu_buffer_rsrc_t xrs = rsrc(a.x_al, a.x_bytes);
    // e = tid + k * kIT walks (c, tl): NCHW tl = e % nt, c = e / nt;
    // channels-last c = e % Cp, tl = e / Cp -- advanced incrementally
    const int inner = kNhwc ? a.Cp : nt;
    const int dq = kIT / inner, dr = kIT - (kIT / inner) * inner;
    int q0 = tid / inner, r0 = tid - (tid / inner) * inner;
    auto advance = [&]() {
        r0 += dr;
        q0 += dq;
        if (r0 >= inner) {
            r0 -= inner;
            q0 += 1;
        }
    };
    PatchRows pr[kPre];
#pragma unroll
    for (int k = 0; k < kPre; k++) {
        pr[k].valid = tid + k * kIT < total;
        if (pr[k].valid) load_patch<R, kNhwc>(a, to, xrs, kNhwc ? r0 : q0, kNhwc ? q0 : r0, pr[k]);
        advance();
    }
    issue_u();
#pragma unroll
    for (int k = 0; k < kPre; k++)
        if (pr[k].valid) transform_patch<R, kNhwc>(a, pr[k], vs, nt);
    for (int e = tid + kPre * kIT; e < total; e += kIT) {
        PatchRows p1;
        load_patch<R, kNhwc>(a, to, xrs, kNhwc ? r0 : q0, kNhwc ? q0 : r0, p1);
        transform_patch<R, kNhwc>(a, p1, vs, nt);
        advance();
    }
}

// KR: 16-row output-channel tiles per workgroup; NSM: the most 32-channel
// steps this instantiation holds (nsteps <= NSM).
template <int KR, int NSM, bool kNhwc, int kPol>
__global__ __launch_bounds__(kIT, 1) void in_gemm_kernel(InGemmArgs a) {
    __shared__ __align__(16) _Float16 vs[8 * kMaxTiles * (NSM * 32 + 8)];
    __shared__ TileOrigin to[kMaxTiles];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // XCD-aware order: the tile groups of one (row, channel group) -- the
    // workgroups that read the same U blocks -- are neighbours
    const int L = xcd_remap(blockIdx.x, a.nwg);
    const int tg = L % a.ntg;
    const int rest = L / a.ntg;
    const int r = rest % 8;
    const int kg = rest / 8;
    const int t0 = tg * a.nt;
    const int nt = min(a.nt, a.BP - t0);
    const int p = 8 * r + wave;

    if (tid < nt) {
        const int bp = t0 + tid;
        const int b = bp / a.P;
        const int tr = bp - b * a.P;
        const int th = tr / a.nw, tw = tr - (tr / a.nw) * a.nw;
        const int h0 = 6 * th - a.pad, w0 = 6 * tw - a.pad;
        unsigned m = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            m |= (h0 + i >= 0 && h0 + i < a.H) ? (1u << i) : 0u;
            m |= (w0 + i >= 0 && w0 + i < a.W) ? (1u << (8 + i)) : 0u;
        }
        TileOrigin o;
        o.off = kNhwc ? 2 * ((b * a.H + h0) * a.W + w0) * a.C
                      : a.xd + 2 * (b * a.C * a.H * a.W + h0 * a.W + w0);
        o.masks = m;
        to[tid] = o;
    }
    __syncthreads();

    // ---- U operands of this wave's position: KR row tiles x all steps,
    // requested once the first patches' input rows are ----
    const __amdgpu_buffer_rsrc_t urs = rsrc(a.Uw, a.u_bytes);
    h8 ua[KR][NSM];
    auto issue_u = [&]() {
#pragma unroll
        for (int kt = 0; kt < KR; kt++) {
            const int ktg = kg * KR + kt;
            const int base =
                ktg < a.nkt ? (p * a.nkt + ktg) * a.nsteps * 1024 + lane * 16 : kIOob;
#pragma unroll
            for (int j = 0; j < NSM; j++)
                if (j < a.nsteps)
                    ua[kt][j] = __builtin_bit_cast(
                        h8, __builtin_amdgcn_raw_buffer_load_b128(urs, base, j * 1024, 0));
        }
    };

    // ---- row r of V for the group's patches, into LDS ----
    // patches whose input rows go ahead of U: as many as the registers hold
    // beside the U operands (4 with at most 16 of them, else 2)
    constexpr int kPre = KR * NSM <= 16 ? 4 : 2;
    switch (r) {
        case 0: v_row_phase<0, kNhwc, kPre>(a, to, vs, nt, issue_u); break;
        case 1: v_row_phase<1, kNhwc, kPre>(a, to, vs, nt, issue_u); break;
        case 2: v_row_phase<2, kNhwc, kPre>(a, to, vs, nt, issue_u); break;
        case 3: v_row_phase<3, kNhwc, kPre>(a, to, vs, nt, issue_u); break;
        case 4: v_row_phase<4, kNhwc, kPre>(a, to, vs, nt, issue_u); break;
        case 5: v_row_phase<5, kNhwc, kPre>(a, to, vs, nt, issue_u); break;
        case 6: v_row_phase<6, kNhwc, kPre>(a, to, vs, nt, issue_u); break;
        default: v_row_phase<7, kNhwc, kPre>(a, to, vs, nt, issue_u); break;
    }
    __syncthreads();

    // ---- products of position p, steps in order ----
    const int slot = lane & 15, g = lane >> 4;
    const bool sok = slot < nt;
    const _Float16* vrow = vs + (wave * nt + (sok ? slot : 0)) * a.vpitch + 8 * g;
    f4 acc[KR];
#pragma unroll
    for (int kt = 0; kt < KR; kt++) acc[kt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NSM; j++) {
        if (j < a.nsteps) {
            h8 bv = *reinterpret_cast<const h8*>(vrow + 32 * j);
            if (!sok || 32 * j + 8 * g >= a.Cp) bv = h8{};  // Cp % 8 == 0: whole octets
#pragma unroll
            for (int kt = 0; kt < KR; kt++)
                acc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ua[kt][j], bv, acc[kt], 0, 0, 0);
        }
    }

    // ---- M (fp16), product layout: lane holds k = 16*kt + 4g + i, tile slot ----
    const __amdgpu_buffer_rsrc_t mrs = rsrc(a.M, a.m_bytes);
    const int mu = 2 * p * a.BP * a.K;  // uniform
    const int bp = t0 + slot;
    const bool vec_store = (a.K & 3) == 0;
#pragma unroll
    for (int kt = 0; kt < KR; kt++) {
        const int k = (kg * KR + kt) * 16 + 4 * g;
        const int off = (sok && k < a.K) ? 2 * (bp * a.K + k) : kIOob;
        if (vec_store) {
            h4 v = {(_Float16)acc[kt][0], (_Float16)acc[kt][1], (_Float16)acc[kt][2],
                    (_Float16)acc[kt][3]};
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, v), mrs, off, mu, kPol);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++)
                __builtin_amdgcn_raw_buffer_store_b16(
                    __builtin_bit_cast(uint16_t, (_Float16)acc[kt][i]), mrs,
                    (sok && k + i < a.K) ? 2 * (bp * a.K + k + i) : kIOob, mu, kPol);
        }
    }
}

// Estimated time of one launch shape, us, fitted to MI355X launches (ResNet-50
// conv3_x at batch 1, every tile-group width and 1 or 2 row tiles): rounds
// of workgroups over the CUs, each ~3.9 us plus 3.5 ns per (channel, tile)
// patch -- the workgroup's input-row loads, 16- and 4-byte pieces of rows
// one channel plane apart, bound the transform rather than its VALU work --
// plus its U bytes at ~200 GB/s per CU. Measured (event-timed launch, us,
// tiles per workgroup x row tiles): 4 x 2 5.75 (224 workgroups), 5 x 2 6.14
// (160), 7 x 1 7.06 (256), 9 x 1 7.94 (192), 13 x 1 9.83 (128); two rounds:
// 4 x 1 8.0 (448), 3 x 2 8.07 (288).
double in_gemm_cost(int Cp, int nkt, int nsteps, int BP, int nt, int kr, int cus) {
    const int ntg = (BP + nt - 1) / nt;
    const int nkg = (nkt + kr - 1) / kr;
    const int64_t grid = (int64_t)8 * ntg * nkg;
    const double u_kb = 8.0 * kr * nsteps;  // 1 KB per (position, row tile, step)
    const double rounds = (double)((grid + cus - 1) / cus);
    return rounds * (3.9 + 0.0035 * Cp * nt + u_kb / 200.0);
}

}  // namespace

bool in_gemm_plan(int B, int C, int K, int Cp, int nh, int nw, int pad, int cus,
                  InGemmPlan* p) {
    const int64_t BP = (int64_t)B * nh * nw;
    const int nsteps = (Cp + 31) / 32;
    const int nkt = (K + 15) / 16;
    // pads up to 4: a row starts at most 2 dwords before x's 16-byte granule
    if (BP < 1 || BP > 4 * kMaxTiles || nsteps > 16 || C < 1 || K < 1 || cus < 1 || pad < 0 ||
        pad > 4)
        return false;
    // 32-bit offsets: U blocks, M and x
    if (2 * u_frag_elems(K, Cp) >= ((int64_t)1 << 31) ||
        2 * (int64_t)64 * BP * K >= ((int64_t)1 << 31))
        return false;
    double best = -1.0;
    for (int ntg = (int)((BP + kMaxTiles - 1) / kMaxTiles); ntg <= BP; ntg++) {
        const int nt = (int)((BP + ntg - 1) / ntg);
        if ((BP + nt - 1) / nt != ntg) continue;  // the same split as a smaller ntg
        for (int kr = 1; kr <= 2; kr++) {
            const double c = in_gemm_cost(Cp, nkt, nsteps, (int)BP, nt, kr, cus);
            const int64_t g = (int64_t)8 * ntg * ((nkt + kr - 1) / kr);
            if (best < 0.0 || c < best - 1e-9 ||
                (c < best + 1e-9 && g < (int64_t)8 * p->ntg * ((nkt + p->kr - 1) / p->kr))) {
                best = c;
                p->nt = nt;
                p->ntg = ntg;
                p->kr = kr;
            }
        }
    }
    p->nsteps = nsteps;
    p->nsm = nsteps <= 4 ? 4 : nsteps <= 8 ? 8 : 16;
    p->nkg = (nkt + p->kr - 1) / p->kr;
    p->grid = (int64_t)8 * p->ntg * p->nkg;
    return true;
}

const char* in_gemm_name(const InGemmPlan& p) {
    static const char* names[2][3] = {
        {"in_gemm_kernel<1, 4>", "in_gemm_kernel<1, 8>", "in_gemm_kernel<1, 16>"},
        {"in_gemm_kernel<2, 4>", "in_gemm_kernel<2, 8>", "in_gemm_kernel<2, 16>"}};
    return names[p.kr - 1][p.nsm == 4 ? 0 : p.nsm == 8 ? 1 : 2];
}

hipError_t launch_in_gemm(const uint16_t* x, const uint16_t* Uw, uint16_t* M, int B, int C,
                          int K, int Cp, int H, int W, int pad, int nh, int nw,
                          const InGemmPlan& p, hipStream_t s, bool nhwc) {
    const int64_t BP = (int64_t)B * nh * nw;
    if (p.nt < 1 || p.nt > kMaxTiles || p.kr < 1 || p.kr > 2 || Cp % 8 != 0 || pad < 0 || pad > 4 ||
        (p.nsm != 4 && p.nsm != 8 && p.nsm != 16) || p.nsteps > p.nsm ||
        p.nsteps != (Cp + 31) / 32 || (int64_t)p.ntg * p.nt < BP ||
        (int64_t)(p.ntg - 1) * p.nt >= BP || p.nkg * p.kr < (K + 15) / 16)
        return hipErrorInvalidValue;
    const uintptr_t xp = reinterpret_cast<uintptr_t>(x);
    const int xd = nhwc ? 0 : (int)(xp & 15);
    const int64_t x_bytes = dword_ceil(2 * (int64_t)B * C * H * W + xd);
    const int64_t u_bytes = 2 * u_frag_elems(K, Cp);
    const int64_t m_bytes = 2 * (int64_t)64 * BP * K;
    if (x_bytes >= ((int64_t)1 << 31) - 64 || u_bytes >= ((int64_t)1 << 31) ||
        m_bytes >= ((int64_t)1 << 31) || p.grid >= ((int64_t)1 << 31))
        return hipErrorInvalidValue;
    InGemmArgs a{};
    a.x_al = reinterpret_cast<const void*>(xp - (uintptr_t)xd);
    a.Uw = reinterpret_cast<const _Float16*>(Uw);
    a.M = reinterpret_cast<_Float16*>(M);
    a.x_bytes = (int)x_bytes;
    a.xd = xd;
    a.u_bytes = (int)u_bytes;
    a.m_bytes = (int)m_bytes;
    a.C = C;
    a.K = K;
    a.Cp = Cp;
    a.H = H;
    a.W = W;
    a.pad = pad;
    a.nw = nw;
    a.P = nh * nw;
    a.BP = (int)BP;
    a.nt = p.nt;
    a.ntg = p.ntg;
    a.nkt = (K + 15) / 16;
    a.nsteps = p.nsteps;
    a.vpitch = Cp + 8;
    const dim3 grid((unsigned)p.grid), block(kIT);
    a.nwg = (int)grid.x;
    auto go = [&](auto kernel) { launch(kernel, grid, block, s, a); };
    // M (8-byte pieces of lines) written through the L2 while it is small
    // (kWTSmallBytes; conv3_x batch 1 8.81 -> 8.66 us in a graph)
    const bool wt = m_bytes <= kWTSmallBytes;
    auto pick = [&](auto nh_, auto pol_) {
        constexpr bool kN = decltype(nh_)::value;
        constexpr int P = decltype(pol_)::value;
        if (p.kr == 1) {
            if (p.nsm == 4) go(in_gemm_kernel<1, 4, kN, P>);
            else if (p.nsm == 8) go(in_gemm_kernel<1, 8, kN, P>);
            else go(in_gemm_kernel<1, 16, kN, P>);
        } else {
            if (p.nsm == 4) go(in_gemm_kernel<2, 4, kN, P>);
            else if (p.nsm == 8) go(in_gemm_kernel<2, 8, kN, P>);
            else go(in_gemm_kernel<2, 16, kN, P>);
        }
    };
    auto by_policy = [&](auto nh_) {
        if (wt)
            pick(nh_, std::integral_constant<int, kWT>());
        else
            pick(nh_, std::integral_constant<int, 0>());
    };
    if (nhwc)
        by_policy(std::true_type());
    else
        by_policy(std::false_type());
    return hipGetLastError();
}

}  // namespace nova
