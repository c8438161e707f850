// Two-pass forward, second pass: the 64 Winograd-domain products and the
// output transform in one launch (path 6). The first pass is the input
// transform of the three-pass path, unchanged (V[p][bp][Cp] in HBM); M never
// leaves the chip.
//
// Workgroup = 16 consecutive tiles (bp, across images) x 32 output channels x
// all 64 positions; 512 threads, wave w owns position row w (8 positions) and
// keeps 8 x 2 fp32 16x16 accumulators (64 registers) for the whole channel
// loop. Grids that would leave CUs idle at 32 channels (at most one
// 16-channel workgroup per CU) take 16 output channels per workgroup and run
// two workgroups per CU instead (8 x 1 accumulators, one step of operands in
// flight per wave, the other workgroup's waves covering its loads). Per 32-channel step a lane loads its operands with the three-pass
// GEMM's lane layout -- A = U_p rows (16 k x 32 c), B = V_p rows (32 c x 16
// bp), lane l holding row l % 16 and channels 8*(l/16) .. +7 -- from copies
// in which that is contiguous (U: launch_u_wfrag blocks; V: the input
// transform's two-pass layout, the same 1 KB blocks per 16 tiles and 32
// channels), so every operand load is one contiguous 1 KB block per wave (in
// the product layouts a load gathers 16 rows of 64 bytes: 2x slower here);
// the steps run in channel order, so M is the three-pass GEMM's, bit for
// bit. After the loop M is rounded to fp16 into
// LDS ([k][tile][position], or [tile][k][position] for channels-last output)
// and every thread runs the output transform + epilogue of one (k, tile) pair
// (the chains of output_transform_kernel), so y equals the three-pass y.
//
// Each workgroup reads 2*64*32*Cp bytes of U and 2*64*16*Cp of V from L2
// (768 KB at Cp = 128): the kernel pays where C is moderate, the grid fills
// the CUs in one round, and the three-pass M round trip (written by the GEMM,
// read by the output transform) is large.
#include <type_traits>

#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kGoT = 16;        // tiles per workgroup
constexpr int kGoThreads = 512;  // 8 waves: one per position row
constexpr int kGoPitch = 72;    // halves per (k, tile) row of M: 64 positions + 8
constexpr int kGoOob = (int)0x80000000;
// Output channels per workgroup: KB 16-row tiles of U (KB = 2: 32 channels,
// one workgroup per CU; KB = 1: 16, two per CU)
template <int KB>
struct GoGeom {
    static constexpr int kK = 16 * KB;
    static constexpr int kTileP = kK * kGoPitch + 8;  // channels-last: halves per tile
    static constexpr int kMsHalves = kGoT * kTileP;   // >= kK * kGoT * kGoPitch
};

struct GoArgs {
    const _Float16* U;  // U blocks [64][nkt][Cp/32][lane][8]
    const _Float16* V;  // V blocks [64][nbb][Cp/32][lane][8]
    _Float16* y;
    int u_bytes, v_bytes, y_bytes;
    int K, Cp, BP, P, nw, Ho, Wo;
    int nkb;      // output-channel blocks (16 * KB channels each)
    int nwg;      // workgroups in the grid (gridDim.x, passed to keep hidden arguments off)
    int nkt;      // 16-row tiles of U
    int nbb;      // 16-tile blocks of V
    int y_pairs;  // 1: NCHW rows stored as 4-byte pairs (even Wo, 4-byte aligned y)
    const _Float16* bias;
    int relu;
    const _Float16* residual;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t go_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// KB = 2: one workgroup per CU, two waves per SIMD, up to 256 registers per
// lane, room for two steps of operands beside the accumulators (double
// buffer). KB = 1: two workgroups per CU, four waves per SIMD, at most 128
// registers, one step of operands (measured on MI355X, graph of ten forwards,
// us, one vs two workgroups per CU at 16 channels: 64@56^2 B=4 13.23 vs
// 12.80, B=8 14.25 vs 13.76; 128@28^2 B=8 16.19 vs 15.95; 96@28^2 B=8 13.76
// vs 13.90).
template <int KB, bool kNhwc, bool kEpi>
__global__ __launch_bounds__(kGoThreads) __attribute__((amdgpu_waves_per_eu(6 - 2 * KB, 6 - 2 * KB)))
void gemm_out_kernel(GoArgs a) {
    static_assert(KB == 1 || KB == 2, "16 or 32 output channels per workgroup");
    using G = GoGeom<KB>;
    __shared__ __align__(16) _Float16 ms[G::kMsHalves];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // = position row

    // output block fastest: the workgroups of one tile block read its V in one L2
    const int L = xcd_remap((int)blockIdx.x, a.nwg);
    const int kbl = L % a.nkb;
    const int bp0 = (L / a.nkb) * kGoT;
    const int k0 = kbl * G::kK;
    const int r16 = lane & 15, g = lane >> 4;

    const __amdgpu_buffer_rsrc_t urs = go_rsrc(a.U, a.u_bytes);
    const __amdgpu_buffer_rsrc_t vrs = go_rsrc(a.V, a.v_bytes);
    const __amdgpu_buffer_rsrc_t yrs = go_rsrc(a.y, a.y_bytes);

    // ---- products: positions 8*wave .. +7, 32-channel steps in order ----
    // (rows past K and channels past Cp are zero in the U copy; V slots of
    // channels past Cp and tiles past BP are never written, so those lanes
    // read zeros through out-of-range offsets)
    const int kt0 = k0 >> 4;
    const bool bok = bp0 + r16 < a.BP;
    f4 acc[8][KB];
#pragma unroll
    for (int s = 0; s < 8; s++)
#pragma unroll
        for (int kb = 0; kb < KB; kb++) acc[s][kb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // operands of one 32-channel step: 8 * (KB + 1) 16-byte loads per lane,
    // all issued before the step's MFMAs; two steps in flight (double buffer)
    struct Ops {
        h8 u[8][KB];
        h8 v[8];
    };
    const int nsteps = (a.Cp + 31) / 32;
    auto load = [&](int j, Ops& o) {
        const bool cok = j < nsteps && 32 * j + 8 * g < a.Cp;  // Cp % 8 == 0: whole groups
        const int lo = cok ? lane * 16 : kGoOob;
        const int vo = cok && bok ? lo : kGoOob;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int p = 8 * wave + s;
#pragma unroll
            for (int kb = 0; kb < KB; kb++)
                o.u[s][kb] = __builtin_bit_cast(
                    h8, __builtin_amdgcn_raw_buffer_load_b128(
                            urs, kt0 + kb < a.nkt ? lo : kGoOob,
                            ((p * a.nkt + kt0 + kb) * nsteps + j) * 1024, 0));
            o.v[s] = __builtin_bit_cast(
                h8, __builtin_amdgcn_raw_buffer_load_b128(
                        vrs, vo, ((p * a.nbb + (bp0 >> 4)) * nsteps + j) * 1024, 0));
        }
    };
    auto multiply = [&](const Ops& o) {
#pragma unroll
        for (int s = 0; s < 8; s++)
#pragma unroll
            for (int kb = 0; kb < KB; kb++)
                acc[s][kb] =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(o.u[s][kb], o.v[s], acc[s][kb], 0, 0, 0);
    };
    if constexpr (KB == 2) {
        Ops o0, o1;
        load(0, o0);
        for (int j = 0; j < nsteps; j += 2) {
            load(j + 1, o1);  // past the last step: zero loads (out-of-range offsets)
            multiply(o0);
            if (j + 1 >= nsteps) break;
            load(j + 2, o0);
            multiply(o1);
        }
    } else {
        for (int j = 0; j < nsteps; j++) {
            Ops o;
            load(j, o);
            multiply(o);
        }
    }

    // ---- M (fp16) to LDS, one 16-byte write per (k, tile) row and lane ----
    // lane (g, r16) holds M[k = 16 kb + 4 g + i][tile r16] for its 8 positions
#pragma unroll
    for (int kb = 0; kb < KB; kb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int kk = 16 * kb + 4 * g + i;
            h8 v;
#pragma unroll
            for (int s = 0; s < 8; s++) v[s] = to_f16(acc[s][kb][i]);
            const int mo =
                kNhwc ? r16 * G::kTileP + kk * kGoPitch : (kk * kGoT + r16) * kGoPitch;
            *reinterpret_cast<h8*>(ms + mo + 8 * wave) = v;
        }
    __syncthreads();

    // ---- output transform: one (k, tile) pair per thread ----
    // NCHW: lanes over tiles (adjacent tiles of a row write adjacent 12-byte
    // row pieces); channels-last: lanes over channels (32 or 64 contiguous
    // bytes per pixel). With KB = 1 the 256 pairs take half the threads.
    const int kk = kNhwc ? (tid & (G::kK - 1)) : (tid >> 4);
    const int t = kNhwc ? (tid / G::kK) : (tid & (kGoT - 1));
    const int k = k0 + kk, bp = bp0 + t;
    if (kk >= G::kK || t >= kGoT || k >= a.K || bp >= a.BP) return;  // no barrier follows
    const int mo = kNhwc ? t * G::kTileP + kk * kGoPitch : (kk * kGoT + t) * kGoPitch;
    h8 mv[8];
#pragma unroll
    for (int ii = 0; ii < 8; ii++) mv[ii] = *reinterpret_cast<const h8*>(ms + mo + 8 * ii);
    float out[6][6];
    output_tile([&](int ii, int jj) { return (float)mv[ii][jj]; }, out);
    const int b = bp / a.P, tl = bp - (bp / a.P) * a.P;
    const int oh = (tl / a.nw) * 6, ow = (tl - (tl / a.nw) * a.nw) * 6;
    const _Float16* res = a.residual;
    const __amdgpu_buffer_rsrc_t rrs = go_rsrc(res, res ? a.y_bytes : 0);
    const ChannelEpilogue<kEpi> epi(a.bias, k, res ? 0 : a.relu);
    if constexpr (kNhwc) {
#pragma unroll
        for (int r = 0; r < 6; r++) {
            if (oh + r >= a.Ho) break;
#pragma unroll
            for (int s = 0; s < 6; s++)
                if (ow + s < a.Wo) {
                    const int off = 2 * (((b * a.Ho + oh + r) * a.Wo + ow + s) * a.K + k);
                    _Float16 v = epi(out[r][s]);
                    if (res)
                        v = add_residual(v,
                                         __builtin_bit_cast(_Float16,
                                                            __builtin_amdgcn_raw_buffer_load_b16(
                                                                rrs, off, 0, 0)),
                                         a.relu);
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs,
                                                          off, 0, 0);
                }
        }
    } else {
        const int ybase = 2 * ((b * a.K + k) * a.Ho * a.Wo + ow);
#pragma unroll
        for (int r = 0; r < 6; r++) {
            if (oh + r >= a.Ho) break;
            const int row = ybase + 2 * (oh + r) * a.Wo;
            if (a.y_pairs) {
#pragma unroll
                for (int s = 0; s < 6; s += 2)
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

}  // namespace

int64_t gemm_out_grid(int K, int BP, int kb) {
    return (int64_t)((BP + kGoT - 1) / kGoT) * ((K + 16 * kb - 1) / (16 * kb));
}

int gemm_out_kb(int K, int BP, int cus) { return gemm_out_grid(K, BP, 1) <= cus ? 1 : 2; }

int64_t gemm_out_v_elems(int Cp, int64_t BP) {
    return (int64_t)64 * ((BP + kGoT - 1) / kGoT) * ((Cp + 31) / 32) * 512;
}

hipError_t launch_gemm_out(const uint16_t* Uw, const uint16_t* V, uint16_t* y, int B, int K,
                           int Cp, int nh, int nw, int Ho, int Wo, hipStream_t s, Epilogue ep,
                           bool nhwc, int kb) {
    if (kb != 1 && kb != 2) return hipErrorInvalidValue;
    const int64_t BP = (int64_t)B * nh * nw;
    const int64_t u_bytes = 2 * u_frag_elems(K, Cp);
    const int64_t v_bytes = 2 * gemm_out_v_elems(Cp, BP);
    const int64_t y_bytes = 2 * (int64_t)B * K * Ho * Wo;
    const int64_t grid = gemm_out_grid(K, (int)BP, kb);
    if (Cp % 8 != 0 || u_bytes >= ((int64_t)1 << 31) || v_bytes >= ((int64_t)1 << 31) ||
        y_bytes >= ((int64_t)1 << 31) || grid >= ((int64_t)1 << 31))
        return hipErrorInvalidValue;
    if (B == 0) return hipSuccess;
    GoArgs a;
    a.U = reinterpret_cast<const _Float16*>(Uw);
    a.V = reinterpret_cast<const _Float16*>(V);
    a.y = reinterpret_cast<_Float16*>(y);
    a.u_bytes = (int)u_bytes;
    a.v_bytes = (int)v_bytes;
    a.y_bytes = (int)y_bytes;
    a.K = K;
    a.Cp = Cp;
    a.BP = (int)BP;
    a.P = nh * nw;
    a.nw = nw;
    a.Ho = Ho;
    a.Wo = Wo;
    a.nkb = (K + 16 * kb - 1) / (16 * kb);
    a.nkt = (K + 15) / 16;
    a.nbb = (int)((BP + kGoT - 1) / kGoT);
    a.y_pairs = (Wo % 2 == 0 &&
                 ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(ep.residual)) & 3) ==
                     0)
                    ? 1
                    : 0;
    a.bias = reinterpret_cast<const _Float16*>(ep.bias);
    a.relu = ep.relu;
    a.residual = reinterpret_cast<const _Float16*>(ep.residual);
    const dim3 g((unsigned)grid), blk(kGoThreads);
    a.nwg = (int)g.x;
    auto go = [&](auto kernel) { launch(kernel, g, blk, s, a); };
    auto pick = [&](auto kbc) {
        constexpr int KB = decltype(kbc)::value;
        if (epilogue_needed(ep.bias, ep.relu, ep.residual))
            nhwc ? go(gemm_out_kernel<KB, true, true>) : go(gemm_out_kernel<KB, false, true>);
        else
            nhwc ? go(gemm_out_kernel<KB, true, false>) : go(gemm_out_kernel<KB, false, false>);
    };
    if (kb == 2)
        pick(std::integral_constant<int, 2>());
    else
        pick(std::integral_constant<int, 1>());
    return hipGetLastError();
}

}  // namespace nova
