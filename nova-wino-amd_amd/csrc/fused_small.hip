// Fused NOVA F(6,3) forward for small problems (C, K <= 64 at batch 1 and
// other grids too small to fill the chip; C, K <= 128 when forced): input
// transform, the 64 Winograd-domain products and the output transform in ONE
// launch, spread over many workgroups without any hand-off between them.
//
// The reference's fused kernel (/root/reference/csrc/nova_winograd_fused.hip:
// 283-440, dispatched for every C, K <= 64 layer at :511) gives a workgroup 16
// tiles x 64 output channels, so ResNet-50 conv2_x at batch 1 (100 tiles) runs
// 7 workgroups on 256 CUs. Here a workgroup is T (2) tiles x 16 output
// channels x all 64 positions; every workgroup of a tile group recomputes the
// group's input transform (cheap at C <= 64) instead of sharing it, so there
// are B * ceil(P / T) * ceil(K / 16) independent workgroups (200 at conv2_x
// batch 1), each on the latency chain of one kernel:
//   * the wave's U fragments (fragment-ordered U, 16 output channels x the
//     wave's positions x NKP 32-channel chunks) are requested first and stay
//     in flight during the transform;
//   * input transform, lane-parallel (8 lanes per patch, row pass, LDS
//     transpose, column pass: the chains of input_lp_kernel, so V is
//     bit-identical), NTH / 8 patches per round; V goes to LDS as
//     v_mfma_f32_16x16x32_f16 B operands with T tile slots (lanes of the
//     empty slots read a zero block);
//   * products: each of the NTH / 64 waves multiplies 64 / (NTH / 64)
//     consecutive positions, one MFMA per position and 32-channel chunk, in
//     the operand order of the fused tile-block kernel (so M is bit-identical
//     to that kernel's);
//   * M rounded to fp16 (the reference's rounding point,
//     nova_winograd_fused.hip:405) to LDS, then the output transform,
//     lane-parallel (the chains of output_lp_kernel) with the epilogue.
// Above 64 input channels (NKP = 4) each workgroup reads 256 KB of U: at
// ResNet-50 conv3_x batch 1 the launch takes 10.7 us against 9.9 us for the
// three passes, so the automatic choice keeps it for C, K <= 64.
#include <algorithm>
#include <type_traits>

#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kSmK = 16;                 // output channels per workgroup
constexpr int kSmPitch = 72;             // floats per row of the transpose buffers
constexpr int kSmOob = (int)0x80000000;  // out-of-range byte offset: loads 0, stores dropped

struct SmallArgs {
    const _Float16* x;
    const _Float16* U;  // fragment-ordered U
    _Float16* y;
    int x_bytes, u_bytes, y_bytes;
    int C, K, H, W, pad, nh, nw, Ho, Wo, P;
    int tfirst;    // first tile of each image
    int ntg;       // tile groups per image, from tfirst on
    int nkb;       // 16-channel output blocks
    int nkt, nkp;  // 16-row tiles and 32-channel chunks of the fragment-ordered U
    int y_pairs;   // 1: NCHW rows stored as 4-byte pairs (even Wo, 4-byte aligned y)
    int nwg;       // workgroups in the grid (gridDim.x; a kernel that reads gridDim gets hidden arguments)
    const _Float16* bias;
    int relu;
    const _Float16* residual;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sm_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// V in LDS, halves: [chunk][channel group of 4][tile slot][position slot]
// [half of the chunk][4 channels], position slot (pos % 8) * 8 + pos / 8:
// lane l's B operand (tile l % 16 < T, channels 4*(l/16) .. +3 of both
// 16-channel halves) is 16 contiguous bytes. A transform write instruction
// covers 8 position rows j (positions 8j + s) of 8 channels: with the
// position slots in that order its 8 j's land 4 dwords apart, and the
// (chunk, group, tile) blocks of sm_blk_halves put its two channel groups 32
// banks apart, so the 64 lanes hit 32 banks, one dword each (the earlier
// [position][...] order, 8 positions 544 dwords apart, put them in 8 banks).
constexpr int sm_blk_halves() { return 64 * 8 + 32; }  // T = 2: groups 32 banks apart
template <int T, int NKP>
constexpr int sm_v_halves() {
    return NKP * 4 * T * sm_blk_halves();
}
template <int T, int NKP>
__device__ __forceinline__ int sm_v_base(int pos, int chunk, int cg, int t) {
    return ((chunk * 4 + cg) * T + t) * sm_blk_halves() + ((pos & 7) * 8 + (pos >> 3)) * 8;
}
template <int T, int NKP>
__device__ __forceinline__ int sm_v_index(int pos, int c, int t) {
    const int chunk = c >> 5, cc = c & 31;
    return sm_v_base<T, NKP>(pos, chunk, (cc >> 2) & 3, t) + ((cc >> 4) & 1) * 4 + (cc & 3);
}

// NTH threads (512 or 1024), NKP 32-channel chunks (input channels up to
// 32 * NKP): the transform takes T * 32 * NKP patches of 8 lanes, NTH / 8
// per round; each wave multiplies 64 / (NTH / 64) positions.
template <int T, int NTH, int NKP, bool kNhwc, bool kEpi>
__global__ __launch_bounds__(NTH, 1) void fused_small_kernel(SmallArgs a) {
    constexpr int kWaves = NTH / 64;
    constexpr int kPpw = 64 / kWaves;                          // positions per wave
    constexpr int kCh = 32 * NKP;                              // channel slots
    constexpr int kPatches = T * kCh;                          // patches of the group
    constexpr int kPpr = NTH / 8;                              // patches per round
    static_assert(kPatches % kPpr == 0, "whole rounds");
    constexpr int kRounds = kPatches / kPpr;
    constexpr int kVHalves = sm_v_halves<T, NKP>();            // V of the group's tiles
    constexpr int kTpFloats = kPpr * kSmPitch;                 // one transpose buffer
    __shared__ __align__(16) _Float16 vs[kVHalves + 8];        // + one zero block
    __shared__ __align__(16) float tps[2][kTpFloats];          // double-buffered transposes
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const int L = xcd_remap((int)blockIdx.x, a.nwg);
    const int kb = L % a.nkb;
    const int rest = L / a.nkb;
    const int tg = rest % a.ntg;
    const int b = rest / a.ntg;
    const int k0 = kb * kSmK;
    const int t0 = a.tfirst + tg * T;
    const int ntiles = min(T, a.P - t0);

    const __amdgpu_buffer_rsrc_t xrs = sm_rsrc(a.x, a.x_bytes);
    const __amdgpu_buffer_rsrc_t urs = sm_rsrc(a.U, a.u_bytes);
    const __amdgpu_buffer_rsrc_t yrs = sm_rsrc(a.y, a.y_bytes);

    // ---- 0. this wave's U operands: positions kPpw*w .. +kPpw-1, both chunks ----
    h8 ua[kPpw][NKP];
#pragma unroll
    for (int s = 0; s < kPpw; s++)
#pragma unroll
        for (int j = 0; j < NKP; j++) {
            const int pos = kPpw * wave + s;
            const int off = j < a.nkp ? ((pos * a.nkt + kb) * a.nkp + j) * 1024 : kSmOob;
            ua[s][j] = __builtin_bit_cast(
                h8, __builtin_amdgcn_raw_buffer_load_b128(urs, lane * 16, off, 0));
        }

    // ---- 1. input columns: lane (patch pc = rd * kPpr + tid / 8, column j);
    // patch pc is channel pc % kCh of tile slot pc / kCh ----
    const int j = tid & 7;
    float d[kRounds][8];
#pragma unroll
    for (int rd = 0; rd < kRounds; rd++) {
        const int pc = rd * kPpr + (tid >> 3);
        const int c = pc % kCh, t = pc / kCh;
        const int tl = t0 + min(t, ntiles - 1);
        const int th = tl / a.nw, tw = tl - (tl / a.nw) * a.nw;
        const int w = 6 * tw - a.pad + j;
        const bool ok = t < ntiles && c < a.C && w >= 0 && w < a.W;
        const int cc = ok ? c : 0, ww = ok ? w : 0;
        const int base = kNhwc ? 2 * ((b * a.H * a.W + ww) * a.C + cc)
                               : 2 * ((b * a.C + cc) * a.H * a.W + ww);
        const int rstep = kNhwc ? 2 * a.W * a.C : 2 * a.W;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int h = 6 * th - a.pad + i;
            const int off = (ok && h >= 0 && h < a.H) ? base + h * rstep : kSmOob;
            d[rd][i] = (float)__builtin_bit_cast(
                _Float16, __builtin_amdgcn_raw_buffer_load_b16(xrs, off, 0, 0));
        }
    }
    if (tid < 2) *reinterpret_cast<unsigned long long*>(vs + kVHalves + 4 * tid) = 0ull;

    // ---- 2. input transform, kPpr patches per round (chains of input_lp_kernel) ----
    const float one = opaque_one();
#pragma unroll
    for (int rd = 0; rd < kRounds; rd++) {
        const int pc = rd * kPpr + (tid >> 3);
        const int c = pc % kCh, t = pc / kCh;
        float* tp = tps[rd & 1] + (tid >> 3) * kSmPitch;
#pragma unroll
        for (int r = 0; r < 8; r++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (kBh[i][r] != 0.0f)
                    acc = __builtin_fmaf(mix_coef(kBh[i][r], one), d[rd][i], acc);
            tp[r * 8 + j] = acc;
        }
        __syncthreads();
        float tt[8];
#pragma unroll
        for (int q = 0; q < 8; q++) tt[q] = tp[j * 8 + q];
#pragma unroll
        for (int s2 = 0; s2 < 8; s2++) {
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (kBh[q][s2] != 0.0f) acc = __builtin_fmaf(tt[q], kBh[q][s2], acc);
            vs[sm_v_index<T, NKP>(8 * j + s2, c, t)] = to_f16(acc);
        }
        // the next round writes the other transpose buffer; the one after
        // that reuses this one only after the next round's barrier
    }
    __syncthreads();

    // ---- 3. products: positions kPpw*w .. +kPpw-1 ----
    const int tl = lane & 15, cg = lane >> 4;
    f4 acc[kPpw];
#pragma unroll
    for (int s = 0; s < kPpw; s++) acc[s] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int jc = 0; jc < NKP; jc++)
#pragma unroll
        for (int s = 0; s < kPpw; s++) {
            const int pos = kPpw * wave + s;
            const int vo = tl < T ? sm_v_base<T, NKP>(pos, jc, cg, tl) : kVHalves;
            const h8 vb = *reinterpret_cast<const h8*>(vs + vo);
            acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ua[s][jc], vb, acc[s], 0, 0, 0);
        }

    // ---- 4. M (fp16) to LDS as [kk][tile][position] (transpose buffer 0) ----
    static_assert(kSmK * T * 72 <= 2 * kTpFloats, "M fits in a transpose buffer");
    static_assert(kSmK * T * kSmPitch <= kTpFloats, "output transposes fit in buffer 1");
    _Float16* ms = reinterpret_cast<_Float16*>(tps[0]);  // 16 x T x 72 halves
    __syncthreads();  // every wave is done with the transpose buffers' last round
    if (tl < T) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int kk = 4 * cg + i;
#pragma unroll
            for (int s = 0; s < kPpw; s++)
                ms[(kk * T + tl) * 72 + kPpw * wave + s] = to_f16(acc[s][i]);
        }
    }
    __syncthreads();

    // ---- 5. output transform, lane-parallel (chains of output_lp_kernel) ----
    // pair = (kk, tile); 8 lanes per pair; T * 16 pairs over the 64 groups of 8
    float* tq = tps[1];  // free since the transform (M is in tps[0]); 64 x kSmPitch floats
    const _Float16* res = a.residual;
    const __amdgpu_buffer_rsrc_t rrs = sm_rsrc(res, res ? a.y_bytes : 0);
    for (int pr0 = 0; pr0 < kSmK * T; pr0 += NTH / 8) {
        const int pr = pr0 + (tid >> 3);
        const int kk = pr / T, t = pr - (pr / T) * T;
        const bool live = pr < kSmK * T;
        float m8[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            m8[i] = live ? (float)ms[(kk * T + t) * 72 + 8 * i + j] : 0.0f;
        float* tp = tq + (tid >> 3) * kSmPitch;
#pragma unroll
        for (int r = 0; r < 6; r++) {
            float s0 = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (kAh[r][i] != 0.0f)
                    s0 = __builtin_fmaf(mix_coef(kAh[r][i], one), m8[i], s0);
            tp[r * 8 + j] = s0;
        }
        __syncthreads();
        const int k = k0 + kk;
        const int tile = t0 + t;
        const int th = tile / a.nw, tw = tile - (tile / a.nw) * a.nw;
        const int r = j, oh = 6 * th + r, ow = 6 * tw;
        if (live && t < ntiles && r < 6 && k < a.K && oh < a.Ho) {
            float t8[8];
#pragma unroll
            for (int q = 0; q < 8; q++) t8[q] = tp[r * 8 + q];
            _Float16 out[6];
            const ChannelEpilogue<kEpi> epi(a.bias, k, res ? 0 : a.relu);
#pragma unroll
            for (int s2 = 0; s2 < 6; s2++) {
                float s0 = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; q++)
                    if (kAh[s2][q] != 0.0f) s0 = __builtin_fmaf(t8[q], kAh[s2][q], s0);
                out[s2] = epi(s0);
            }
            if constexpr (kNhwc) {
                const int pix = 2 * (((b * a.Ho + oh) * a.Wo + ow) * a.K + k);
#pragma unroll
                for (int s2 = 0; s2 < 6; s2++)
                    if (ow + s2 < a.Wo) {
                        const int off = pix + 2 * s2 * a.K;
                        _Float16 v = out[s2];
                        if (res)
                            v = add_residual(v,
                                             __builtin_bit_cast(_Float16,
                                                                __builtin_amdgcn_raw_buffer_load_b16(
                                                                    rrs, off, 0, 0)),
                                             a.relu);
                        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs,
                                                              off, 0, 0);
                    }
            } else {
                const int row = 2 * (((b * a.K + k) * a.Ho + oh) * a.Wo + ow);
                if (a.y_pairs) {
#pragma unroll
                    for (int s2 = 0; s2 < 6; s2 += 2)
                        if (ow + s2 < a.Wo) {
                            unsigned v = (unsigned)__builtin_bit_cast(uint16_t, out[s2]) |
                                         ((unsigned)__builtin_bit_cast(uint16_t, out[s2 + 1]) << 16);
                            if (res)
                                v = add_residual2(
                                    v, __builtin_amdgcn_raw_buffer_load_b32(rrs, row + 2 * s2, 0, 0),
                                    a.relu);
                            __builtin_amdgcn_raw_buffer_store_b32(v, yrs, row + 2 * s2, 0, 0);
                        }
                } else {
#pragma unroll
                    for (int s2 = 0; s2 < 6; s2++)
                        if (ow + s2 < a.Wo) {
                            _Float16 v = out[s2];
                            if (res)
                                v = add_residual(
                                    v,
                                    __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(
                                                                     rrs, row + 2 * s2, 0, 0)),
                                    a.relu);
                            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v),
                                                                  yrs, row + 2 * s2, 0, 0);
                        }
                }
            }
        }
        __syncthreads();  // the transpose area is reused by the next round of pairs
    }
}

}  // namespace

bool fused_small_plan(int B, int C, int K, int Cp, int nh, int nw, int cus, FusedSmallPlan* p,
                      int tfirst, int tiles) {
    if (B < 1 || C < 1 || K < 1 || C > 128 || K > 128 || Cp > 128) return false;
    if (tfirst < 0 || tfirst >= nh * nw) return false;
    p->nkp = Cp <= 64 ? 2 : 4;
    if (tiles != 2 && (tiles != 4 || p->nkp != 2)) return false;
    const int P = nh * nw;
    // 2 tiles per workgroup: measured at conv2_x batch 1 (100 tiles), one
    // launch of 1, 2 or 4 tiles per workgroup took 8.3, 7.4 and 9.4 us (the
    // input transform of a workgroup's tiles runs on one CU); 4 on request
    // (up to 64 input channels), for grids that would otherwise hold more
    // than two workgroups per CU
    p->tiles = tiles;
    p->tfirst = tfirst;
    p->ntg = (P - tfirst + p->tiles - 1) / p->tiles;
    p->nkb = (K + kSmK - 1) / kSmK;
    p->grid = (int64_t)B * p->ntg * p->nkb;
    // 1024 threads (one transform round, 4 positions per wave) while every
    // workgroup has a CU of its own (91 KB of LDS: one per CU); 512 threads
    // (54 KB, two per CU) beyond. Measured, us, 1024 vs 512 threads:
    // conv2_x B=1 (200 workgroups) 7.5 vs 7.8, 32@56^2 B=2 (200) 6.9 vs 7.3,
    // 64@28^2 B=4 (208) 7.3 vs 7.8; conv2_x B=2 (400) 13.4 vs 10.4.
    // More than 64 input channels: 1024 threads always (512 would hold
    // 32 x 16 U fragment registers per thread).
    p->threads = (p->grid <= (int64_t)cus || p->nkp == 4) ? 1024 : 512;
    return p->grid < ((int64_t)1 << 31);
}

hipError_t launch_fused_small(const uint16_t* x, const uint16_t* U, uint16_t* y, int B, int C,
                              int K, int Cp, int H, int W, int pad, int nh, int nw, int Ho,
                              int Wo, const FusedSmallPlan& p, hipStream_t s, Epilogue ep,
                              bool nhwc) {
    SmallArgs a;
    a.x = reinterpret_cast<const _Float16*>(x);
    a.U = reinterpret_cast<const _Float16*>(U);
    a.y = reinterpret_cast<_Float16*>(y);
    a.x_bytes = (int)(2 * (int64_t)B * C * H * W);
    a.u_bytes = (int)(2 * u_frag_elems(K, Cp));
    a.y_bytes = (int)(2 * (int64_t)B * K * Ho * Wo);
    a.C = C;
    a.K = K;
    a.H = H;
    a.W = W;
    a.pad = pad;
    a.nh = nh;
    a.nw = nw;
    a.Ho = Ho;
    a.Wo = Wo;
    a.P = nh * nw;
    a.tfirst = p.tfirst;
    a.ntg = p.ntg;
    a.nkb = p.nkb;
    a.nkt = (K + 15) / 16;
    a.nkp = (Cp + 31) / 32;
    a.y_pairs = (Wo % 2 == 0 &&
                 ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(ep.residual)) & 3) ==
                     0)
                    ? 1
                    : 0;
    a.bias = reinterpret_cast<const _Float16*>(ep.bias);
    a.relu = ep.relu;
    a.residual = reinterpret_cast<const _Float16*>(ep.residual);
    const dim3 grid((unsigned)p.grid), block((unsigned)p.threads);
    a.nwg = (int)grid.x;
    if ((p.tiles != 2 && (p.tiles != 4 || p.nkp != 2)) || (p.threads != 512 && p.threads != 1024) ||
        (p.nkp != 2 && p.nkp != 4) || (p.nkp == 4 && p.threads != 1024) || Cp > 32 * p.nkp)
        return hipErrorInvalidConfiguration;
    auto go = [&](auto kernel) { launch(kernel, grid, block, s, a); };
    auto go_th = [&](auto tl, auto nth, auto nkp) {
        constexpr int T = decltype(tl)::value, N = decltype(nth)::value,
                      NK = decltype(nkp)::value;
        if (epilogue_needed(ep.bias, ep.relu, ep.residual))
            nhwc ? go(fused_small_kernel<T, N, NK, true, true>)
                 : go(fused_small_kernel<T, N, NK, false, true>);
        else
            nhwc ? go(fused_small_kernel<T, N, NK, true, false>)
                 : go(fused_small_kernel<T, N, NK, false, false>);
    };
    using two = std::integral_constant<int, 2>;
    using four = std::integral_constant<int, 4>;
    using n1024 = std::integral_constant<int, 1024>;
    using n512 = std::integral_constant<int, 512>;
    if (p.nkp == 4)
        go_th(two(), n1024(), four());
    else if (p.tiles == 4)
        p.threads == 1024 ? go_th(four(), n1024(), two()) : go_th(four(), n512(), two());
    else if (p.threads == 1024)
        go_th(two(), n1024(), two());
    else
        go_th(two(), n512(), two());
    return hipGetLastError();
}

}  // namespace nova
