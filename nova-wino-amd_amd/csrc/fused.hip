// Fused NOVA F(6,3) kernel for gfx950: input transform -> 64 Winograd-domain
// MFMA products -> output transform in one launch, with V and M kept on chip.
//
// Replaces the reference's fused kernel
// (/root/reference/csrc/nova_winograd_fused.hip:283-440; 1024 threads, 16
// tiles, 16x16x16 MFMA, K super-chunks of 64, input transform recomputed per
// K chunk) with a gfx950 design:
//   * workgroup = 512 threads (8 waves) = 16 tiles x 64 output channels; the
//     grid is (tile groups) x (output-channel blocks), so B=1 layers still
//     spread over many CUs;
//   * per 32-channel chunk: each thread loads one 8x8 patch (tile, channel)
//     straight from x (zero padding applied at load), transforms it row by row
//     and writes V into LDS in v_mfma_f32_16x16x32_f16 B-fragment order
//     ([p][channel octet][tile][8]: one conflict-free 16-byte LDS read per
//     lane per position);
//   * each wave owns 8 of the 64 positions and 4 16-channel row blocks of the
//     filter: 4 MFMAs per position per chunk, U streamed from L2 with 16-byte
//     loads, fp32 accumulators in registers for the whole channel loop;
//   * epilogue: M rounded to fp16 (the reference's rounding point,
//     nova_winograd_fused.hip:405) into LDS as [k][tile][p] (144 KB of the
//     160 KB LDS), then one thread per (k, tile) runs the output transform and
//     writes its 6x6 tile.
// Arithmetic of both transforms is the shared tile math (bit-identical to the
// standalone kernels); the MFMA accumulation order is the hardware's.
#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kFT = 16;        // tiles per workgroup (MFMA N)
constexpr int kFK = 64;        // output channels per workgroup (4 MFMA row blocks)
constexpr int kFC = 32;        // input channels per chunk (MFMA K)
constexpr int kFThreads = 512;  // 8 waves
constexpr int kMPitch = 72;     // halves per (k, tile) row of M in LDS (64 + 8 pad)
constexpr int kVHalves = 64 * kFC * kFT;              // 32768
constexpr int kMHalves = kFK * kFT * kMPitch;         // 73728 (144 KB)
constexpr int kLdsHalves = kVHalves > kMHalves ? kVHalves : kMHalves;

__global__ __launch_bounds__(kFThreads, 1) void fused_kernel(
    const _Float16* __restrict__ x, const _Float16* __restrict__ U, _Float16* __restrict__ y,
    int C, int K, int Cp, int H, int W, int pad, int nh, int nw, int Ho, int Wo, int64_t BP,
    int x_bytes, int u_bytes) {
    __shared__ __align__(16) _Float16 lds[kLdsHalves];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int64_t bp0 = (int64_t)blockIdx.x * kFT;
    const int k0 = blockIdx.y * kFK;
    const int P = nh * nw;

    // ---- input-side mapping: one (tile, channel) pair per thread ----
    const int t = tid & (kFT - 1);
    const int cl = tid >> 4;  // channel within the chunk, 0..31
    const int64_t bp = bp0 + t;
    const bool tile_ok = bp < BP;
    const int b = tile_ok ? (int)(bp / P) : 0;
    const int tile = tile_ok ? (int)(bp % P) : 0;
    const int hbase = (tile / nw) * 6 - pad, wbase = (tile % nw) * 6 - pad;
    // x is read through a buffer resource: an offset outside the tensor reads
    // 0 (never faults), so the patch needs no address clamping; positions
    // outside the image but inside the tensor (row wrap-around) are zeroed
    // with the row/column validity masks below.
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, x_bytes, 0x00020000);
    uint32_t rmask = 0, cm2[4];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int h = hbase + i;
        rmask |= (tile_ok && h >= 0 && h < H) ? (1u << i) : 0u;
    }
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        const int w0 = wbase + 2 * jj, w1 = w0 + 1;
        cm2[jj] = ((w0 >= 0 && w0 < W) ? 0x0000ffffu : 0u) | ((w1 >= 0 && w1 < W) ? 0xffff0000u : 0u);
    }
    const int HWi = H * W;
    // byte offset of the patch origin inside image b, channel 0 (may be < 0)
    const int org = 2 * (b * C * HWi + hbase * W + wbase);
    // LDS slot of this thread's V values: [p][cl/8][t][cl%8]
    const int vslot = ((cl >> 3) * kFT + t) * 8 + (cl & 7);

    const int r16 = lane & 15;
    const int g = lane >> 4;
    const int u_lane_b = 2 * (r16 * Cp + 8 * g);  // byte offset of this lane's U octet
    const __amdgpu_buffer_rsrc_t urs =
        __builtin_amdgcn_make_buffer_rsrc((void*)U, (short)0, u_bytes, 0x00020000);

    f4 acc[8][4];
#pragma unroll
    for (int q = 0; q < 8; q++)
#pragma unroll
        for (int m = 0; m < 4; m++) acc[q][m] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int c0 = 0; c0 < Cp; c0 += kFC) {
        // -- input transform of one (tile, channel) patch into LDS --
        {
            const int c = c0 + cl;
            // invalid channel: push the offset past the end of the buffer
            const int cbase = c < C ? org + 2 * c * HWi : (int)0x80000000;
            uint32_t pr[8][4];
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int o = cbase + 2 * (i * W + 2 * jj);
                    const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(xrs, o, 0, 0);
                    const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(xrs, o + 2, 0, 0);
                    pr[i][jj] = lo | (hi << 16);
                }
            h2 d2[8][4];
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const uint32_t v = pr[i][jj] & (((rmask >> i) & 1u) ? cm2[jj] : 0u);
                    d2[i][jj] = __builtin_bit_cast(h2, v);
                }
            input_tile_rows([&](int i, int j) { return (float)d2[i][j >> 1][j & 1]; },
                            [&](int r, int s, float v) {
                                lds[(r * 8 + s) * (kFC * kFT) + vslot] = to_f16(v);
                            });
        }
        __syncthreads();
        // -- 64 position GEMM slices, 8 per wave. Software pipelined by hand:
        // the fragments of position q+1 load while q's MFMAs run; the
        // scheduling barrier keeps the compiler from hoisting more loads (all
        // 32 U fragments would not fit beside the accumulators). --
        {
            // U fragments through a buffer resource: byte offset = per-lane
            // part (row, channel octet) + wave-uniform part (position, row
            // block, chunk). Lanes whose row is >= K or whose channel octet
            // is past Cp get an offset beyond the buffer and read zeros --
            // no branches, so the loads of position q+1 stay in flight while
            // q's MFMAs run.
            const bool cok = c0 + 8 * g < Cp;
            int voff[4];
#pragma unroll
            for (int m = 0; m < 4; m++)
                voff[m] = (cok && k0 + 16 * m + r16 < K) ? u_lane_b : (int)0x80000000;
            auto load_a = [&](int p, h8 a[4]) {
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const int soff = 2 * (((p * K) + k0 + 16 * m) * Cp + c0);  // uniform
                    a[m] = __builtin_bit_cast(
                        h8, __builtin_amdgcn_raw_buffer_load_b128(urs, voff[m], soff, 0));
                }
            };
            h8 a_cur[4], a_nxt[4];
            load_a(wave_u * 8, a_cur);
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int p = wave_u * 8 + q;
                if (q < 7) load_a(p + 1, a_nxt);
                const h8 bf = *reinterpret_cast<const h8*>(lds + p * (kFC * kFT) + lane * 8);
#pragma unroll
                for (int m = 0; m < 4; m++)
                    acc[q][m] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(a_cur[m], bf, acc[q][m], 0, 0, 0);
                if (q < 7) {
#pragma unroll
                    for (int m = 0; m < 4; m++) a_cur[m] = a_nxt[m];
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();
    }

    // ---- epilogue: M = fp16(acc) for all 64 output channels into LDS, then
    // the output transform, two (k, tile) pairs per thread ----
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const int p = wave_u * 8 + q;
#pragma unroll
        for (int m = 0; m < 4; m++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kk = m * 16 + 4 * g + i;
                lds[(kk * kFT + r16) * kMPitch + p] = to_f16(acc[q][m][i]);
            }
    }
    __syncthreads();
    uint16_t* yr = reinterpret_cast<uint16_t*>(y);
#pragma unroll 1
    for (int pass = 0; pass < 2; pass++) {
        const int kk = pass * 32 + (tid >> 4);  // 0..63
        const int to = tid & (kFT - 1);          // tile
        const int k = k0 + kk;
        const int64_t bpo = bp0 + to;
        if (k < K && bpo < BP) {
            const _Float16* mrow = lds + (kk * kFT + to) * kMPitch;
            h8 mv[8];
#pragma unroll
            for (int v = 0; v < 8; v++) mv[v] = *reinterpret_cast<const h8*>(mrow + v * 8);
            float out[6][6];
            output_tile([&](int i, int j) { return (float)mv[i][j]; }, out);
            const int bo = (int)(bpo / P);
            const int tl = (int)(bpo % P);
            const int oh = (tl / nw) * 6, ow = (tl % nw) * 6;
            const uint32_t ybase = ((uint32_t)bo * (uint32_t)K + (uint32_t)k) * (uint32_t)(Ho * Wo);
#pragma unroll
            for (int r = 0; r < 6; r++) {
                if (oh + r >= Ho) break;
#pragma unroll
                for (int s = 0; s < 6; s++)
                    if (ow + s < Wo)
                        yr[ybase + (uint32_t)((oh + r) * Wo + ow + s)] =
                            __builtin_bit_cast(uint16_t, to_f16(out[r][s]));
            }
        }
    }
}

bool fused_supported(int K, int C) { return K >= 1 && C >= 1; }

// The kernel addresses x and U through buffer resources with 32-bit byte
// offsets and y with 32-bit element offsets.
bool fused_fits(int64_t x_elems, int64_t u_elems, int64_t y_elems) {
    const int64_t lim = (int64_t)1 << 31;
    return 2 * x_elems < lim && 2 * u_elems < lim && y_elems < lim;
}

const char* fused_name(int, int, int64_t) { return "fused_kernel"; }

hipError_t launch_fused(const uint16_t* x, const uint16_t* U, uint16_t* y, int B, int C, int K,
                        int Cp, int H, int W, int pad, int nh, int nw, int Ho, int Wo,
                        hipStream_t s) {
    const int64_t BP = (int64_t)B * nh * nw;
    dim3 grid((unsigned)((BP + kFT - 1) / kFT), (unsigned)((K + kFK - 1) / kFK));
    fused_kernel<<<grid, dim3(kFThreads), 0, s>>>(
        reinterpret_cast<const _Float16*>(x), reinterpret_cast<const _Float16*>(U),
        reinterpret_cast<_Float16*>(y), C, K, Cp, H, W, pad, nh, nw, Ho, Wo, BP,
        (int)(2 * (int64_t)B * C * H * W), (int)(2 * (int64_t)64 * K * Cp));
    return hipGetLastError();
}

}  // namespace nova
