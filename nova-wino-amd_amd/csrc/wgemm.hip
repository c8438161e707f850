// Winograd-domain batched GEMM on CDNA4 matrix cores (gfx950).
//
// Replaces the reference's rocBLAS call
// (/root/reference/csrc/nova_winograd.hip:589-601: 64 GEMMs, m=K, n=BP, k=C,
// fp16 operands, fp32 accumulate, fp16 result) with one hand-written kernel:
//
//   M_p[bp][k] = fp16( sum_c U_p[k][c] * V_p[bp][c] ),  p = 0..63
//
// Operand layouts keep the reduction index (c) contiguous so every lane feeds
// v_mfma_f32_16x16x32_f16 with one 16-byte load: A = U_p rows (16 k x 32 c),
// B = V_p rows (32 c x 16 bp). Lane l holds row/column (l % 16) and the eight
// channels 8*(l/16) .. 8*(l/16)+7 of the current 32-channel step; the
// accumulator lane holds D[4*(l/16) + i][l % 16]. The channel pitch Cp is a
// multiple of 8 and zero padded, so partial 32-channel steps only mask whole
// 8-channel groups. No atomics, no split-K: results are deterministic.
#include "nova_internal.h"

namespace nova {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

// MT x NT 16x16 MFMA tiles per wave, WGM x WGN waves per workgroup.
template <int MT, int NT, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void wgemm_kernel(
    const _Float16* __restrict__ U, const _Float16* __restrict__ V, _Float16* __restrict__ M,
    int K, int Cp, int BP) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave % WGM, wn = wave / WGM;
    const int p = blockIdx.z;
    const int kbase = blockIdx.y * (MT * 16 * WGM) + wm * MT * 16;
    const int nbase = blockIdx.x * (NT * 16 * WGN) + wn * NT * 16;
    const int r16 = lane & 15;
    const int g = lane >> 4;

    const _Float16* Up = U + (int64_t)p * K * Cp;
    const _Float16* Vp = V + (int64_t)p * BP * Cp;

    const _Float16* arow[MT];
    bool aok[MT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        const int k = kbase + mi * 16 + r16;
        aok[mi] = k < K;
        arow[mi] = Up + (int64_t)(aok[mi] ? k : 0) * Cp + 8 * g;
    }
    const _Float16* brow[NT];
    bool bok[NT];
#pragma unroll
    for (int ni = 0; ni < NT; ni++) {
        const int n = nbase + ni * 16 + r16;
        bok[ni] = n < BP;
        brow[ni] = Vp + (int64_t)(bok[ni] ? n : 0) * Cp + 8 * g;
    }

    f4 acc[MT][NT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int ni = 0; ni < NT; ni++) acc[mi][ni] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    const h8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll 2
    for (int c = 0; c < Cp; c += 32) {
        const bool cok = c + 8 * g < Cp;
        h8 a[MT], b[NT];
#pragma unroll
        for (int mi = 0; mi < MT; mi++)
            a[mi] = (aok[mi] && cok) ? *reinterpret_cast<const h8*>(arow[mi] + c) : zero8;
#pragma unroll
        for (int ni = 0; ni < NT; ni++)
            b[ni] = (bok[ni] && cok) ? *reinterpret_cast<const h8*>(brow[ni] + c) : zero8;
#pragma unroll
        for (int mi = 0; mi < MT; mi++)
#pragma unroll
            for (int ni = 0; ni < NT; ni++)
                acc[mi][ni] =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
    }

    _Float16* Mp = M + (int64_t)p * BP * K;
    const bool vec_store = (K & 3) == 0;
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int ni = 0; ni < NT; ni++) {
            const int bp = nbase + ni * 16 + r16;
            const int k = kbase + mi * 16 + 4 * g;
            if (bp >= BP) continue;
            _Float16* dst = Mp + (int64_t)bp * K + k;
            if (vec_store && k + 3 < K) {
                h4 v = {(_Float16)acc[mi][ni][0], (_Float16)acc[mi][ni][1],
                        (_Float16)acc[mi][ni][2], (_Float16)acc[mi][ni][3]};
                *reinterpret_cast<h4*>(dst) = v;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (k + i < K) dst[i] = (_Float16)acc[mi][ni][i];
            }
        }
}

template <int MT, int NT, int WGM, int WGN>
static hipError_t launch_cfg(const uint16_t* U, const uint16_t* V, uint16_t* M, int K, int Cp,
                             int BP, hipStream_t s) {
    constexpr int TM = MT * 16 * WGM, TN = NT * 16 * WGN;
    dim3 grid((unsigned)((BP + TN - 1) / TN), (unsigned)((K + TM - 1) / TM), 64);
    wgemm_kernel<MT, NT, WGM, WGN><<<grid, dim3(64 * WGM * WGN), 0, s>>>(
        reinterpret_cast<const _Float16*>(U), reinterpret_cast<const _Float16*>(V),
        reinterpret_cast<_Float16*>(M), K, Cp, BP);
    return hipGetLastError();
}

hipError_t launch_wgemm(const uint16_t* U, const uint16_t* V, uint16_t* M, int K, int Cp,
                        int BP, hipStream_t s) {
    if (BP <= 16) return launch_cfg<1, 1, 4, 1>(U, V, M, K, Cp, BP, s);   // 64 x 16
    if (BP <= 64) return launch_cfg<1, 2, 4, 1>(U, V, M, K, Cp, BP, s);   // 64 x 32
    return launch_cfg<2, 2, 2, 2>(U, V, M, K, Cp, BP, s);                 // 64 x 64
}

}  // namespace nova
