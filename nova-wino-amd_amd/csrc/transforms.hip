// NOVA F(6,3) transforms for gfx950: filter (G w G^T), input (B^T d B) and
// output (A M A^T).
//
// Arithmetic contract (shared with the CPU oracle): every dot product is an
// fp32 fused-multiply-add chain in the reference's loop order starting from
// +0; input/output transforms skip zero table coefficients (exact for finite
// operands); results are rounded once to fp16. This file is compiled with
// -ffp-contract=off, so the only fused operations are the explicit fmaf calls.
//
// Reference behaviour followed:
//   filter  /root/reference/csrc/nova_winograd.hip:214-255
//   input   /root/reference/csrc/nova_winograd.hip:336-392 (fused zero padding :368-370)
//   output  /root/reference/csrc/nova_winograd.hip:398-450 (masking of h>=Ho, w>=Wo)
#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

// ---------------------------------------------------------------------------
// Filter transform: one thread per (k, c) pair computes all 64 positions.
// ---------------------------------------------------------------------------
template <bool kRefLayout>
__global__ __launch_bounds__(256) void filter_transform_kernel(const float* __restrict__ w,
                                                               _Float16* __restrict__ U, int K,
                                                               int C, int Cp) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int cols = kRefLayout ? C : Cp;  // threads along c (product layout pads)
    if (idx >= (int64_t)K * cols) return;
    int k, c;
    if (kRefLayout) {
        // c-major thread order: consecutive threads write consecutive k.
        c = (int)(idx / K);
        k = (int)(idx % K);
    } else {
        k = (int)(idx / cols);
        c = (int)(idx % cols);
    }
    float u[8][8];
    if (c < C) {
        float f[3][3];
        const float* wp = w + ((int64_t)k * C + c) * 9;
#pragma unroll
        for (int i = 0; i < 9; i++) f[i / 3][i % 3] = wp[i];
        filter_tile(f, u);
    } else {
#pragma unroll
        for (int r = 0; r < 8; r++)
#pragma unroll
            for (int s = 0; s < 8; s++) u[r][s] = 0.0f;
    }
    if (kRefLayout) {
        const int64_t KC = (int64_t)K * C;
        _Float16* out = U + (int64_t)c * K + k;
#pragma unroll
        for (int p = 0; p < 64; p++) out[p * KC] = to_f16(u[p >> 3][p & 7]);
    } else {
        const int64_t KCp = (int64_t)K * Cp;
        _Float16* out = U + (int64_t)k * Cp + c;
#pragma unroll
        for (int p = 0; p < 64; p++) out[p * KCp] = to_f16(u[p >> 3][p & 7]);
    }
}

hipError_t launch_filter_transform_ref(const float* w, uint16_t* U, int K, int C,
                                       hipStream_t s) {
    const int64_t n = (int64_t)K * C;
    const int64_t blocks = (n + 255) / 256;
    filter_transform_kernel<true><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        w, reinterpret_cast<_Float16*>(U), K, C, C);
    return hipGetLastError();
}

hipError_t launch_filter_transform_gemm(const float* w, uint16_t* U, int K, int C, int Cp,
                                        hipStream_t s) {
    const int64_t n = (int64_t)K * Cp;
    const int64_t blocks = (n + 255) / 256;
    filter_transform_kernel<false><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        w, reinterpret_cast<_Float16*>(U), K, C, Cp);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Input transform.
// Workgroup = one tile row (th) x kTW tiles along w x kCB channels of one
// image. The 8 x (6*kTW+2) input strip of every channel is staged in LDS with
// row-coalesced global loads (zero padding applied at load time); each thread
// then transforms one (tile, channel) patch out of LDS and writes its 64
// positions, lanes covering consecutive channels (coalesced 128 B per store).
// ---------------------------------------------------------------------------
constexpr int kInTW = 4;                 // tiles per workgroup along w
constexpr int kInCB = 64;                // channels per workgroup
constexpr int kInCols = kInTW * 6 + 2;   // input columns per strip
constexpr int kInPlane = 8 * kInCols + 2;  // halves per channel plane (odd dword stride)

__global__ __launch_bounds__(256) void input_transform_kernel(
    const _Float16* __restrict__ x, _Float16* __restrict__ V, int C, int H, int W, int pad,
    int nh, int nw, int ldv, int64_t pstride, int cblocks) {
    __shared__ _Float16 sx[kInCB * kInPlane];
    const int tw0 = blockIdx.x * kInTW;
    const int th = blockIdx.y;
    const int b = blockIdx.z / cblocks;
    const int c0 = (blockIdx.z % cblocks) * kInCB;
    const int h0 = th * 6 - pad, w0 = tw0 * 6 - pad;
    const _Float16* xb = x + (int64_t)b * C * H * W;

    for (int idx = threadIdx.x; idx < kInCB * 8 * kInCols; idx += 256) {
        const int cc = idx / (8 * kInCols);
        const int rem = idx - cc * (8 * kInCols);
        const int i = rem / kInCols;
        const int j = rem - i * kInCols;
        const int c = c0 + cc, h = h0 + i, ww = w0 + j;
        _Float16 v = (_Float16)0.0f;
        if (c < C && h >= 0 && h < H && ww >= 0 && ww < W) v = xb[((int64_t)c * H + h) * W + ww];
        sx[cc * kInPlane + i * kInCols + j] = v;
    }
    __syncthreads();

    const int cc = threadIdx.x & 63;
    const int t = threadIdx.x >> 6;
    const int tw = tw0 + t;
    const int c = c0 + cc;
    if (tw >= nw || c >= ldv) return;
    const int64_t bp = ((int64_t)b * nh + th) * nw + tw;
    _Float16* out = V + bp * ldv + c;
    if (c >= C) {  // zero padding of the channel pitch
#pragma unroll
        for (int p = 0; p < 64; p++) out[p * pstride] = (_Float16)0.0f;
        return;
    }
    const _Float16* sp = sx + cc * kInPlane + t * 6;
    float v[8][8];
    input_tile([&](int i, int j) { return (float)sp[i * kInCols + j]; }, v);
#pragma unroll
    for (int p = 0; p < 64; p++) out[p * pstride] = to_f16(v[p >> 3][p & 7]);
}

hipError_t launch_input_transform(const uint16_t* x, uint16_t* V, int B, int C, int H, int W,
                                  int pad, int nh, int nw, int ldv, int64_t pstride,
                                  hipStream_t s) {
    const int cblocks = (ldv + kInCB - 1) / kInCB;
    dim3 grid((unsigned)((nw + kInTW - 1) / kInTW), (unsigned)nh, (unsigned)(B * cblocks));
    input_transform_kernel<<<grid, dim3(256), 0, s>>>(
        reinterpret_cast<const _Float16*>(x), reinterpret_cast<_Float16*>(V), C, H, W, pad, nh,
        nw, ldv, pstride, cblocks);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Output transform.
// Workgroup = one tile row x kOutTW tiles x kOutKB output channels of one
// image. Each thread reads the 64 positions of one (tile, k) (lanes over
// consecutive k: coalesced), computes the 6x6 tile, parks it in LDS, and the
// workgroup then writes the tile row's output rows with w-contiguous stores.
// ---------------------------------------------------------------------------
constexpr int kOutTW = 4;
constexpr int kOutKB = 64;
constexpr int kOutCols = kOutTW * 6;
constexpr int kOutPlane = 6 * kOutCols + 2;  // 146 halves = 73 dwords (odd)

__global__ __launch_bounds__(256) void output_transform_kernel(
    const _Float16* __restrict__ M, _Float16* __restrict__ y, int K, int Ho, int Wo, int nh,
    int nw, int ldm, int64_t pstride, int kblocks) {
    __shared__ _Float16 sy[kOutKB * kOutPlane];
    const int tw0 = blockIdx.x * kOutTW;
    const int th = blockIdx.y;
    const int b = blockIdx.z / kblocks;
    const int k0 = (blockIdx.z % kblocks) * kOutKB;

    const int kk = threadIdx.x & 63;
    const int t = threadIdx.x >> 6;
    const int tw = tw0 + t;
    const int k = k0 + kk;
    if (tw < nw && k < K) {
        const int64_t bp = ((int64_t)b * nh + th) * nw + tw;
        const _Float16* mp = M + bp * ldm + k;
        float out[6][6];
        output_tile([&](int i, int j) { return (float)mp[(i * 8 + j) * pstride]; }, out);
        _Float16* sp = sy + kk * kOutPlane + t * 6;
#pragma unroll
        for (int r = 0; r < 6; r++)
#pragma unroll
            for (int s = 0; s < 6; s++) sp[r * kOutCols + s] = to_f16(out[r][s]);
    }
    __syncthreads();

    const int wbase = tw0 * 6;
    for (int idx = threadIdx.x; idx < kOutKB * 6 * kOutCols; idx += 256) {
        const int q = idx / (6 * kOutCols);
        const int rem = idx - q * (6 * kOutCols);
        const int r = rem / kOutCols;
        const int col = rem - r * kOutCols;
        const int kq = k0 + q, h = th * 6 + r, ww = wbase + col;
        if (kq < K && h < Ho && ww < Wo && (col / 6) + tw0 < nw)
            y[(((int64_t)b * K + kq) * Ho + h) * Wo + ww] = sy[q * kOutPlane + r * kOutCols + col];
    }
}

hipError_t launch_output_transform(const uint16_t* M, uint16_t* y, int B, int K, int Ho,
                                   int Wo, int nh, int nw, int ldm, int64_t pstride,
                                   hipStream_t s) {
    const int kblocks = (K + kOutKB - 1) / kOutKB;
    dim3 grid((unsigned)((nw + kOutTW - 1) / kOutTW), (unsigned)nh, (unsigned)(B * kblocks));
    output_transform_kernel<<<grid, dim3(256), 0, s>>>(
        reinterpret_cast<const _Float16*>(M), reinterpret_cast<_Float16*>(y), K, Ho, Wo, nh, nw,
        ldm, pstride, kblocks);
    return hipGetLastError();
}

}  // namespace nova
