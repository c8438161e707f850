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
// Buffer-resource helpers. Every tensor is addressed through a raw buffer
// resource: an offset at or past num_records reads 0 and drops stores, so
// padding, tails and invalid lanes need no branches, and loads/stores take
// their constant parts as instruction immediates or scalar offsets (no
// per-access vector address arithmetic).
// ---------------------------------------------------------------------------
constexpr int kOob = (int)0x80000000;  // byte offset beyond any buffer used here

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                             (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                             0x00020000);
}

// ---------------------------------------------------------------------------
// Input transform.
// Workgroup = one tile row (th) x kInTW tiles along w x kInCB channels of one
// image. Staging: each thread copies two full input rows (kInCols elements)
// of the 8-row strip into LDS -- one vector offset per row, the column in the
// load/store immediates; rows outside the image and channels past C read as
// zeros through the buffer bounds. Compute: one (tile, channel) patch per
// thread out of LDS (4-byte pair reads), 64 positions written with lanes over
// consecutive channels (128 B per store instruction), position stride as a
// scalar offset.
// ---------------------------------------------------------------------------
constexpr int kInTW = 4;                   // tiles per workgroup along w
constexpr int kInCB = 64;                  // channels per workgroup
constexpr int kInCols = kInTW * 6 + 2;     // 26 input columns per strip
constexpr int kInPlane = 8 * kInCols + 2;  // 210 halves per channel (odd dword stride)

__global__ __launch_bounds__(256) void input_transform_kernel(
    const _Float16* __restrict__ x, _Float16* __restrict__ V, int C, int H, int W, int pad,
    int nh, int nw, int ldv, int64_t pstride, int cblocks, int64_t x_bytes, int64_t v_bytes) {
    __shared__ __align__(16) _Float16 sx[kInCB * kInPlane];
    // 1-D grid over (tile block, tile row, image x channel block), x fastest
    const int nwb = (nw + kInTW - 1) / kInTW;
    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int tw0 = (L % nwb) * kInTW;
    const int th = (L / nwb) % nh;
    const int bz = L / (nwb * nh);
    const int b = bz / cblocks;
    const int c0 = (bz % cblocks) * kInCB;
    const int h0 = th * 6 - pad, w0 = tw0 * 6 - pad;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, x_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, v_bytes);

    // ---- staging: thread (row i, column col) copies its element for all 64
    // channels. Lanes run along the row (two rows per wave: each load covers
    // two 52-byte runs), the channel stride is a scalar offset, and row /
    // column validity is folded into the vector offset (out of range -> 0). ----
    {
        const int i = threadIdx.x >> 5, col = threadIdx.x & 31;
        if (col < kInCols) {
            const int h = h0 + i, w = w0 + col;
            const bool ok = h >= 0 && h < H && w >= 0 && w < W;
            const int voff = ok ? 2 * (((b * C + c0) * H + h) * W + w) : kOob;
            const int HW2 = 2 * H * W;
            const int ncc = min(kInCB, C - c0);  // uniform
            _Float16* sdst = sx + i * kInCols + col;
            uint16_t v[kInCB];
            if (ncc == kInCB) {  // full channel block: all 64 loads in flight at once
#pragma unroll
                for (int u = 0; u < kInCB; u++)
                    v[u] = __builtin_amdgcn_raw_buffer_load_b16(xrs, voff, u * HW2, 0);
            } else {
#pragma unroll
                for (int u = 0; u < kInCB; u++)
                    v[u] = u < ncc ? __builtin_amdgcn_raw_buffer_load_b16(xrs, voff, u * HW2, 0)
                                   : (uint16_t)0;
            }
#pragma unroll
            for (int u = 0; u < kInCB; u++) sdst[u * kInPlane] = __builtin_bit_cast(_Float16, v[u]);
        }
    }
    __syncthreads();

    // ---- compute: (tile t, channel cc) per thread ----
    const int cc = threadIdx.x & 63;
    const int t = threadIdx.x >> 6;
    const int tw = tw0 + t;
    const int c = c0 + cc;
    const int bp = (b * nh + th) * nw + tw;
    const int voff = (tw < nw && c < ldv) ? 2 * (bp * ldv + c) : kOob;
    const _Float16* sp = sx + cc * kInPlane + t * 6;
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 d2[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
            d2[i][jj] = *reinterpret_cast<const h2*>(sp + i * kInCols + 2 * jj);
    input_tile_rows([&](int i, int j) { return (float)d2[i][j >> 1][j & 1]; },
                    [&](int r, int s, float v) {
                        const int p = r * 8 + s;
                        __builtin_amdgcn_raw_buffer_store_b16(
                            __builtin_bit_cast(uint16_t, to_f16(v)), vrs, voff,
                            (int)(2 * p * pstride), 0);
                    });
}

hipError_t launch_input_transform(const uint16_t* x, uint16_t* V, int B, int C, int H, int W,
                                  int pad, int nh, int nw, int ldv, int64_t pstride,
                                  hipStream_t s) {
    const int cblocks = (ldv + kInCB - 1) / kInCB;
    const int64_t nblocks = (int64_t)((nw + kInTW - 1) / kInTW) * nh * B * cblocks;
    if (nblocks >= ((int64_t)1 << 31)) return hipErrorInvalidConfiguration;
    input_transform_kernel<<<dim3((unsigned)nblocks), dim3(256), 0, s>>>(
        reinterpret_cast<const _Float16*>(x), reinterpret_cast<_Float16*>(V), C, H, W, pad, nh,
        nw, ldv, pstride, cblocks, 2 * (int64_t)B * C * H * W, 2 * 64 * pstride);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Output transform.
// Workgroup = one tile row x kOutTW tiles x kOutKB output channels of one
// image. Each thread reads the 64 positions of one (tile, k) (lanes over
// consecutive k: coalesced; position stride as a scalar offset), computes the
// 6x6 tile into LDS; the workgroup then writes whole output rows (one vector
// offset per row, the column in the store immediate). Rows past Ho and
// channels past K fall outside the buffer and are dropped; columns past Wo
// are skipped with a workgroup-uniform bound.
// ---------------------------------------------------------------------------
constexpr int kOutTW = 4;
constexpr int kOutKB = 64;
constexpr int kOutCols = kOutTW * 6;         // 24
constexpr int kOutPlane = 6 * kOutCols + 2;  // 146 halves = 73 dwords (odd)

__global__ __launch_bounds__(256) void output_transform_kernel(
    const _Float16* __restrict__ M, _Float16* __restrict__ y, int K, int Ho, int Wo, int nh,
    int nw, int ldm, int64_t pstride, int kblocks, int64_t m_bytes, int64_t y_bytes) {
    __shared__ __align__(16) _Float16 sy[kOutKB * kOutPlane];
    const int nwb = (nw + kOutTW - 1) / kOutTW;
    const int L = xcd_remap(blockIdx.x, gridDim.x);
    const int tw0 = (L % nwb) * kOutTW;
    const int th = (L / nwb) % nh;
    const int bz = L / (nwb * nh);
    const int b = bz / kblocks;
    const int k0 = (bz % kblocks) * kOutKB;
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(M, m_bytes);
    const __amdgpu_buffer_rsrc_t yrs = make_rsrc(y, y_bytes);

    {
        const int kk = threadIdx.x & 63;
        const int t = threadIdx.x >> 6;
        const int tw = tw0 + t;
        const int k = k0 + kk;
        const int bp = (b * nh + th) * nw + tw;
        const int moff = (tw < nw && k < K) ? 2 * (bp * ldm + k) : kOob;
        uint16_t m[64];
#pragma unroll
        for (int p = 0; p < 64; p++)
            m[p] = __builtin_amdgcn_raw_buffer_load_b16(mrs, moff, (int)(2 * p * pstride), 0);
        float out[6][6];
        output_tile([&](int i, int j) { return (float)__builtin_bit_cast(_Float16, m[i * 8 + j]); },
                    out);
        _Float16* sp = sy + kk * kOutPlane + t * 6;
#pragma unroll
        for (int r = 0; r < 6; r++)
#pragma unroll
            for (int s = 0; s < 6; s++) sp[r * kOutCols + s] = to_f16(out[r][s]);
    }
    __syncthreads();

    // ---- store: thread (row r, column col) writes its element for all 64
    // channels: lanes run along the output row (two rows per wave), the
    // channel stride is a scalar offset; rows past Ho / columns past the
    // tile block or Wo fall outside and are dropped. ----
    {
        const int r = threadIdx.x >> 5, col = threadIdx.x & 31;
        const int h = th * 6 + r, w = tw0 * 6 + col;
        const int ncols = min(kOutCols, (nw - tw0) * 6);  // uniform
        if (r < 6 && col < ncols) {
            const bool ok = h < Ho && w < Wo;
            const int yoff = ok ? 2 * (((b * K + k0) * Ho + h) * Wo + w) : kOob;
            const int HoWo2 = 2 * Ho * Wo;
            const int nkk = min(kOutKB, K - k0);  // uniform
            const _Float16* ssrc = sy + r * kOutCols + col;
#pragma unroll 16
            for (int u = 0; u < kOutKB; u++) {
                if (u < nkk)
                    __builtin_amdgcn_raw_buffer_store_b16(
                        __builtin_bit_cast(uint16_t, ssrc[u * kOutPlane]), yrs, yoff, u * HoWo2, 0);
            }
        }
    }
}

hipError_t launch_output_transform(const uint16_t* M, uint16_t* y, int B, int K, int Ho,
                                   int Wo, int nh, int nw, int ldm, int64_t pstride,
                                   hipStream_t s) {
    const int kblocks = (K + kOutKB - 1) / kOutKB;
    const int64_t nblocks = (int64_t)((nw + kOutTW - 1) / kOutTW) * nh * B * kblocks;
    if (nblocks >= ((int64_t)1 << 31)) return hipErrorInvalidConfiguration;
    output_transform_kernel<<<dim3((unsigned)nblocks), dim3(256), 0, s>>>(
        reinterpret_cast<const _Float16*>(M), reinterpret_cast<_Float16*>(y), K, Ho, Wo, nh, nw,
        ldm, pstride, kblocks, 2 * 64 * pstride, 2 * (int64_t)B * K * Ho * Wo);
    return hipGetLastError();
}

}  // namespace nova
