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
#include <algorithm>
#include <type_traits>

#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

// ---------------------------------------------------------------------------
// Filter transform: one thread per (k, c) pair computes all 64 positions.
// ---------------------------------------------------------------------------
template <bool kRefLayout, typename WT>
__global__ __launch_bounds__(256) void filter_transform_kernel(const WT* __restrict__ w,
                                                               _Float16* __restrict__ U, int K,
                                                               int C, int Cp) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 256-thread blocks
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
        // fp16 weights widen to fp32 exactly: the same U as their fp32 copy
        const WT* wp = w + ((int64_t)k * C + c) * 9;
#pragma unroll
        for (int i = 0; i < 9; i++) f[i / 3][i % 3] = (float)wp[i];
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
    launch(filter_transform_kernel<true, float>, dim3((unsigned)blocks), dim3(256), s,
        w, reinterpret_cast<_Float16*>(U), K, C, C);
    return hipGetLastError();
}

hipError_t launch_filter_transform_gemm(const void* w, bool w_f16, uint16_t* U, int K, int C,
                                        int Cp, hipStream_t s) {
    const int64_t n = (int64_t)K * Cp;
    const int64_t blocks = (n + 255) / 256;
    if (w_f16)
        launch(filter_transform_kernel<false, _Float16>, dim3((unsigned)blocks), dim3(256), s,
            static_cast<const _Float16*>(w), reinterpret_cast<_Float16*>(U), K, C, Cp);
    else
        launch(filter_transform_kernel<false, float>, dim3((unsigned)blocks), dim3(256), s,
            static_cast<const float*>(w), reinterpret_cast<_Float16*>(U), K, C, Cp);
    return hipGetLastError();
}

// Reorder U[p][k][Cp] into the fused kernels' A-operand order (zero padded),
// one thread per 4-channel slot (lane, half ks) of a fragment.
__global__ __launch_bounds__(256) void u_frag_kernel(const _Float16* __restrict__ U,
                                                      _Float16* __restrict__ Uf, int K, int Cp,
                                                      int nkt, int nkp, int64_t nslots) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 256-thread blocks
    if (i >= nslots) return;
    const int ks = (int)(i & 1);
    const int lane = (int)((i >> 1) & 63);
    const int64_t frag = i >> 7;  // (p*nkt + kt)*nkp + j
    const int j = (int)(frag % nkp);
    const int kt = (int)((frag / nkp) % nkt);
    const int p = (int)(frag / ((int64_t)nkp * nkt));
    const int k = kt * 16 + (lane & 15);
    const int c = j * 32 + ks * 16 + 4 * (lane >> 4);
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 v = {(_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
    if (k < K && c < Cp) v = *reinterpret_cast<const h4*>(U + ((int64_t)p * K + k) * Cp + c);
    *reinterpret_cast<h4*>(Uf + i * 4) = v;
}

hipError_t launch_u_frag(const uint16_t* U, uint16_t* Uf, int K, int Cp, hipStream_t s) {
    const int nkt = (K + 15) / 16, nkp = (Cp + 31) / 32;
    const int64_t nslots = (int64_t)64 * nkt * nkp * 128;
    launch(u_frag_kernel, dim3((unsigned)((nslots + 255) / 256)), dim3(256), s,
        reinterpret_cast<const _Float16*>(U), reinterpret_cast<_Float16*>(Uf), K, Cp, nkt, nkp,
        nslots);
    return hipGetLastError();
}

// Reorder U[p][k][Cp] into the two-pass kernel's A-operand blocks: per
// (position, 16-row tile, 32-channel chunk) 1 KB in which lane l holds row
// l % 16 and channels 8*(l/16) .. +7 -- the three-pass GEMM's lane layout,
// stored contiguously (zero padded). One thread per lane slot.
__global__ __launch_bounds__(256) void u_wfrag_kernel(const _Float16* __restrict__ U,
                                                       _Float16* __restrict__ Uw, int K, int Cp,
                                                       int nkt, int nkp, int64_t nslots) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 256-thread blocks
    if (i >= nslots) return;
    const int lane = (int)(i & 63);
    const int64_t frag = i >> 6;  // (p*nkt + kt)*nkp + j
    const int j = (int)(frag % nkp);
    const int kt = (int)((frag / nkp) % nkt);
    const int p = (int)(frag / ((int64_t)nkp * nkt));
    const int k = kt * 16 + (lane & 15);
    const int c = j * 32 + 8 * (lane >> 4);
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 v = {};
    if (k < K && c < Cp) v = *reinterpret_cast<const h8*>(U + ((int64_t)p * K + k) * Cp + c);
    *reinterpret_cast<h8*>(Uw + i * 8) = v;
}

hipError_t launch_u_wfrag(const uint16_t* U, uint16_t* Uw, int K, int Cp, hipStream_t s) {
    const int nkt = (K + 15) / 16, nkp = (Cp + 31) / 32;
    const int64_t nslots = (int64_t)64 * nkt * nkp * 64;
    launch(u_wfrag_kernel, dim3((unsigned)((nslots + 255) / 256)), dim3(256), s,
        reinterpret_cast<const _Float16*>(U), reinterpret_cast<_Float16*>(Uw), K, Cp, nkt, nkp,
        nslots);
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

// Byte offset of V element (tile bp, channel c) within one position's plane.
// vfrag == 0: the product layout [bp][ldv]. vfrag = number of 32-channel
// chunks: the two-pass layout, 1 KB blocks (bp / 16, c / 32) in which lane
// (bp % 16) + 16 * ((c % 32) / 8) holds 8 consecutive channels -- the B
// operand of v_mfma_f32_16x16x32_f16 for 16 tiles, one contiguous 1 KB load
// per wave.
__device__ __forceinline__ int v_plane_off(int bp, int c, int ldv, int vfrag) {
    if (vfrag == 0) return 2 * (bp * ldv + c);
    return ((bp >> 4) * vfrag + (c >> 5)) * 1024 + ((bp & 15) + 16 * ((c & 31) >> 3)) * 16 +
           (c & 7) * 2;
}

// ---------------------------------------------------------------------------
// Input transform.
// Workgroup (256 threads) = one tile row (th) x TW tiles along w x 256/TW
// channels of one image; TW (2, 4 or 8) is picked per layer so that padded
// tile and channel slots waste the least work. Staging: the strip's 8 input
// rows of every channel are copied into LDS as whole 16-byte-aligned row spans
// (one buffer load per 16 bytes; rows outside the image and channels past C
// are stored as zeros). Compute: one (tile, channel) patch per thread, each
// row read as five aligned dwords and shifted into place with v_alignbyte;
// columns outside the image (zero padding, or neighbour-row bytes that the
// aligned span picked up) are masked. The 64 positions are written with lanes
// over consecutive channels, the position stride as a scalar offset.
// ---------------------------------------------------------------------------
template <int TW>
struct InGeom {
    static constexpr int kCB = 256 / TW;                           // channels per workgroup
    static constexpr int kCols = TW * 6 + 2;                       // input columns per strip
    static constexpr int kRP = ((2 * kCols + 14 + 4) + 15) & ~15;  // bytes per row span (columns,
                                                                   // alignment slack, one dword
                                                                   // of read-ahead)
    static constexpr int kNJ = kRP / 16;                           // loads per span
    // Channel pitch: an odd number of dwords for TW = 2 and 4, so the compute
    // threads (lanes over 64-128 consecutive channels, one dword per read)
    // spread over all 64 banks: rocprofv3 SQ_LDS_BANK_CONFLICT at ResNet-50
    // conv4_x batch 32 (TW = 4) read 2.6x the LDS's active cycles with an
    // even pitch; staging writes are then single dwords. For TW = 8 an odd
    // multiple of 8 bytes conflicts less (2-way at most on the reads).
    static constexpr int kCP = TW == 8 ? 8 * kRP + 8 : 8 * kRP + 4;
    static constexpr int kUnits = kCB * 8 / 256;                    // (channel, row) spans per
                                                                   // thread
    static constexpr int kBytes = kCB * kCP;
    static_assert(kCB * 8 % 256 == 0, "staged spans must tile the workgroup");
    static_assert(TW == 8 ? (kCP / 8) % 2 == 1 : (kCP / 4) % 2 == 1, "odd channel pitch");
    __device__ static int base(int c) { return c * kCP; }
};

// Staging of the tile-block input transforms: the strip's 8 input rows of
// every channel of the block, copied into LDS as whole 16-byte-aligned row
// spans. Thread = row r (tid % 8) of channels tid / 8 + 32u; each thread
// copies whole row spans (kNJ 16-byte loads at immediate offsets); its spans
// are 32 channels apart, a constant byte step, and their LDS destinations are
// immediate offsets. The whole offset stays in the range-checked vector
// offset, so span bytes past the end of x read zero, as do rows outside the
// image and channels past C.
template <int TW>
__device__ __forceinline__ void input_stage(unsigned char* sx, __amdgpu_buffer_rsrc_t xrs,
                                            int xbase, int C, int H, int W, int HW, int h0,
                                            int c0) {
    using G = InGeom<TW>;
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    const int r = threadIdx.x & 7, c = threadIdx.x >> 3;
    const int h = h0 + r;
    const bool row_ok = h >= 0 && h < H;
    // 64*HW bytes per 32 channels is a multiple of 16: every span of this
    // thread starts at the same offset within its 16-byte granule
    const int ga = (xbase + 2 * (c * HW + h * W)) & ~15;
    unsigned char* dst = sx + G::base(c) + r * G::kRP;
    u4 val[G::kUnits][G::kNJ];
#pragma unroll
    for (int u = 0; u < G::kUnits; u++) {
        const int vo = (row_ok && c0 + c + 32 * u < C) ? ga + 64 * u * HW : kOob;
#pragma unroll
        for (int q = 0; q < G::kNJ; q++)
            val[u][q] = __builtin_amdgcn_raw_buffer_load_b128(xrs, vo + 16 * q, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < G::kUnits; u++)
#pragma unroll
        for (int q = 0; q < G::kNJ; q++) {
            unsigned char* d = dst + 32 * u * G::kCP + 16 * q;
            if constexpr (G::kCP % 8 == 0) {
                *reinterpret_cast<u2*>(d) = u2{val[u][q][0], val[u][q][1]};
                *reinterpret_cast<u2*>(d + 8) = u2{val[u][q][2], val[u][q][3]};
            } else {  // 4-byte aligned spans
#pragma unroll
                for (int k = 0; k < 4; k++) reinterpret_cast<unsigned*>(d)[k] = val[u][q][k];
            }
        }
}

template <int TW, int kPol>
__global__ __launch_bounds__(256) void input_transform_kernel(
    const void* __restrict__ x_al, _Float16* __restrict__ V, int C, int H, int W, int pad,
    int nh, int nw, int ldv, int64_t pstride, int cblocks, int x_bytes, int xd,
    int64_t v_bytes, int vfrag, int nwg) {
    using G = InGeom<TW>;
    __shared__ __align__(16) unsigned char sx[G::kBytes];
    // 1-D grid over (tile block, tile row, image x channel block), x fastest
    const int nwb = (nw + TW - 1) / TW;
    const int L = xcd_remap(blockIdx.x, nwg);
    const int tw0 = (L % nwb) * TW;
    const int th = (L / nwb) % nh;
    const int bz = L / (nwb * nh);
    const int b = bz / cblocks;
    const int c0 = (bz % cblocks) * G::kCB;
    const int h0 = th * 6 - pad, w0 = tw0 * 6 - pad;
    const int HW = H * W;
    // Byte offset (from x_al) of element (b, c0, h=0, w=w0). Spans start at
    // the strip's first column even when it is left of the image (w0 < 0):
    // offsets below 0 wrap past the buffer end and read zeros, and every
    // compute read then lies at or after its span's start.
    const int xbase = xd + 2 * ((b * C + c0) * HW + w0);
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x_al, x_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, v_bytes);

    input_stage<TW>(sx, xrs, xbase, C, H, W, HW, h0, c0);
    __syncthreads();

    // ---- compute: (tile t, channel cc) per thread, lanes over channels ----
    const int cc = threadIdx.x % G::kCB;
    const int t = threadIdx.x / G::kCB;
    const int tw = tw0 + t;
    const int c = c0 + cc;
    // slots past the last tile or channel have nothing to store (no barrier
    // follows: whole idle waves retire and free their SIMD)
    if (tw >= nw || c >= ldv) return;
    const int bp = (b * nh + th) * nw + tw;
    const int voff = v_plane_off(bp, c, ldv, vfrag);
    unsigned cmask = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int w = w0 + 6 * t + j;
        cmask |= (w >= 0 && w < W) ? (1u << j) : 0u;
    }
    // column mask as four dword masks over the packed halves
    unsigned dm[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
        dm[q] = (((cmask >> (2 * q)) & 1u) ? 0xffffu : 0u) |
                (((cmask >> (2 * q + 1)) & 1u) ? 0xffff0000u : 0u);
    // Row i of the patch: 8 halves at byte sb = rho + 12t of its span. Read
    // the five aligned dwords from floor4(sb) and shift each output dword by
    // (sb & 3) bytes (0 or 2) with v_alignbyte: aligned LDS reads only.
    unsigned d4[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int rho = (xbase + 2 * (cc * HW + (h0 + i) * W)) & 15;
        const int sb = rho + 12 * t;
        const unsigned* src = reinterpret_cast<const unsigned*>(sx + G::base(cc) + i * G::kRP +
                                                                (sb & ~3));
        unsigned w5[5];
#pragma unroll
        for (int q = 0; q < 5; q++) w5[q] = src[q];
#pragma unroll
        for (int q = 0; q < 4; q++)
            d4[i][q] = __builtin_amdgcn_alignbyte(w5[q + 1], w5[q], (unsigned)(sb & 3));
    }
    // edge tiles: zero the columns outside the image (zero padding, or bytes of
    // the neighbouring row that the aligned span picked up)
    if (cmask != 0xffu) {
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) d4[i][q] &= dm[q];
    }
    input_tile_rows(
        [&](int i, int j) {
            const unsigned pair = d4[i][j >> 1];
            const unsigned short bits = (unsigned short)((j & 1) ? (pair >> 16) : (pair & 0xffffu));
            return (float)__builtin_bit_cast(_Float16, bits);
        },
        [&](int r, int s, float v) {
            const int p = r * 8 + s;
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, to_f16(v)), vrs,
                                                  voff, (int)(2 * p * pstride), kPol);
        });
}

// ---------------------------------------------------------------------------
// Input transform, NHWC (channels-last) x, tile-block form. Workgroup = one
// tile row x TW tiles x 256/TW channels, as for NCHW. Staging: the strip's 8
// rows x (6*TW + 2) pixels x the block's channels, 16-byte loads of 8
// channels of one pixel (pixels outside the image and channels past C read
// zero through out-of-range offsets), into LDS as [row][pixel][channel] with
// the channel run padded by 8 halves. Compute: thread (channel cc, tile t)
// reads its 64 values as 2-byte LDS reads (lanes over consecutive channels,
// consecutive addresses), the shared FMA chains, and stores V like the NCHW
// kernel. Zero padding is already in LDS, so no masks. Needs C % 8 == 0 and a
// 16-byte aligned x (the launcher checks; otherwise the lane-parallel form).
// ---------------------------------------------------------------------------
template <int TW, int kPol>
__global__ __launch_bounds__(256) void input_nhwc_kernel(
    const _Float16* __restrict__ x, _Float16* __restrict__ V, int C, int H, int W, int pad,
    int nh, int nw, int ldv, int64_t pstride, int cblocks, int x_bytes, int64_t v_bytes,
    int vfrag, int nwg) {
    constexpr int kCB = 256 / TW;
    constexpr int kCols = 6 * TW + 2;
    constexpr int kPix = kCB + 8;            // halves per staged pixel
    constexpr int kGroups = kCB / 8;         // 16-byte channel groups per pixel
    constexpr int kUnits = 8 * kCols * kGroups;
    constexpr int kRounds = (kUnits + 255) / 256;
    __shared__ __align__(16) _Float16 sx[8 * kCols * kPix];
    const int nwb = (nw + TW - 1) / TW;
    const int L = xcd_remap(blockIdx.x, nwg);
    const int tw0 = (L % nwb) * TW;
    const int th = (L / nwb) % nh;
    const int bz = L / (nwb * nh);
    const int b = bz / cblocks;
    const int c0 = (bz % cblocks) * kCB;
    const int h0 = th * 6 - pad, w0 = tw0 * 6 - pad;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, x_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, v_bytes);
    {
        typedef unsigned u4 __attribute__((ext_vector_type(4)));
        u4 val[kRounds];
        int dst[kRounds];
#pragma unroll
        for (int u = 0; u < kRounds; u++) {
            const int e = threadIdx.x + 256 * u;
            const int g = e % kGroups, pix = (e / kGroups) % kCols, r = e / (kGroups * kCols);
            const int h = h0 + r, w = w0 + pix, c = c0 + 8 * g;
            const bool ok = e < kUnits && h >= 0 && h < H && w >= 0 && w < W && c < C;
            val[u] = __builtin_amdgcn_raw_buffer_load_b128(
                xrs, ok ? 2 * (((b * H + h) * W + w) * C + c) : kOob, 0, 0);
            dst[u] = e < kUnits ? (r * kCols + pix) * kPix + 8 * g : -1;
        }
#pragma unroll
        for (int u = 0; u < kRounds; u++)
            if (dst[u] >= 0) *reinterpret_cast<u4*>(sx + dst[u]) = val[u];
    }
    __syncthreads();
    const int cc = threadIdx.x % kCB;
    const int t = threadIdx.x / kCB;
    const int tw = tw0 + t;
    const int c = c0 + cc;
    if (tw >= nw || c >= ldv) return;  // nothing to store; no barrier follows
    const int bp = (b * nh + th) * nw + tw;
    const int voff = v_plane_off(bp, c, ldv, vfrag);
    const _Float16* src = sx + 6 * t * kPix + cc;
    input_tile_rows([&](int i, int j) { return (float)src[(i * kCols + j) * kPix]; },
                    [&](int r, int s2, float v) {
                        const int p = r * 8 + s2;
                        __builtin_amdgcn_raw_buffer_store_b16(
                            __builtin_bit_cast(uint16_t, to_f16(v)), vrs, voff,
                            (int)(2 * p * pstride), kPol);
                    });
}

// ---------------------------------------------------------------------------
// Input transform, lane-parallel form: 8 lanes per (tile, channel) patch, so a
// wave carries 8 channels of one tile and a thread's instruction chain is an
// eighth of the one-patch-per-thread form (short latency at batch 1, many
// waves to hide memory latency at large batch). Lane (channel cl, column j):
//   1. loads column j of the 8x8 patch straight from x (8 two-byte loads;
//      rows and columns outside the image and channels past C read zero
//      through out-of-range buffer offsets);
//   2. row pass: t[r][j] = chain_i Bh[i][r] * d[i][j]          (r = 0..7);
//   3. transposes t through LDS within its 8-lane group;
//   4. column pass as lane (cl, r = j): v[r][s] = chain_j t[r][j] * Bh[j][s];
//   5. stores positions 8r .. 8r+7 (lanes over channels: 16-byte runs).
// The chains are those of input_tile_rows, so V is bit-identical to the
// one-patch-per-thread kernel. Workgroup = 4 waves = 32 channels of a tile.
// ---------------------------------------------------------------------------
constexpr int kLpPitch = 72;  // floats per channel in the transpose buffer

template <bool kNhwc, int kPol>
__global__ __launch_bounds__(256) void input_lp_kernel(const _Float16* __restrict__ x,
                                                       _Float16* __restrict__ V, int C, int H,
                                                       int W, int pad, int nh, int nw, int ldv,
                                                       int64_t pstride, int ncg, int x_bytes,
                                                       int64_t v_bytes, int vfrag, int nwg) {
    __shared__ float tls[4 * 8 * kLpPitch];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int j = lane & 7, cl = lane >> 3;
    const int item = xcd_remap(blockIdx.x, nwg);  // (tile bp, 32-channel group)
    const int bp = item / ncg;
    const int c = (item - bp * ncg) * 32 + wv * 8 + cl;
    const int tw = bp % nw;
    const int th = (bp / nw) % nh;
    const int b = bp / (nw * nh);
    const int h0 = 6 * th - pad, w = 6 * tw - pad + j;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, x_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, v_bytes);

    const bool ok = c < C && w >= 0 && w < W;
    // element (b, c, h, w): NCHW ((b*C + c)*H + h)*W + w, NHWC ((b*H + h)*W + w)*C + c
    const int cc = ok ? c : 0, ww = ok ? w : 0;
    const int base = kNhwc ? 2 * ((b * H * W + ww) * C + cc) : 2 * ((b * C + cc) * H * W + ww);
    const int rstep = kNhwc ? 2 * W * C : 2 * W;
    float d[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int h = h0 + i;
        const int off = (ok && h >= 0 && h < H) ? base + h * rstep : kOob;
        d[i] = (float)__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(
                                                       xrs, off, 0, 0));
    }
    const float one = opaque_one();
    float* tp = tls + (wv * 8 + cl) * kLpPitch;
#pragma unroll
    for (int r = 0; r < 8; r++) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (kBh[i][r] != 0.0f) acc = __builtin_fmaf(mix_coef(kBh[i][r], one), d[i], acc);
        tp[r * 8 + j] = acc;
    }
    __syncthreads();
    float t[8];
#pragma unroll
    for (int q = 0; q < 8; q++) t[q] = tp[j * 8 + q];
    const int voff = c < ldv ? 2 * (int)(8 * j * pstride) + v_plane_off(bp, c, ldv, vfrag) : kOob;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (kBh[q][s] != 0.0f) acc = __builtin_fmaf(t[q], kBh[q][s], acc);
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, to_f16(acc)), vrs,
                                              voff, (int)(2 * s * pstride), kPol);
    }
}

static hipError_t launch_input_lp(const uint16_t* x, uint16_t* V, int B, int C, int H, int W,
                                  int pad, int nh, int nw, int ldv, int64_t pstride,
                                  hipStream_t s, bool nhwc, int vfrag) {
    const int ncg = (ldv + 31) / 32;
    const int64_t items = (int64_t)B * nh * nw * ncg;
    if (items >= ((int64_t)1 << 31)) return hipErrorInvalidConfiguration;
    const int64_t x_bytes = 2 * (int64_t)B * C * H * W;
    if (x_bytes >= ((int64_t)1 << 31) - 64) return hipErrorInvalidValue;
    // a wave's stores are 16-byte pieces of 8 lines: written through the L2
    // only while V is small (whole forwards in a graph, us: conv4_x batch 1
    // 9.22 -> 9.00, conv5_x 11.71 -> 11.46, SD-1.5 1280@8^2 batch 2 (1.3 MB)
    // 38.7 -> 38.4; at 2.5-5.9 MB it lost 0.5-2 us)
    const bool wt = 2 * 64 * pstride <= kWTSmallBytes;
    auto go = [&](auto kernel) {
        launch_n(kernel, dim3((unsigned)items), dim3(256), s,
                 reinterpret_cast<const _Float16*>(x), reinterpret_cast<_Float16*>(V), C, H, W,
                 pad, nh, nw, ldv, pstride, ncg, (int)x_bytes, 2 * 64 * pstride, vfrag);
    };
    if (nhwc)
        wt ? go(input_lp_kernel<true, kWT>) : go(input_lp_kernel<true, 0>);
    else
        wt ? go(input_lp_kernel<false, kWT>) : go(input_lp_kernel<false, 0>);
    return hipGetLastError();
}

// Tile-block width for a transform over rows x n tile columns and ch
// channels with 256/TW channels per workgroup. Small problems (the widest
// grid still under 256 workgroups, e.g. batch 1) take the widest grid, since
// their time is one workgroup's latency; otherwise the least padded work,
// ties to the wider block.
static int pick_tw(int64_t rows, int n, int ch) {
    int best = 8, widest = 8;
    int64_t best_w = -1, widest_g = -1;
    for (int tw = 8; tw >= 2; tw /= 2) {
        const int cb = 256 / tw;
        const int64_t nb = (int64_t)((n + tw - 1) / tw) * ((ch + cb - 1) / cb);
        const int64_t w = nb * tw * cb;
        if (best_w < 0 || w < best_w) {
            best_w = w;
            best = tw;
        }
        if (nb * rows > widest_g) {
            widest_g = nb * rows;
            widest = tw;
        }
    }
    return widest_g < 256 ? widest : best;
}

// ---------------------------------------------------------------------------
// Input transform into the two-pass block layout, run form. The tile-block
// kernel above covers tiles of one tile row, so each 128-byte line of a V
// block (8 consecutive tiles x 8 channels of one position) collects its
// 16-byte pieces from several workgroups and has to merge in the L2. Here a
// workgroup takes 16 consecutive tiles (bp, across tile rows and images:
// one block column) x 16 channels; wave w holds tiles 8*(w & 1) .. +7 x
// channels 8*(w >> 1) .. +7 of them, lane = (tile % 8, channel % 8), so each
// store instruction writes one whole line of a position's block (written
// through the L2, kWT). Each thread loads its patch's 8 rows straight
// from global memory (a 16-byte and a 4-byte load from the dword at or below
// the row start, shifted by 0 or 2 bytes; rows outside the image and
// channels past C read zero; a row starting before x_al, only the tensor's
// first row with left padding, is loaded from 0 and shifted into place),
// masks the columns outside the image and runs the shared chains: V is the
// tile-block kernel's, bit for bit. NCHW only.
// ---------------------------------------------------------------------------
template <int kPol>
__global__ __launch_bounds__(256) void input_run_kernel(
    const void* __restrict__ x_al, _Float16* __restrict__ V, int C, int Cp, int H, int W,
    int pad, int nw, int P, int BP, int ncg, int vfrag, int64_t pstride, int x_bytes, int xd,
    int64_t v_bytes, int nwg) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int L = xcd_remap(blockIdx.x, nwg);
    const int cg = L % ncg, blk = L / ncg;
    const int c = cg * 16 + 8 * (wave >> 1) + (lane & 7);
    const int t = 8 * (wave & 1) + (lane >> 3);
    const int bp = blk * 16 + t;
    if (bp >= BP || c >= Cp) return;  // nothing to store (no barrier in this kernel)
    const int b = bp / P, tr = bp - (bp / P) * P;
    const int th = tr / nw, tw = tr - (tr / nw) * nw;
    const int h0 = 6 * th - pad, w0 = 6 * tw - pad;
    const int HW = H * W;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x_al, x_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, v_bytes);
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    unsigned w5[8][5];
    unsigned odd = 0, neg = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int h = h0 + i;
        const bool ok = c < C && h >= 0 && h < H;
        const int o = xd + 2 * ((b * C + c) * HW + h * W + w0);
        odd |= (unsigned)((o >> 1) & 1) << i;
        neg |= (ok && o < 0) ? (1u << i) : 0u;
        const int A = !ok ? kOob : (o < 0 ? 0 : (o & ~3));
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, A, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; q++) w5[i][q] = v[q];
        w5[i][4] = __builtin_amdgcn_raw_buffer_load_b32(xrs, A + 16, 0, 0);
    }
    if (neg != 0) {
        // rows loaded from 0 instead of up to 8 bytes (pads up to 4) before
        // x_al: move their dwords up by the missing ones (the zeros land in
        // masked columns)
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (!((neg >> i) & 1u)) continue;
            const int o = xd + 2 * ((b * C + c) * HW + (h0 + i) * W + w0);
            const int sh = -(o >> 2);
            unsigned l5[5];
#pragma unroll
            for (int q = 0; q < 5; q++) l5[q] = w5[i][q];
#pragma unroll
            for (int q = 0; q < 5; q++) {
                unsigned v = 0;
#pragma unroll
                for (int rr = 0; rr < 5; rr++) v = (q - sh == rr) ? l5[rr] : v;
                w5[i][q] = v;
            }
        }
    }
    unsigned cmask = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int w = w0 + j;
        cmask |= (w >= 0 && w < W) ? (1u << j) : 0u;
    }
    unsigned d4[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const unsigned sb = ((odd >> i) & 1u) * 2;
#pragma unroll
        for (int q = 0; q < 4; q++) d4[i][q] = __builtin_amdgcn_alignbyte(w5[i][q + 1], w5[i][q], sb);
    }
    if (cmask != 0xffu) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const unsigned m = (((cmask >> (2 * q)) & 1u) ? 0xffffu : 0u) |
                               (((cmask >> (2 * q + 1)) & 1u) ? 0xffff0000u : 0u);
#pragma unroll
            for (int i = 0; i < 8; i++) d4[i][q] &= m;
        }
    }
    const int voff = v_plane_off(bp, c, Cp, vfrag);
    input_tile_rows(
        [&](int i, int j) {
            const unsigned pair = d4[i][j >> 1];
            const unsigned short bits = (unsigned short)((j & 1) ? (pair >> 16) : (pair & 0xffffu));
            return (float)__builtin_bit_cast(_Float16, bits);
        },
        [&](int r, int s2, float v) {
            const int p = r * 8 + s2;
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, to_f16(v)), vrs,
                                                  voff, (int)(2 * p * pstride), kPol);
        });
}

static hipError_t launch_input_run(const uint16_t* x, uint16_t* V, int B, int C, int H, int W,
                                   int pad, int nh, int nw, int ldv, int64_t pstride,
                                   hipStream_t s, int vfrag) {
    const int P = nh * nw;
    const int64_t BP = (int64_t)B * P;
    const int ncg = (ldv + 15) / 16;
    const int64_t nblocks = ((BP + 15) / 16) * ncg;
    if (nblocks >= ((int64_t)1 << 31) || BP >= ((int64_t)1 << 31) || pad > 4)
        return hipErrorInvalidConfiguration;
    const uintptr_t xp = reinterpret_cast<uintptr_t>(x);
    const int xd = (int)(xp & 15);
    const int64_t x_bytes = dword_ceil(2 * (int64_t)B * C * H * W + xd);
    if (x_bytes >= ((int64_t)1 << 31) - 64) return hipErrorInvalidValue;
    const void* xa = reinterpret_cast<const void*>(xp - (uintptr_t)xd);
    auto go = [&](auto kernel) {
        launch_n(kernel, dim3((unsigned)nblocks), dim3(256), s, xa, reinterpret_cast<_Float16*>(V),
               C, ldv, H, W, pad, nw, P, (int)BP, ncg, vfrag, pstride, (int)x_bytes, xd,
               2 * 64 * pstride);
    };
    go(input_run_kernel<kWT>);
    return hipGetLastError();
}

// Small problems (the tile-block grid under 256 workgroups, e.g. batch 1)
// are latency-bound: they take the lane-parallel transforms, whose threads
// run an eighth of the instruction chain. Large ones keep the tile-block
// kernels, which issue half as many memory instructions per patch (measured
// on MI355X: lane-parallel input 5.5 us vs 6.8 us for ResNet-50 conv2_x at
// batch 1, 20.2 us vs 14.0 us at batch 32).
static int64_t widest_grid(int64_t rows, int n, int ch) {
    int64_t widest_g = 0;
    for (int tw = 8; tw >= 2; tw /= 2) {
        const int cb = 256 / tw;
        widest_g = std::max(widest_g, (int64_t)((n + tw - 1) / tw) * ((ch + cb - 1) / cb) * rows);
    }
    return widest_g;
}
static bool latency_bound(int64_t rows, int n, int ch) { return widest_grid(rows, n, ch) < 256; }

hipError_t launch_input_transform(const uint16_t* x, uint16_t* V, int B, int C, int H, int W,
                                  int pad, int nh, int nw, int ldv, int64_t pstride,
                                  hipStream_t s, bool nhwc, bool stream_v, int vfrag) {
    // The two-pass block layout from the run form when its grid fills the
    // CUs (whole forwards in a graph, us, tile-block vs run form: conv3_x
    // batch 32 24.25 vs 23.41 (input transform 8.78 vs 7.77), batch 24 22.75
    // vs 21.94; 96@28^2 batch 32 19.91 vs 18.85; 48->40@13^2 batch 128 17.09
    // vs 15.92; 128->256@14^2 batch 32 (144 workgroups) 21.18 vs 21.03; with
    // few workgroups it loses: 128@28^2 batch 3 (40) 17.49 vs 18.44). Its
    // whole-line V stores write through the L2 (kWT): conv3_x batch 32 23.69
    // -> 22.39 us in a graph (streamed with nt instead, the input transform
    // ran 1 us faster but the products 1.4 us slower).
    if (!nhwc && vfrag > 0 && pad <= 4 &&
        ((int64_t)B * nh * nw + 15) / 16 * ((ldv + 15) / 16) >= 256)
        return launch_input_run(x, V, B, C, H, W, pad, nh, nw, ldv, pstride, s, vfrag);
    if (latency_bound((int64_t)B * nh, nw, ldv) ||
        (nhwc && (C % 8 != 0 || (reinterpret_cast<uintptr_t>(x) & 15) != 0)))
        return launch_input_lp(x, V, B, C, H, W, pad, nh, nw, ldv, pstride, s, nhwc, vfrag);
    const int tw = pick_tw((int64_t)B * nh, nw, ldv);
    const int cb = 256 / tw;
    const int cblocks = (ldv + cb - 1) / cb;
    const int64_t nblocks = (int64_t)((nw + tw - 1) / tw) * nh * B * cblocks;
    if (nblocks >= ((int64_t)1 << 31)) return hipErrorInvalidConfiguration;
    const dim3 grid((unsigned)nblocks), block(256);
    _Float16* Vh = reinterpret_cast<_Float16*>(V);
    // V stores: a wave writes 64 consecutive channels of one (tile,
    // position) -- whole 128-byte lines in the product layout when the
    // workgroup holds at least 64 channels and rows are whole lines -- written
    // through the L2 (kWT); otherwise nt when the GEMM reads V few times
    // (stream_v), else write-back. Whole forwards in a graph, us, before ->
    // after: ResNet-50 batch 32 256@14^2 25.75 -> 24.49, 512@7^2 25.42 ->
    // 23.24; batch 128 256@14^2 49.4 -> 45.8; SD-1.5 320@64^2 batch 2 28.3 ->
    // 25.7, 640->320@64^2 34.2 -> 31.7; SDXL 320@128^2 38.0 -> 35.3.
    const bool whole_lines = vfrag == 0 && tw <= 4 && ldv % 64 == 0;
    const int pol = whole_lines ? kWT : stream_v ? kNt : 0;
    auto by_policy = [&](auto tw_c, auto go) {
        constexpr int T = decltype(tw_c)::value;
        if (pol == kWT)
            go(std::integral_constant<int, T>(), std::integral_constant<int, kWT>());
        else if (pol == kNt)
            go(std::integral_constant<int, T>(), std::integral_constant<int, kNt>());
        else
            go(std::integral_constant<int, T>(), std::integral_constant<int, 0>());
    };
    auto by_tw = [&](auto go) {
        if (tw == 2)
            by_policy(std::integral_constant<int, 2>(), go);
        else if (tw == 4)
            by_policy(std::integral_constant<int, 4>(), go);
        else
            by_policy(std::integral_constant<int, 8>(), go);
    };
    if (nhwc) {
        const int64_t x_bytes = 2 * (int64_t)B * C * H * W;
        if (x_bytes >= ((int64_t)1 << 31) - 64) return hipErrorInvalidValue;
        const _Float16* xh = reinterpret_cast<const _Float16*>(x);
        by_tw([&](auto tw_c, auto pol_c) {
            launch_n(input_nhwc_kernel<decltype(tw_c)::value, decltype(pol_c)::value>, grid, block,
                     s, xh, Vh, C, H, W, pad, nh, nw, ldv, pstride, cblocks, (int)x_bytes,
                     2 * 64 * pstride, vfrag);
        });
        return hipGetLastError();
    }
    // x is addressed from the 16-byte boundary at or below it (same granule,
    // so no byte outside x's pages is touched); offsets stay 32-bit.
    const uintptr_t xp = reinterpret_cast<uintptr_t>(x);
    const int xd = (int)(xp & 15);
    const int64_t x_bytes = dword_ceil(2 * (int64_t)B * C * H * W + xd);
    if (x_bytes >= ((int64_t)1 << 31) - 64) return hipErrorInvalidValue;
    const void* xa = reinterpret_cast<const void*>(xp - (uintptr_t)xd);
    by_tw([&](auto tw_c, auto pol_c) {
        launch_n(input_transform_kernel<decltype(tw_c)::value, decltype(pol_c)::value>, grid,
                 block, s, xa, Vh, C, H, W, pad, nh, nw, ldv, pstride, cblocks, (int)x_bytes, xd,
                 2 * 64 * pstride, vfrag);
    });
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Output transform.
// Workgroup (256 threads) = one tile row x TW tiles x 256/TW output channels of
// one image (TW picked per layer like the input transform). Each thread reads
// the 64 positions of one (tile, k) (lanes over consecutive k: coalesced;
// position stride as a scalar offset) and computes its 6x6 tile into LDS; the
// workgroup then writes whole output row segments of kVW halves per store
// (kVW = 4, 2 or 1, the widest the output row pitch and base alignment allow).
// A segment cut by the right edge of the image is stored one half at a time;
// rows past Ho and channels past K are skipped.
// ---------------------------------------------------------------------------
template <int TW>
struct OutGeom {
    static constexpr int kKB = 256 / TW;          // output channels per workgroup
    static constexpr int kCols = TW * 6;          // output columns per block
    // halves per channel: with 8-byte segments (kVW = 4) a multiple of 4
    // (2-way write conflicts, lanes over consecutive channels); otherwise an
    // odd number of dwords, so the 64 lanes of a write hit 64 banks
    template <int kVW>
    static constexpr int plane() { return kVW == 4 ? 6 * kCols + 4 : 6 * kCols + 2; }
};

template <int TW, int kVW, bool kEpi>
__global__ __launch_bounds__(256) void output_transform_kernel(
    const _Float16* __restrict__ M, _Float16* __restrict__ y, int K, int Ho, int Wo, int nh,
    int nw, int ldm, int64_t pstride, int kblocks, int64_t m_bytes, int64_t y_bytes,
    const _Float16* __restrict__ bias, int relu, const _Float16* __restrict__ res, int nwg) {
    using G = OutGeom<TW>;
    constexpr int kPlane = G::template plane<kVW>();
    __shared__ __align__(16) _Float16 sy[G::kKB * kPlane];
    const int nwb = (nw + TW - 1) / TW;
    const int L = xcd_remap(blockIdx.x, nwg);
    const int tw0 = (L % nwb) * TW;
    const int th = (L / nwb) % nh;
    const int bz = L / (nwb * nh);
    const int b = bz / kblocks;
    const int k0 = (bz % kblocks) * G::kKB;
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(M, m_bytes);
    const __amdgpu_buffer_rsrc_t yrs = make_rsrc(y, y_bytes);

    // slots past the last tile or channel skip the transform (the store
    // phase never reads their LDS rows); whole idle waves wait at the barrier
    // without issuing
    if (tw0 + (int)threadIdx.x / G::kKB < nw && k0 + (int)threadIdx.x % G::kKB < K) {
        const int kk = threadIdx.x % G::kKB;
        const int t = threadIdx.x / G::kKB;
        const int tw = tw0 + t;
        const int k = k0 + kk;
        const int bp = (b * nh + th) * nw + tw;
        const int moff = 2 * (bp * ldm + k);
        uint16_t m[64];
#pragma unroll
        for (int p = 0; p < 64; p++)
            m[p] = __builtin_amdgcn_raw_buffer_load_b16(mrs, moff, (int)(2 * p * pstride), 0);
        float out[6][6];
        output_tile([&](int i, int j) { return (float)__builtin_bit_cast(_Float16, m[i * 8 + j]); },
                    out);
        _Float16* sp = sy + kk * kPlane + t * 6;
        const ChannelEpilogue<kEpi> epi(bias, k, res ? 0 : relu);
#pragma unroll
        for (int r = 0; r < 6; r++)
#pragma unroll
            for (int s = 0; s < 6; s++) sp[r * G::kCols + s] = epi(out[r][s]);
    }
    __syncthreads();

    // ---- store: e = (channel kk, row r, segment of kVW halves) ----
    const int nkk = min(G::kKB, K - k0);              // uniform
    const int ncols = min(G::kCols, Wo - tw0 * 6);    // uniform
    const int h0 = th * 6;
    const int nr = min(6, Ho - h0);                   // uniform
    const int nseg = (ncols + kVW - 1) / kVW;         // uniform
    const int per_k = nr * nseg;
    const int total = nkk * per_k;
    const int ybase = 2 * (((b * K + k0) * Ho + h0) * Wo + tw0 * 6);  // byte offset
    // e advances by 256: decode once, then step (kk, r, sg) by carries
    int e = threadIdx.x;
    int kk = e / per_k;
    int rem = e - kk * per_k;
    int r = rem / nseg;
    int sg = rem - r * nseg;
    const int dk = 256 / per_k, drem = 256 - dk * per_k;
    const int dr = drem / nseg, ds = drem - dr * nseg;
    // residual (same layout as y): added per stored segment, then the ReLU
    const __amdgpu_buffer_rsrc_t rrs = make_rsrc(res, res ? y_bytes : 0);
    for (; e < total; e += 256) {
        const _Float16* src = sy + kk * kPlane + r * G::kCols + sg * kVW;
        const int off = ybase + 2 * ((kk * Ho + r) * Wo + sg * kVW);
        if (sg * kVW + kVW <= ncols) {
            if constexpr (kVW == 4) {
                typedef unsigned u2 __attribute__((ext_vector_type(2)));
                u2 v = *reinterpret_cast<const u2*>(src);
                if (res) {
                    const u2 rv = __builtin_bit_cast(
                        u2, __builtin_amdgcn_raw_buffer_load_b64(rrs, off, 0, 0));
                    v = u2{add_residual2(v[0], rv[0], relu), add_residual2(v[1], rv[1], relu)};
                }
                __builtin_amdgcn_raw_buffer_store_b64(v, yrs, off, 0, 0);
            } else if constexpr (kVW == 2) {
                unsigned v = *reinterpret_cast<const unsigned*>(src);
                if (res) v = add_residual2(v, __builtin_amdgcn_raw_buffer_load_b32(rrs, off, 0, 0),
                                           relu);
                __builtin_amdgcn_raw_buffer_store_b32(v, yrs, off, 0, 0);
            } else {
                _Float16 v = *src;
                if (res)
                    v = add_residual(v, __builtin_bit_cast(_Float16,
                                                           __builtin_amdgcn_raw_buffer_load_b16(
                                                               rrs, off, 0, 0)),
                                     relu);
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs, off,
                                                      0, 0);
            }
        } else {
            for (int q = 0; sg * kVW + q < ncols; q++) {
                _Float16 v = src[q];
                if (res)
                    v = add_residual(v, __builtin_bit_cast(_Float16,
                                                           __builtin_amdgcn_raw_buffer_load_b16(
                                                               rrs, off + 2 * q, 0, 0)),
                                     relu);
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs,
                                                      off + 2 * q, 0, 0);
            }
        }
        sg += ds;
        r += dr;
        kk += dk;
        if (sg >= nseg) {
            sg -= nseg;
            r++;
        }
        if (r >= nr) {
            r -= nr;
            kk++;
        }
    }
}

// ---------------------------------------------------------------------------
// Output transform, NHWC (channels-last) y, tile-block form: thread (tile, k)
// reads its 64 positions as in the NCHW kernel and stores its 36 outputs
// straight to y[b][h][w][k] -- lanes over consecutive k, so every store
// instruction writes 128 contiguous bytes and no LDS transpose is needed.
// The epilogue (bias, residual in y's layout, ReLU) is applied per value.
// ---------------------------------------------------------------------------
template <int TW, bool kEpi>
__global__ __launch_bounds__(256) void output_nhwc_kernel(
    const _Float16* __restrict__ M, _Float16* __restrict__ y, int K, int Ho, int Wo, int nh,
    int nw, int ldm, int64_t pstride, int kblocks, int64_t m_bytes, int64_t y_bytes,
    const _Float16* __restrict__ bias, int relu, const _Float16* __restrict__ res, int nwg) {
    constexpr int kKB = 256 / TW;
    const int nwb = (nw + TW - 1) / TW;
    const int L = xcd_remap(blockIdx.x, nwg);
    const int tw0 = (L % nwb) * TW;
    const int th = (L / nwb) % nh;
    const int bz = L / (nwb * nh);
    const int b = bz / kblocks;
    const int k0 = (bz % kblocks) * kKB;
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(M, m_bytes);
    const __amdgpu_buffer_rsrc_t yrs = make_rsrc(y, y_bytes);
    const __amdgpu_buffer_rsrc_t rrs = make_rsrc(res, res ? y_bytes : 0);
    const int kk = threadIdx.x % kKB;
    const int t = threadIdx.x / kKB;
    const int tw = tw0 + t;
    const int k = k0 + kk;
    if (tw >= nw || k >= K) return;
    const int bp = (b * nh + th) * nw + tw;
    const int moff = 2 * (bp * ldm + k);
    uint16_t m[64];
#pragma unroll
    for (int p = 0; p < 64; p++)
        m[p] = __builtin_amdgcn_raw_buffer_load_b16(mrs, moff, (int)(2 * p * pstride), 0);
    float out[6][6];
    output_tile([&](int i, int j) { return (float)__builtin_bit_cast(_Float16, m[i * 8 + j]); },
                out);
    const int oh = 6 * th, ow = 6 * tw;
    const ChannelEpilogue<kEpi> epi(bias, k, res ? 0 : relu);
#pragma unroll
    for (int r = 0; r < 6; r++) {
        if (oh + r >= Ho) break;
#pragma unroll
        for (int s2 = 0; s2 < 6; s2++) {
            if (ow + s2 >= Wo) break;
            const int off = 2 * (((b * Ho + oh + r) * Wo + ow + s2) * K + k);
            _Float16 v = epi(out[r][s2]);
            if (res)
                v = add_residual(
                    v,
                    __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rrs, off, 0, 0)),
                    relu);
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs, off, 0, 0);
        }
    }
}

// ---------------------------------------------------------------------------
// Output transform, image-block form (NCHW, small images at batch): workgroup
// = one image x KB consecutive output channels x all P tiles of the image, so
// its outputs are one contiguous span of y (KB whole channel planes). Thread e
// < P * KB takes (channel e % KB, tile e / KB): it reads the 64 positions (lanes
// over consecutive channels), runs the chains of output_tile and writes the
// in-image outputs into LDS as the span's image; the workgroup then stores the
// span as 16-byte pieces (whole lines written through the L2 when the span is
// line-aligned: the next launch has no dirty y to write back first).
// ---------------------------------------------------------------------------
template <bool kEpi, int kPol>
__global__ __launch_bounds__(512) void output_image_kernel(const _Float16* __restrict__ M, _Float16* __restrict__ y,
                                    int K, int Ho, int Wo, int nh, int nw, int KB, int nkb,
                                    int64_t pstride, int64_t m_bytes, int64_t y_bytes,
                                    const _Float16* __restrict__ bias, int relu,
                                    const _Float16* __restrict__ res, int nthr, int nwg) {
    extern __shared__ __align__(16) _Float16 sy[];  // KB planes of Ho x Wo halves
    const int P = nh * nw;
    const int L = xcd_remap(blockIdx.x, nwg);
    const int b = L / nkb;
    const int k0 = (L - b * nkb) * KB;
    const int nk = min(KB, K - k0);  // channels of this span
    const int plane = Ho * Wo;
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(M, m_bytes);
    const __amdgpu_buffer_rsrc_t yrs = make_rsrc(y, y_bytes);
    const int e = threadIdx.x;
    const int kk = e % KB, t = e / KB;
    if (t < P && kk < nk) {
        const int th = t / nw, tw = t - th * nw;
        const int k = k0 + kk;
        const int moff = 2 * ((b * P + t) * K + k);
        uint16_t m[64];
#pragma unroll
        for (int p = 0; p < 64; p++)
            m[p] = __builtin_amdgcn_raw_buffer_load_b16(mrs, moff, (int)(2 * p * pstride), 0);
        float out[6][6];
        output_tile([&](int i, int j) { return (float)__builtin_bit_cast(_Float16, m[i * 8 + j]); },
                    out);
        const ChannelEpilogue<kEpi> epi(bias, k, res ? 0 : relu);
        _Float16* sp = sy + kk * plane + (6 * th) * Wo + 6 * tw;
#pragma unroll
        for (int r = 0; r < 6; r++) {
            if (6 * th + r >= Ho) break;
#pragma unroll
            for (int s2 = 0; s2 < 6; s2++)
                if (6 * tw + s2 < Wo) sp[r * Wo + s2] = epi(out[r][s2]);
        }
    }
    __syncthreads();

    // ---- store the span as 16-byte pieces (a multiple of 16 bytes: K and KB
    // planes are, output_image_kb) ----
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    const int span = 2 * nk * plane;  // bytes
    const int ybase = 2 * (b * K + k0) * plane;
    const __amdgpu_buffer_rsrc_t rrs = make_rsrc(res, res ? y_bytes : 0);
    const int n16 = span >> 4;
    for (int c = e; c < n16; c += nthr) {
        u4 v = *reinterpret_cast<const u4*>(reinterpret_cast<const unsigned char*>(sy) + 16 * c);
        if (res) {
            const u4 rv =
                __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rrs, ybase + 16 * c, 0, 0));
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] = add_residual2(v[q], rv[q], relu);
        }
        __builtin_amdgcn_raw_buffer_store_b128(v, yrs, ybase + 16 * c, 0, kPol);
    }
}

// The image-block form when its span layout fits: NCHW, at most 512 (tile,
// channel) pairs per workgroup with at least 16 channels, a grid that fills
// the CUs, spans of 16-byte multiples (K and KB channel planes, so every
// span, the last channel block's included) from a 16-byte aligned y (and
// residual), at most 48 KB of LDS. Returns the channels per workgroup, or 0.
static int output_image_kb(int B, int K, int Ho, int Wo, int nh, int nw, int cus, const void* y,
                           const void* res) {
    const int P = nh * nw;
    const int64_t plane2 = 2 * (int64_t)Ho * Wo;
    if (((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(res)) & 15) != 0 ||
        (K * plane2) % 16 != 0)
        return 0;
    for (int kb = 64; kb >= 16; kb /= 2) {
        const int64_t grid = (int64_t)B * ((K + kb - 1) / kb);
        if (P * kb <= 512 && grid >= cus && (kb * plane2) % 16 == 0 && kb * plane2 <= 48 * 1024)
            return kb;
    }
    return 0;
}

template <int TW>
static void launch_out_tw(int vw, bool epi, dim3 grid, hipStream_t s, const _Float16* Mh,
                          _Float16* yh, int K, int Ho, int Wo, int nh, int nw, int ldm,
                          int64_t pstride, int kblocks, int64_t m_bytes, int64_t y_bytes,
                          const _Float16* bias, int relu, const _Float16* res) {
    const dim3 block(256);
    auto go = [&](auto kernel) {
        launch_n(kernel, grid, block, s, Mh, yh, K, Ho, Wo, nh, nw, ldm, pstride, kblocks, m_bytes,
               y_bytes, bias, relu, res);
    };
    if (epi) {
        if (vw == 4)
            go(output_transform_kernel<TW, 4, true>);
        else if (vw == 2)
            go(output_transform_kernel<TW, 2, true>);
        else
            go(output_transform_kernel<TW, 1, true>);
    } else {
        if (vw == 4)
            go(output_transform_kernel<TW, 4, false>);
        else if (vw == 2)
            go(output_transform_kernel<TW, 2, false>);
        else
            go(output_transform_kernel<TW, 1, false>);
    }
}

// ---------------------------------------------------------------------------
// Output transform, lane-parallel form (small problems): 8 lanes per (tile,
// output channel). Lane (channel kl, column j) loads column j of the 8x8 M
// patch (positions j, 8+j, ..., 56+j; lanes over channels), runs the row pass
// t[r][j] = chain_i Ah[r][i] * m[i][j] (r < 6), transposes t through LDS and,
// as lane (kl, r = j < 6), runs the column pass y[r][s] = chain_j t[r][j] *
// Ah[s][j] -- the chains of output_tile -- then the epilogue, and stores
// output row r of the tile (three 4-byte pairs when the row pitch and y allow,
// else six halves; rows past Ho and columns past Wo are skipped).
// Workgroup = 4 waves = 32 output channels of one tile.
// ---------------------------------------------------------------------------
template <bool kNhwc, bool kEpi>
__global__ __launch_bounds__(256) void output_lp_kernel(
    const _Float16* __restrict__ M, _Float16* __restrict__ y, int K, int Ho, int Wo, int nh,
    int nw, int ldm, int64_t pstride, int nkg, int64_t m_bytes, int64_t y_bytes, int pairs,
    const _Float16* __restrict__ bias, int relu, const _Float16* __restrict__ res, int nwg) {
    __shared__ float tls[4 * 8 * kLpPitch];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int j = lane & 7, kl = lane >> 3;
    const int item = xcd_remap(blockIdx.x, nwg);  // (tile bp, 32-channel group)
    const int bp = item / nkg;
    const int k = (item - bp * nkg) * 32 + wv * 8 + kl;
    const int tw = bp % nw;
    const int th = (bp / nw) % nh;
    const int b = bp / (nw * nh);
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(M, m_bytes);
    const __amdgpu_buffer_rsrc_t yrs = make_rsrc(y, y_bytes);

    const int moff = k < K ? 2 * (int)(j * pstride + (int64_t)bp * ldm + k) : kOob;
    float m[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        m[i] = (float)__builtin_bit_cast(
            _Float16, __builtin_amdgcn_raw_buffer_load_b16(mrs, moff, (int)(16 * i * pstride), 0));
    const float one = opaque_one();
    float* tp = tls + (wv * 8 + kl) * kLpPitch;
#pragma unroll
    for (int r = 0; r < 6; r++) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (kAh[r][i] != 0.0f) acc = __builtin_fmaf(mix_coef(kAh[r][i], one), m[i], acc);
        tp[r * 8 + j] = acc;
    }
    __syncthreads();
    const int r = j;  // output row of this lane in the column pass
    const int oh = 6 * th + r;
    if (r < 6 && k < K && oh < Ho) {
        float t[8];
#pragma unroll
        for (int q = 0; q < 8; q++) t[q] = tp[r * 8 + q];
        _Float16 out[6];
        const ChannelEpilogue<kEpi> epi(bias, k, res ? 0 : relu);
#pragma unroll
        for (int s2 = 0; s2 < 6; s2++) {
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (kAh[s2][q] != 0.0f) acc = __builtin_fmaf(t[q], kAh[s2][q], acc);
            out[s2] = epi(acc);
        }
        const int ow = 6 * tw;
        const __amdgpu_buffer_rsrc_t rrs = make_rsrc(res, res ? y_bytes : 0);
        if (kNhwc) {
            // y[b][oh][ow + s][k]: lanes over channels, one half per pixel
            const int pix = 2 * (((b * Ho + oh) * Wo + ow) * K + k);
#pragma unroll
            for (int s2 = 0; s2 < 6; s2++)
                if (ow + s2 < Wo) {
                    const int off = pix + 2 * s2 * K;
                    _Float16 v = out[s2];
                    if (res)
                        v = add_residual(v,
                                         __builtin_bit_cast(_Float16,
                                                            __builtin_amdgcn_raw_buffer_load_b16(
                                                                rrs, off, 0, 0)),
                                         relu);
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs, off,
                                                          0, 0);
                }
            return;
        }
        const int row = 2 * (((b * K + k) * Ho + oh) * Wo + ow);
        if (pairs) {
#pragma unroll
            for (int s2 = 0; s2 < 6; s2 += 2)
                if (ow + s2 < Wo) {
                    unsigned v = (unsigned)__builtin_bit_cast(uint16_t, out[s2]) |
                                 ((unsigned)__builtin_bit_cast(uint16_t, out[s2 + 1]) << 16);
                    if (res)
                        v = add_residual2(
                            v, __builtin_amdgcn_raw_buffer_load_b32(rrs, row + 2 * s2, 0, 0),
                            relu);
                    __builtin_amdgcn_raw_buffer_store_b32(v, yrs, row + 2 * s2, 0, 0);
                }
        } else {
#pragma unroll
            for (int s2 = 0; s2 < 6; s2++)
                if (ow + s2 < Wo) {
                    _Float16 v = out[s2];
                    if (res)
                        v = add_residual(v,
                                         __builtin_bit_cast(_Float16,
                                                            __builtin_amdgcn_raw_buffer_load_b16(
                                                                rrs, row + 2 * s2, 0, 0)),
                                         relu);
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), yrs,
                                                          row + 2 * s2, 0, 0);
                }
        }
    }
}

static hipError_t launch_output_lp(const uint16_t* M, uint16_t* y, int B, int K, int Ho, int Wo,
                                   int nh, int nw, int ldm, int64_t pstride, hipStream_t s,
                                   Epilogue ep, bool nhwc) {
    const int nkg = (K + 31) / 32;
    const int64_t items = (int64_t)B * nh * nw * nkg;
    if (items >= ((int64_t)1 << 31)) return hipErrorInvalidConfiguration;
    const int64_t y_bytes = 2 * (int64_t)B * K * Ho * Wo;
    if (y_bytes >= ((int64_t)1 << 31) - 64) return hipErrorInvalidValue;
    // 4-byte pairs: every pair starts at an even column of a row whose pitch
    // is even, in a 4-byte aligned y
    const int pairs = (Wo % 2 == 0 &&
                       ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(ep.residual)) &
                        3) == 0)
                          ? 1
                          : 0;
    auto go = [&](auto kernel) {
        launch_n(kernel, dim3((unsigned)items), dim3(256), s, reinterpret_cast<const _Float16*>(M),
               reinterpret_cast<_Float16*>(y), K, Ho, Wo, nh, nw, ldm, pstride, nkg,
               2 * 64 * pstride, y_bytes, pairs, reinterpret_cast<const _Float16*>(ep.bias),
               ep.relu, reinterpret_cast<const _Float16*>(ep.residual));
    };
    const bool epi = epilogue_needed(ep.bias, ep.relu, ep.residual);
    if (nhwc)
        epi ? go(output_lp_kernel<true, true>) : go(output_lp_kernel<true, false>);
    else
        epi ? go(output_lp_kernel<false, true>) : go(output_lp_kernel<false, false>);
    return hipGetLastError();
}

hipError_t launch_output_transform(const uint16_t* M, uint16_t* y, int B, int K, int Ho,
                                   int Wo, int nh, int nw, int ldm, int64_t pstride,
                                   hipStream_t s, Epilogue ep, bool nhwc) {
    // An odd output row pitch leaves the NCHW tile-block kernel one 2-byte
    // store per output; on images one or two tiles wide the lane-parallel
    // form then wins up to 640 workgroups (us, tile-block vs lane-parallel:
    // 512@7^2 batch 16 (512 workgroups) 7.0 vs 5.5, 256@7^2 batch 32 (512)
    // 7.1 vs 5.5, 512@7^2 batch 24 (768) 7.0 vs 6.9, batch 32 (1024) 7.0 vs
    // 8.7; five tiles wide, 130@27^2 batch 12 (300), it lost: 7.7 vs 8.2).
    const int64_t widest = widest_grid((int64_t)B * nh, nw, K);
    if (widest < 256 || (!nhwc && (Wo & 1) != 0 && nw <= 2 && widest < 640))
        return launch_output_lp(M, y, B, K, Ho, Wo, nh, nw, ldm, pstride, s, ep, nhwc);
    // Small images at batch (NCHW, the product layout): the image-block form
    // (whole forwards in a graph, us, tile-block -> image-block: ResNet-50
    // batch 32 256@14^2 24.96 -> 22.99, 512@7^2 23.38 -> 21.98; batch 128
    // 48.11 -> 45.29, 49.52 -> 46.17; 512@7^2 batch 64 30.48 -> 28.61;
    // 128->256@14^2 batch 32 20.40 -> 18.91; bit-identical)
    const int okb = (nhwc || ldm != K || pstride != (int64_t)K * B * nh * nw)
                        ? 0
                        : output_image_kb(B, K, Ho, Wo, nh, nw, 256, y, ep.residual);
    if (okb > 0) {
        const int P = nh * nw;
        const int nkb = (K + okb - 1) / okb;
        const int64_t nblocks = (int64_t)B * nkb;
        const int64_t y_bytes = 2 * (int64_t)B * K * Ho * Wo;
        if (nblocks >= ((int64_t)1 << 31) || y_bytes >= ((int64_t)1 << 31) - 64)
            return hipErrorInvalidValue;
        const int64_t plane2 = 2 * (int64_t)Ho * Wo;
        // whole 128-byte lines in every span: written through the L2
        const bool lines = (okb * plane2) % 128 == 0 && (K * plane2) % 128 == 0 &&
                           (reinterpret_cast<uintptr_t>(y) & 127) == 0;
        const dim3 grid((unsigned)nblocks), block((unsigned)((P * okb + 63) / 64 * 64));
        const size_t lds = (size_t)(okb * plane2);
        const _Float16* bias = reinterpret_cast<const _Float16*>(ep.bias);
        const _Float16* res = reinterpret_cast<const _Float16*>(ep.residual);
        auto go = [&](auto kernel) {
            launch_n_lds(kernel, grid, block, lds, s, reinterpret_cast<const _Float16*>(M),
                         reinterpret_cast<_Float16*>(y), K, Ho, Wo, nh, nw, okb, nkb, pstride,
                         2 * 64 * pstride, y_bytes, bias, ep.relu, res);
        };
        const bool epi = epilogue_needed(bias, ep.relu, res);
        if (lines)
            epi ? go(output_image_kernel<true, kWT>) : go(output_image_kernel<false, kWT>);
        else
            epi ? go(output_image_kernel<true, 0>) : go(output_image_kernel<false, 0>);
        return hipGetLastError();
    }
    if (nhwc) {
        const int tw = pick_tw((int64_t)B * nh, nw, K);
        const int kb = 256 / tw;
        const int kblocks = (K + kb - 1) / kb;
        const int64_t nblocks = (int64_t)((nw + tw - 1) / tw) * nh * B * kblocks;
        const int64_t y_bytes = 2 * (int64_t)B * K * Ho * Wo;
        if (nblocks >= ((int64_t)1 << 31)) return hipErrorInvalidConfiguration;
        if (y_bytes >= ((int64_t)1 << 31) - 64) return hipErrorInvalidValue;
        const _Float16* Mh = reinterpret_cast<const _Float16*>(M);
        _Float16* yh = reinterpret_cast<_Float16*>(y);
        const _Float16* bias = reinterpret_cast<const _Float16*>(ep.bias);
        const _Float16* res = reinterpret_cast<const _Float16*>(ep.residual);
        const dim3 grid((unsigned)nblocks), block(256);
        auto go = [&](auto kernel) {
            launch_n(kernel, grid, block, s, Mh, yh, K, Ho, Wo, nh, nw, ldm, pstride, kblocks,
                   2 * 64 * pstride, y_bytes, bias, ep.relu, res);
        };
        const bool epi = epilogue_needed(bias, ep.relu, res);
        if (tw == 2)
            epi ? go(output_nhwc_kernel<2, true>) : go(output_nhwc_kernel<2, false>);
        else if (tw == 4)
            epi ? go(output_nhwc_kernel<4, true>) : go(output_nhwc_kernel<4, false>);
        else
            epi ? go(output_nhwc_kernel<8, true>) : go(output_nhwc_kernel<8, false>);
        return hipGetLastError();
    }
    const _Float16* bias = reinterpret_cast<const _Float16*>(ep.bias);
    const int tw = pick_tw((int64_t)B * nh, nw, K);
    const int kb = 256 / tw;
    const int kblocks = (K + kb - 1) / kb;
    const int64_t nblocks = (int64_t)((nw + tw - 1) / tw) * nh * B * kblocks;
    if (nblocks >= ((int64_t)1 << 31)) return hipErrorInvalidConfiguration;
    const int64_t y_bytes = 2 * (int64_t)B * K * Ho * Wo;
    if (y_bytes >= ((int64_t)1 << 31) - 64) return hipErrorInvalidValue;
    // widest row segment: every segment start must be aligned to its width
    // (tw0*6 columns is a multiple of 12, so the row pitch decides)
    // (a residual is read with the same widths, so it must share the alignment)
    const _Float16* res = reinterpret_cast<const _Float16*>(ep.residual);
    const uintptr_t ya = reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(ep.residual);
    const int vw = (Wo % 4 == 0 && ya % 8 == 0) ? 4 : (Wo % 2 == 0 && ya % 4 == 0) ? 2 : 1;
    const dim3 grid((unsigned)nblocks);
    const _Float16* Mh = reinterpret_cast<const _Float16*>(M);
    _Float16* yh = reinterpret_cast<_Float16*>(y);
    const int64_t m_bytes = 2 * 64 * pstride;
    const bool epi = epilogue_needed(bias, ep.relu, res);
    switch (tw) {
        case 2:
            launch_out_tw<2>(vw, epi, grid, s, Mh, yh, K, Ho, Wo, nh, nw, ldm, pstride, kblocks,
                             m_bytes, y_bytes, bias, ep.relu, res);
            break;
        case 4:
            launch_out_tw<4>(vw, epi, grid, s, Mh, yh, K, Ho, Wo, nh, nw, ldm, pstride, kblocks,
                             m_bytes, y_bytes, bias, ep.relu, res);
            break;
        default:
            launch_out_tw<8>(vw, epi, grid, s, Mh, yh, K, Ho, Wo, nh, nw, ldm, pstride, kblocks,
                             m_bytes, y_bytes, bias, ep.relu, res);
            break;
    }
    return hipGetLastError();
}

}  // namespace nova
