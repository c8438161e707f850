// Weight gradient of the NOVA F(6,3) convolution, on the Winograd domain.
//
// The reference's backward computes dL/dw in fp32 PyTorch with a per-sample
// unfold loop (/root/reference/nova_winograd/conv2d.py:121-147). Here it is
// the transpose of the forward's products. Per tile, y = A^T (U . V) A with
// U = G w G^T and V = B^T d B, so dL/dU = sum over tiles of (A dY A^T) . V and
//
//   dw[k][c] = G^T ( sum_bp dM_p[k][bp] * V_p[c][bp] )_{p = 0..63} G,
//
// 64 Winograd-domain products (K x C each) whose reduction runs over the
// tiles, between an input transform and a gradient-side transform of dY:
//
//   wg_input_kernel   Vt[p][c][bp]  = (B^T d B)_p        x fp16 -> fp32
//   wg_grad_kernel    Mt[p][k][bp]  = (A dY A^T)_p       dY fp16/fp32 -> fp32
//                     (dY = 0 outside the Ho x Wo output, so edge tiles
//                     contribute only what the forward wrote)
//   wg_gemm_proj_kernel  part[s][k][c] = G^T (sum_{bp in split s} Mt[p][k][bp]
//                     Vt[p][c][bp])_p G: the 64 products (v_mfma_f32_16x16x4_f32)
//                     each folded into the 3 x 3 result as soon as it is
//                     formed; the tile range is split so the grid fills the
//                     chip; a later sub-batch adds to part
//   wg_reduce_kernel  dw = sum over the splits, in order
//
// The tile index bp = b*P + th*nw + tw (minimal tiling) is padded with zeros
// to BPp, a multiple of 16; the reduction index is contiguous in both
// operands, so every lane loads 4 consecutive tiles with one 16-byte load and
// feeds them to 4 MFMA k-steps (the same 4 in A and B: a permutation of the
// reduction order only).
//
// Precision: fp32 throughout, with the exact-rational tables rounded to fp32
// (kA, kB, kG), not the fp16-rounded A and B of the forward: rounding V or
// dM to fp16 costs about 3 % rel-L2 on dw (measured on the CPU) where this
// stays at the fp32 PyTorch gradient's level (about 5e-6). Deterministic: no
// atomics, splits summed in a fixed order.
#include <algorithm>
#include <type_traits>

#include "nova_internal.h"
#include "nova_tables.h"
#include "nova_tile_math.h"

namespace nova {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

constexpr int kWgOob = (int)0x80000000;  // out-of-range byte offset: loads 0, stores dropped
constexpr int kWgThreads = 256;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t wg_rsrc(const void* p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                             (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                             0x00020000);
}

// Vt[p][c][bp] = (B^T d B)[p] for every (channel c, tile bp < BPp); lanes run
// over consecutive tiles of one channel, so each position's 64 stores of a
// wave are 256 contiguous bytes. Tiles bp >= BP are written as zeros.
__global__ __launch_bounds__(kWgThreads) void wg_input_kernel(const _Float16* __restrict__ x,
                                                              float* __restrict__ Vt, int C,
                                                              int H, int W, int pad, int nh,
                                                              int nw, int BP, int BPp,
                                                              int x_bytes) {
    const int64_t t = (int64_t)blockIdx.x * kWgThreads + threadIdx.x;
    if (t >= (int64_t)C * BPp) return;
    const int c = (int)(t / BPp), bp = (int)(t - (int64_t)c * BPp);
    const int P = nh * nw;
    const bool live = bp < BP;
    const int b = live ? bp / P : 0, tile = live ? bp - (bp / P) * P : 0;
    const int th = tile / nw, tw = tile - (tile / nw) * nw;
    const int h0 = 6 * th - pad, w0 = 6 * tw - pad;
    const __amdgpu_buffer_rsrc_t xr = wg_rsrc(x, x_bytes);
    const int base = 2 * ((b * C + c) * H * W);
    float d[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int h = h0 + i, w = w0 + j;
            const bool ok = live && h >= 0 && h < H && w >= 0 && w < W;
            d[i][j] = (float)__builtin_bit_cast(
                _Float16, __builtin_amdgcn_raw_buffer_load_b16(
                              xr, ok ? base + 2 * (h * W + w) : kWgOob, 0, 0));
        }
    const __amdgpu_buffer_rsrc_t vr = wg_rsrc(Vt, 4 * (int64_t)64 * C * BPp);
    const int pstride = 4 * C * BPp;
    const int off = 4 * (c * BPp + bp);
#pragma unroll
    for (int r = 0; r < 8; r++) {
        float tr[8];  // row r of B^T d
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (kB[i][r] != 0.0f) acc = __builtin_fmaf(kB[i][r], d[i][j], acc);
            tr[j] = acc;
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (kB[j][s] != 0.0f) acc = __builtin_fmaf(tr[j], kB[j][s], acc);
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, acc), vr, off,
                                                  (8 * r + s) * pstride, 0);
        }
    }
}

// Mt[p][k][bp] = (A dY A^T)[p] for every (output channel k, tile bp < BPp),
// with A the 8x6 transpose of kA: Mt[i][j] = sum_r sum_s kA[r][i] g[r][s]
// kA[s][j] over the tile's 6x6 gradient g, zero outside Ho x Wo.
template <typename T>
__global__ __launch_bounds__(kWgThreads) void wg_grad_kernel(const T* __restrict__ dy,
                                                             float* __restrict__ Mt, int K,
                                                             int Ho, int Wo, int nh, int nw,
                                                             int BP, int BPp, int dy_bytes) {
    const int64_t t = (int64_t)blockIdx.x * kWgThreads + threadIdx.x;
    if (t >= (int64_t)K * BPp) return;
    const int k = (int)(t / BPp), bp = (int)(t - (int64_t)k * BPp);
    const int P = nh * nw;
    const bool live = bp < BP;
    const int b = live ? bp / P : 0, tile = live ? bp - (bp / P) * P : 0;
    const int th = tile / nw, tw = tile - (tile / nw) * nw;
    const int oh0 = 6 * th, ow0 = 6 * tw;
    const __amdgpu_buffer_rsrc_t gr = wg_rsrc(dy, dy_bytes);
    const int base = (b * K + k) * Ho * Wo;
    float g[6][6];
#pragma unroll
    for (int r = 0; r < 6; r++)
#pragma unroll
        for (int s = 0; s < 6; s++) {
            const bool ok = live && oh0 + r < Ho && ow0 + s < Wo;
            const int e = base + (oh0 + r) * Wo + ow0 + s;
            if constexpr (sizeof(T) == 4) {
                g[r][s] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(gr, ok ? 4 * e : kWgOob, 0, 0));
            } else {
                g[r][s] = (float)__builtin_bit_cast(
                    _Float16, __builtin_amdgcn_raw_buffer_load_b16(gr, ok ? 2 * e : kWgOob, 0, 0));
            }
        }
    const __amdgpu_buffer_rsrc_t mr = wg_rsrc(Mt, 4 * (int64_t)64 * K * BPp);
    const int pstride = 4 * K * BPp;
    const int off = 4 * (k * BPp + bp);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float ti[6];  // row i of A g
#pragma unroll
        for (int s = 0; s < 6; s++) {
            float acc = 0.0f;
#pragma unroll
            for (int r = 0; r < 6; r++)
                if (kA[r][i] != 0.0f) acc = __builtin_fmaf(kA[r][i], g[r][s], acc);
            ti[s] = acc;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < 6; s++)
                if (kA[s][j] != 0.0f) acc = __builtin_fmaf(ti[s], kA[s][j], acc);
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, acc), mr, off,
                                                  (8 * i + j) * pstride, 0);
        }
    }
}

// Products and the filter-side transform in one pass. dw is linear in the
// 64 position planes of dU: dw[k][c][a][b] = sum_p G[i][a] G[j][b] dU_p[k][c]
// (p = 8i + j), so every 16-tile slice of each position's product is folded
// into 9 accumulators per (k, c) as soon as it is formed, and dU never
// leaves the registers. Workgroup: a 32 (k) x 32 (c) tile and one range of
// tiles; 4 waves, wave w takes positions 16w .. 16w+15 (2 x 2 MFMA tiles of
// 16 x 16, v_mfma_f32_16x16x4_f32). The wave walks
// (16-tile step, position) in one straight sequence per step with the loads
// of the next kAhead positions in flight (one 16-byte load per operand tile
// and lane: 4 consecutive tiles of its row or column), crossing into the next
// step. The 4 waves' accumulators are summed through LDS in a fixed order;
// out[s][k][c][3][3] gets the range's sum (added to what is there when
// accumulate != 0: later sub-batches).
constexpr int kProjK = 32, kProjC = 32;
constexpr int kAhead = 2;

__global__ __launch_bounds__(kWgThreads, 1) void wg_gemm_proj_kernel(
    const float* __restrict__ Mt, const float* __restrict__ Vt, float* __restrict__ out, int K,
    int C, int BPp, int chunk, int nsplit, int accumulate, int nwg) {
    __shared__ float red[4][144][64];  // 144 KB: every wave's accumulators
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ntk = (K + kProjK - 1) / kProjK, ntc = (C + kProjC - 1) / kProjC;
    const int L = xcd_remap((int)blockIdx.x, nwg);
    const int tile = L % (ntk * ntc), sp = L / (ntk * ntc);
    const int k0 = (tile % ntk) * kProjK, c0 = (tile / ntk) * kProjC;
    const int r16 = lane & 15, g = lane >> 4;
    const int p0 = 16 * wave;
    const __amdgpu_buffer_rsrc_t ar = wg_rsrc(Mt, 4 * (int64_t)64 * K * BPp);
    const __amdgpu_buffer_rsrc_t br = wg_rsrc(Vt, 4 * (int64_t)64 * C * BPp);
    int aoff[2], boff[2];
#pragma unroll
    for (int n = 0; n < 2; n++) {
        const int k = k0 + 16 * n + r16, c = c0 + 16 * n + r16;
        aoff[n] = k < K ? 4 * (k * BPp + 4 * g) : kWgOob;
        boff[n] = c < C ? 4 * (c * BPp + 4 * g) : kWgOob;
    }
    const int bp_lo = sp * chunk, bp_hi = min(BPp, bp_lo + chunk);
    const int pa = 4 * K * BPp, pb = 4 * C * BPp;  // position strides (bytes)

    f4 a[kAhead][2], b[kAhead][2];
    // item (step s, position q): slot q % kAhead
    auto load = [&](int slot, int bp0, int q) {
        const bool ok = bp0 < bp_hi;
        const int ua = (p0 + q) * pa + 4 * bp0, ub = (p0 + q) * pb + 4 * bp0;
#pragma unroll
        for (int n = 0; n < 2; n++)
            a[slot][n] = __builtin_bit_cast(
                f4, __builtin_amdgcn_raw_buffer_load_b128(ar, ok ? aoff[n] : kWgOob, ok ? ua : 0,
                                                          0));
#pragma unroll
        for (int n = 0; n < 2; n++)
            b[slot][n] = __builtin_bit_cast(
                f4, __builtin_amdgcn_raw_buffer_load_b128(br, ok ? boff[n] : kWgOob, ok ? ub : 0,
                                                          0));
    };

    float dwa[9][16], t[3][16];
#pragma unroll
    for (int q = 0; q < 9; q++)
#pragma unroll
        for (int e = 0; e < 16; e++) dwa[q][e] = 0.0f;
#pragma unroll
    for (int bb = 0; bb < 3; bb++)
#pragma unroll
        for (int e = 0; e < 16; e++) t[bb][e] = 0.0f;

#pragma unroll
    for (int q = 0; q < kAhead; q++) load(q, bp_lo, q);
    for (int bp0 = bp_lo; bp0 < bp_hi; bp0 += 16) {
        static_for<0, 16>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            const int slot = q % kAhead;
            f4 acc[4];  // (m, n) tiles
#pragma unroll
            for (int u = 0; u < 4; u++) acc[u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < 4; st++)
#pragma unroll
                for (int m = 0; m < 2; m++)
#pragma unroll
                    for (int n = 0; n < 2; n++)
                        acc[2 * m + n] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            a[slot][m][st], b[slot][n][st], acc[2 * m + n], 0, 0, 0);
            // the item kAhead ahead: this step's position q + kAhead, or the
            // next step's position q + kAhead - 16
            if (q + kAhead < 16)
                load(slot, bp0, q + kAhead);
            else
                load(slot, bp0 + 16, q + kAhead - 16);
            // fold, separably: t[b] += G[j][b] dU_p over the row's 8
            // positions (j = q % 8 is a compile-time index: zero
            // coefficients vanish), then dwa[a][b] += G[i][a] t[b] per row
            constexpr int j = q & 7;
#pragma unroll
            for (int bb = 0; bb < 3; bb++)
                if (kG[j][bb] != 0.0f)
#pragma unroll
                    for (int u = 0; u < 4; u++)
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            t[bb][4 * u + e] = __builtin_fmaf(kG[j][bb], acc[u][e], t[bb][4 * u + e]);
            if constexpr (j == 7) {
                const int i = 2 * wave + (q >> 3);
#pragma unroll
                for (int aa = 0; aa < 3; aa++) {
                    const float ga = kG[i][aa];
#pragma unroll
                    for (int bb = 0; bb < 3; bb++)
#pragma unroll
                        for (int e = 0; e < 16; e++) {
                            dwa[3 * aa + bb][e] = __builtin_fmaf(ga, t[bb][e], dwa[3 * aa + bb][e]);
                        }
                }
#pragma unroll
                for (int bb = 0; bb < 3; bb++)
#pragma unroll
                    for (int e = 0; e < 16; e++) t[bb][e] = 0.0f;
            }
        });
    }
#pragma unroll
    for (int q = 0; q < 9; q++)
#pragma unroll
        for (int e = 0; e < 16; e++) red[wave][16 * q + e][lane] = dwa[q][e];
    __syncthreads();
    // the 4 waves summed in order; thread (u, lane) handles accumulators u,
    // u + 4, ...: lane holds rows k0 + 4g + e (e < 4) of columns c0 + 16n + r16
    const __amdgpu_buffer_rsrc_t orr = wg_rsrc(out, 4 * (int64_t)nsplit * K * C * 9);
    for (int u = wave; u < 144; u += 4) {
        const float v0 = red[0][u][lane] + red[1][u][lane] + red[2][u][lane] + red[3][u][lane];
        const int q = u >> 4, m = (u >> 3) & 1, n = (u >> 2) & 1, e = u & 3;
        const int k = k0 + 16 * m + 4 * g + e, c = c0 + 16 * n + r16;
        const int o = (k < K && c < C) ? 4 * (((sp * K + k) * C + c) * 9 + q) : kWgOob;
        float v = v0;
        if (accumulate)
            v += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(orr, o, 0, 0));
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), orr, o, 0, 0);
    }
}

// dw[k][c][3][3] = sum over splits of part[s][k][c][3][3], in split order.
__global__ __launch_bounds__(kWgThreads) void wg_reduce_kernel(const float* __restrict__ part,
                                                               float* __restrict__ dw,
                                                               int64_t n, int nsplit) {
    const int64_t t = (int64_t)blockIdx.x * kWgThreads + threadIdx.x;
    if (t >= n) return;
    // 8 splits' loads in flight, summed in split order
    float v = 0.0f;
    int s = 0;
    for (; s + 8 <= nsplit; s += 8) {
        float r[8];
#pragma unroll
        for (int u = 0; u < 8; u++) r[u] = part[(int64_t)(s + u) * n + t];
#pragma unroll
        for (int u = 0; u < 8; u++) v += r[u];
    }
    for (; s < nsplit; s++) v += part[(int64_t)s * n + t];
    dw[t] = v;
}

inline int64_t round16_64(int64_t v) { return (v + 15) & ~(int64_t)15; }

}  // namespace

WgradPlan wgrad_plan(int B, int C, int K, int H, int W, int pad, int cus) {
    WgradPlan pl{};
    const int Ho = H + 2 * pad - 2, Wo = W + 2 * pad - 2;
    const int64_t P = (int64_t)tiles_min(Ho) * tiles_min(Wo);
    // images per sub-batch: Vt and Mt each below 2^31 bytes (32-bit buffer
    // offsets) and together at most 1 GiB
    const int64_t per_img = 256 * P;  // bytes of one channel's 64 fp32 positions
    const int64_t by_off = (((int64_t)1 << 31) - 256 * 16 - 1) / (per_img * std::max(C, K));
    const int64_t by_total = ((int64_t)1 << 30) / (per_img * (C + K));
    pl.chunk_images = (int)std::max<int64_t>(1, std::min<int64_t>(std::max(B, 1),
                                                                  std::min(by_off, by_total)));
    const int64_t BPp = round16_64(pl.chunk_images * P);
    pl.BPp_max = BPp;
    // splits of the tile range: about one workgroup per CU, at least one
    // 16-tile step per split, partial filters below 2^31 bytes
    const int64_t base = (int64_t)((K + kProjK - 1) / kProjK) * ((C + kProjC - 1) / kProjC);
    int64_t ns = std::max<int64_t>(1, ((int64_t)cus + base - 1) / base);
    ns = std::min<int64_t>(ns, std::max<int64_t>(1, BPp / 16));
    while (ns > 1 && 4 * ns * 9 * (int64_t)K * C >= ((int64_t)1 << 31)) ns--;
    pl.nsplit = (int)ns;
    // Vt, Mt, and the splits' partial filters (none with one split)
    pl.ws_bytes = 4 * 64 * (int64_t)(C + K) * BPp + (ns > 1 ? 4 * ns * 9 * (int64_t)K * C : 0);
    pl.ok = 4 * 64 * (int64_t)std::max(C, K) * BPp < ((int64_t)1 << 31) &&
            4 * ns * 9 * (int64_t)K * C < ((int64_t)1 << 31) &&
            2 * (int64_t)pl.chunk_images * C * H * W < ((int64_t)1 << 31) &&
            4 * (int64_t)pl.chunk_images * K * Ho * Wo < ((int64_t)1 << 31);
    return pl;
}

hipError_t launch_wgrad(const uint16_t* x, const void* dy, bool dy_f32, float* dw, int B, int C,
                        int K, int H, int W, int pad, const WgradPlan& pl, void* ws,
                        hipStream_t s) {
    const int Ho = H + 2 * pad - 2, Wo = W + 2 * pad - 2;
    const int nh = tiles_min(Ho), nw = tiles_min(Wo);
    const int P = nh * nw;
    const int64_t n_dw = (int64_t)K * C * 9;
    float* Vt = static_cast<float*>(ws);
    float* part = pl.nsplit > 1 ? Vt + (int64_t)64 * (C + K) * pl.BPp_max : dw;
    if (B == 0) {  // no images: zero gradient
        launch(wg_reduce_kernel, dim3((unsigned)((n_dw + kWgThreads - 1) / kWgThreads)),
               dim3(kWgThreads), s, static_cast<const float*>(dw), dw, n_dw, 0);
        return hipGetLastError();
    }
    for (int b0 = 0; b0 < B; b0 += pl.chunk_images) {
        const int Bc = std::min(pl.chunk_images, B - b0);
        const int BP = Bc * P;
        const int BPp = (int)round16_64(BP);
        float* Mt = Vt + (int64_t)64 * C * BPp;
        const uint16_t* xb = x + (int64_t)b0 * C * H * W;
        const int esz = dy_f32 ? 4 : 2;
        const char* gb = static_cast<const char*>(dy) + (int64_t)b0 * K * Ho * Wo * esz;
        launch(wg_input_kernel, dim3((unsigned)(((int64_t)C * BPp + kWgThreads - 1) / kWgThreads)),
               dim3(kWgThreads), s, reinterpret_cast<const _Float16*>(xb), Vt, C, H, W, pad, nh,
               nw, BP, BPp, (int)(2 * (int64_t)Bc * C * H * W));
        const dim3 ggrid((unsigned)(((int64_t)K * BPp + kWgThreads - 1) / kWgThreads));
        const int gbytes = (int)((int64_t)esz * Bc * K * Ho * Wo);
        if (dy_f32)
            launch(wg_grad_kernel<float>, ggrid, dim3(kWgThreads), s,
                   reinterpret_cast<const float*>(gb), Mt, K, Ho, Wo, nh, nw, BP, BPp, gbytes);
        else
            launch(wg_grad_kernel<_Float16>, ggrid, dim3(kWgThreads), s,
                   reinterpret_cast<const _Float16*>(gb), Mt, K, Ho, Wo, nh, nw, BP, BPp, gbytes);
        // tile ranges of this sub-batch, in 16-tile steps
        const int steps = BPp / 16;
        const int chunk = 16 * ((steps + pl.nsplit - 1) / pl.nsplit);
        const int64_t grid = (int64_t)pl.nsplit * ((K + kProjK - 1) / kProjK) *
                             ((C + kProjC - 1) / kProjC);
        launch_n(wg_gemm_proj_kernel, dim3((unsigned)grid), dim3(kWgThreads), s,
               static_cast<const float*>(Mt), static_cast<const float*>(Vt), part, K, C, BPp,
               chunk, pl.nsplit, b0 > 0 ? 1 : 0);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (pl.nsplit > 1)
        launch(wg_reduce_kernel, dim3((unsigned)((n_dw + kWgThreads - 1) / kWgThreads)),
               dim3(kWgThreads), s, static_cast<const float*>(part), dw, n_dw, pl.nsplit);
    return hipGetLastError();
}

}  // namespace nova
