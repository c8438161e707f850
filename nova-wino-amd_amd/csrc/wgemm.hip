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
// Byte offsets are 32-bit: U, V and M must each stay below 2 GB.
#include <type_traits>

#include "nova_internal.h"
#include "nova_tile_math.h"

namespace nova {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

constexpr int kOob = (int)0x80000000;  // byte offset past every buffer: loads 0, stores dropped

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                             (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                             0x00020000);
}

// MT x NT 16x16 MFMA tiles per wave, WGM x WGN waves per workgroup. Operands
// are read through buffer resources: the per-lane part of each offset (row,
// channel octet) is fixed, the wave-uniform part (position, channel step)
// goes in a scalar offset, and lanes outside K / BP / Cp read zeros. A ring
// of PD channel steps is kept in flight (register prefetch) so the loop is
// not bound by load latency; steps past Cp are zero loads.
template <int MT, int NT, int WGM, int WGN, int PD>
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

    const __amdgpu_buffer_rsrc_t urs = make_rsrc(U, 2 * (int64_t)64 * K * Cp);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, 2 * (int64_t)64 * BP * Cp);
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(M, 2 * (int64_t)64 * BP * K);

    int aoff[MT], boff[NT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++) {
        const int k = kbase + mi * 16 + r16;
        aoff[mi] = k < K ? 2 * (k * Cp + 8 * g) : kOob;
    }
#pragma unroll
    for (int ni = 0; ni < NT; ni++) {
        const int n = nbase + ni * 16 + r16;
        boff[ni] = n < BP ? 2 * (n * Cp + 8 * g) : kOob;
    }
    const int au = 2 * p * K * Cp;   // uniform
    const int bu = 2 * p * BP * Cp;  // uniform
    const int nsteps = (Cp + 31) / 32;

    h8 a[PD][MT], b[PD][NT];
    auto load_step = [&](int step, h8 af[MT], h8 bf[NT]) {
        const int c = step * 32;
        const bool cok = c + 8 * g < Cp;
#pragma unroll
        for (int mi = 0; mi < MT; mi++)
            af[mi] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
                                                urs, cok ? aoff[mi] : kOob, au + 2 * c, 0));
#pragma unroll
        for (int ni = 0; ni < NT; ni++)
            bf[ni] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
                                                vrs, cok ? boff[ni] : kOob, bu + 2 * c, 0));
    };

    f4 acc[MT][NT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int ni = 0; ni < NT; ni++) acc[mi][ni] = f4{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
    for (int j = 0; j < PD; j++) load_step(j, a[j], b[j]);
    for (int s0 = 0; s0 < nsteps; s0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; j++) {
#pragma unroll
            for (int mi = 0; mi < MT; mi++)
#pragma unroll
                for (int ni = 0; ni < NT; ni++)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j][mi], b[j][ni],
                                                                         acc[mi][ni], 0, 0, 0);
            if (s0 + PD < nsteps) load_step(s0 + PD + j, a[j], b[j]);
        }
    }

    const int mu = 2 * p * BP * K;  // uniform
    const bool vec_store = (K & 3) == 0;
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int ni = 0; ni < NT; ni++) {
            const int bp = nbase + ni * 16 + r16;
            const int k = kbase + mi * 16 + 4 * g;
            const int off = bp < BP ? 2 * (bp * K + k) : kOob;
            if (vec_store) {
                h4 v = {(_Float16)acc[mi][ni][0], (_Float16)acc[mi][ni][1],
                        (_Float16)acc[mi][ni][2], (_Float16)acc[mi][ni][3]};
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, v), mrs,
                                                      k < K ? off : kOob, mu, 0);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    __builtin_amdgcn_raw_buffer_store_b16(
                        __builtin_bit_cast(uint16_t, (_Float16)acc[mi][ni][i]), mrs,
                        k + i < K ? off + 2 * i : kOob, mu, 0);
            }
        }
}

template <int MT, int NT, int WGM, int WGN, int PD>
static hipError_t launch_cfg(const uint16_t* U, const uint16_t* V, uint16_t* M, int K, int Cp,
                             int BP, hipStream_t s) {
    constexpr int TM = MT * 16 * WGM, TN = NT * 16 * WGN;
    dim3 grid((unsigned)((BP + TN - 1) / TN), (unsigned)((K + TM - 1) / TM), 64);
    launch(wgemm_kernel<MT, NT, WGM, WGN, PD>, grid, dim3(64 * WGM * WGN), s,
        reinterpret_cast<const _Float16*>(U), reinterpret_cast<const _Float16*>(V),
        reinterpret_cast<_Float16*>(M), K, Cp, BP);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// LDS-tiled variant for larger shapes. Workgroup tile = TK output channels x
// TB tiles (bp) of one position, WK x WB waves, channels in stages of 64
// (two MFMA k-steps): every stage is copied global -> registers -> LDS with
// 16-byte loads (one 128-byte line per row when Cp >= 64), double buffered so
// the next stage's loads are in flight while the current one is multiplied.
// LDS rows are 128 bytes with an XOR swizzle of their 16-byte chunks (see
// the kernel), conflict-free for both the staging writes and the fragment
// reads.
// ---------------------------------------------------------------------------
constexpr int kStageC = 64;

template <int TK, int TB, int WK, int WB, int PF, int SM>
__global__ __launch_bounds__(64 * WK * WB) void wgemm_lds_kernel(const _Float16* __restrict__ U,
                                                        const _Float16* __restrict__ V,
                                                        _Float16* __restrict__ M, int K, int Cp,
                                                        int BP, int nwg) {
    constexpr int kThreads = 64 * WK * WB;
    constexpr int MT = TK / WK / 16;  // 16x16 tiles per wave along k
    constexpr int NT = TB / WB / 16;  // along bp
    constexpr int kChunksU = TK * kStageC / 8;  // 16-byte chunks per stage
    constexpr int kChunksV = TB * kStageC / 8;
    constexpr int kPerThreadU = (kChunksU + kThreads - 1) / kThreads;
    constexpr int kPerThreadV = (kChunksV + kThreads - 1) / kThreads;
    // Double-buffered stages, U then V: rows of kStageC channels (128 bytes),
    // 16-byte chunk c of row r stored at chunk c ^ ((r >> 1) & 7). The XOR
    // swizzle keeps both access patterns conflict-free on the 64 banks: the
    // staging writes (8 lanes per row, two rows per 16 lanes) and the
    // fragment reads (16 lanes on 16 consecutive rows, one chunk each).
    __shared__ __align__(16) _Float16 smem[2 * (TK + TB) * kStageC];
    auto sU = [&](int buf) { return smem + buf * TK * kStageC; };
    auto sV = [&](int buf) { return smem + 2 * TK * kStageC + buf * TB * kStageC; };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wk = wave % WK, wb = wave / WK;
    // One-dimensional grid, XCD-aware: every XCD takes a contiguous run of
    // (position, k-tile, bp-tile) items with the bp tile fastest, so all
    // tiles of a position meet in one L2 and U_p, V_p leave HBM once.
    const int nbt = (BP + TB - 1) / TB, nkt = (K + TK - 1) / TK;
    const int item = xcd_remap((int)blockIdx.x, nwg);
    const int p = item / (nbt * nkt);
    const int rem = item - p * (nbt * nkt);
    const int k0 = (rem / nbt) * TK;
    const int n0 = (rem % nbt) * TB;
    const int r16 = lane & 15, g = lane >> 4;

    const __amdgpu_buffer_rsrc_t urs = make_rsrc(U, 2 * (int64_t)64 * K * Cp);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, 2 * (int64_t)64 * BP * Cp);
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(M, 2 * (int64_t)64 * BP * K);
    const int au = 2 * p * K * Cp;  // uniform byte offsets of position p
    const int bu = 2 * p * BP * Cp;

    // staging assignment: chunk id -> (row, 8-channel group); 8 chunks per row
    int uoff[kPerThreadU], ulds[kPerThreadU], voff[kPerThreadV], vlds[kPerThreadV];
#pragma unroll
    for (int j = 0; j < kPerThreadU; j++) {
        const int ch = tid + j * kThreads;
        const int row = ch >> 3, cg = ch & 7;
        const bool ok = ch < kChunksU && k0 + row < K;
        uoff[j] = ok ? 2 * ((k0 + row) * Cp + cg * 8) : kOob;
        ulds[j] = ch < kChunksU ? row * kStageC + (cg ^ ((row >> 1) & 7)) * 8 : -1;
    }
#pragma unroll
    for (int j = 0; j < kPerThreadV; j++) {
        const int ch = tid + j * kThreads;
        const int row = ch >> 3, cg = ch & 7;
        const bool ok = ch < kChunksV && n0 + row < BP;
        voff[j] = ok ? 2 * ((n0 + row) * Cp + cg * 8) : kOob;
        vlds[j] = ch < kChunksV ? row * kStageC + (cg ^ ((row >> 1) & 7)) * 8 : -1;
    }
    const int nstages = (Cp + kStageC - 1) / kStageC;
    // PF stages in flight in registers: slot st % PF holds stage st from its
    // load until its copy into LDS
    h8 ru[PF][kPerThreadU], rv[PF][kPerThreadV];
    auto gload = [&](int st, h8 (&u)[kPerThreadU], h8 (&v)[kPerThreadV]) {
        const int c = st * kStageC;
#pragma unroll
        for (int j = 0; j < kPerThreadU; j++) {
            const int cg = (tid + j * kThreads) & 7;
            const bool cok = c + cg * 8 < Cp;
            u[j] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
                                              urs, cok ? uoff[j] : kOob, au + 2 * c, 0));
        }
#pragma unroll
        for (int j = 0; j < kPerThreadV; j++) {
            const int cg = (tid + j * kThreads) & 7;
            const bool cok = c + cg * 8 < Cp;
            v[j] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
                                              vrs, cok ? voff[j] : kOob, bu + 2 * c, 0));
        }
    };
    auto lstore = [&](int buf, const h8 (&u)[kPerThreadU], const h8 (&v)[kPerThreadV]) {
#pragma unroll
        for (int j = 0; j < kPerThreadU; j++)
            if (ulds[j] >= 0) *reinterpret_cast<h8*>(sU(buf) + ulds[j]) = u[j];
#pragma unroll
        for (int j = 0; j < kPerThreadV; j++)
            if (vlds[j] >= 0) *reinterpret_cast<h8*>(sV(buf) + vlds[j]) = v[j];
    };

    f4 acc[MT][NT];
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int ni = 0; ni < NT; ni++) acc[mi][ni] = f4{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
    for (int j = 0; j < PF; j++)
        if (j < nstages) gload(j, ru[j], rv[j]);
    lstore(0, ru[0], rv[0]);
    __syncthreads();
    for (int st0 = 0; st0 < nstages; st0 += PF) {
#pragma unroll
        for (int j = 0; j < PF; j++) {
            const int st = st0 + j;
            if (st >= nstages) break;
            const int buf = st & 1;
            if (st + PF < nstages) gload(st + PF, ru[j], rv[j]);
            // lane (row r16 of each 16-row tile, chunk 4*kk + g); every tile
            // starts at a multiple of 16 rows, so the swizzle depends on r16
            const int c0 = g ^ ((r16 >> 1) & 7);
            const _Float16* su = sU(buf) + (wk * MT * 16 + r16) * kStageC;
            const _Float16* sv = sV(buf) + (wb * NT * 16 + r16) * kStageC;
#pragma unroll
            for (int kk = 0; kk < kStageC / 32; kk++) {
                const int co = (c0 ^ (4 * kk)) * 8;
                h8 a[MT], b[NT];
#pragma unroll
                for (int mi = 0; mi < MT; mi++)
                    a[mi] = *reinterpret_cast<const h8*>(su + mi * 16 * kStageC + co);
#pragma unroll
                for (int ni = 0; ni < NT; ni++)
                    b[ni] = *reinterpret_cast<const h8*>(sv + ni * 16 * kStageC + co);
#pragma unroll
                for (int mi = 0; mi < MT; mi++)
#pragma unroll
                    for (int ni = 0; ni < NT; ni++)
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mi], b[ni],
                                                                             acc[mi][ni], 0, 0, 0);
            }
            if (st + 1 < nstages) lstore(buf ^ 1, ru[(j + 1) % PF], rv[(j + 1) % PF]);
            __syncthreads();
        }
    }

    const int mu = 2 * p * BP * K;
    if constexpr (SM != 0) {
        // SM 1/2: the M tile goes through LDS as [bp][k] rows and leaves as
        // whole rows, 16 bytes per lane (SM 2: written through the L2, sc1);
        // the L2 then holds whole lines instead of 32-byte pieces of 16.
        if ((K & 7) == 0) {
            constexpr int kMP = TK + 8;  // halves per staged row
            static_assert(TB * kMP <= 2 * (TK + TB) * kStageC, "M tile fits in the stages");
            _Float16* sm = smem;
#pragma unroll
            for (int mi = 0; mi < MT; mi++)
#pragma unroll
                for (int ni = 0; ni < NT; ni++) {
                    const int bpl = (wb * NT + ni) * 16 + r16;
                    const int kl = (wk * MT + mi) * 16 + 4 * g;
                    *reinterpret_cast<h4*>(sm + bpl * kMP + kl) =
                        h4{(_Float16)acc[mi][ni][0], (_Float16)acc[mi][ni][1],
                           (_Float16)acc[mi][ni][2], (_Float16)acc[mi][ni][3]};
                }
            __syncthreads();
            typedef unsigned u4 __attribute__((ext_vector_type(4)));
            constexpr int kCh = TK / 8;  // 16-byte chunks per row
#pragma unroll
            for (int e = tid; e < TB * kCh; e += kThreads) {
                const int row = e / kCh, ch = e % kCh;
                const int bp = n0 + row, k = k0 + 8 * ch;
                const u4 v = *reinterpret_cast<const u4*>(sm + row * kMP + 8 * ch);
                __builtin_amdgcn_raw_buffer_store_b128(
                    v, mrs, (bp < BP && k < K) ? 2 * (bp * K + k) : kOob, mu, SM == 2 ? kWT : 0);
            }
            return;
        }
    }
    const bool vec_store = (K & 3) == 0;
#pragma unroll
    for (int mi = 0; mi < MT; mi++)
#pragma unroll
        for (int ni = 0; ni < NT; ni++) {
            const int bp = n0 + (wb * NT + ni) * 16 + r16;
            const int k = k0 + (wk * MT + mi) * 16 + 4 * g;
            const int off = bp < BP ? 2 * (bp * K + k) : kOob;
            if (vec_store) {
                h4 v = {(_Float16)acc[mi][ni][0], (_Float16)acc[mi][ni][1],
                        (_Float16)acc[mi][ni][2], (_Float16)acc[mi][ni][3]};
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, v), mrs,
                                                      k < K ? off : kOob, mu, 0);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    __builtin_amdgcn_raw_buffer_store_b16(
                        __builtin_bit_cast(uint16_t, (_Float16)acc[mi][ni][i]), mrs,
                        k + i < K ? off + 2 * i : kOob, mu, 0);
            }
        }
}

// M epilogue of the LDS kernels (SM of wgemm_lds_kernel): always staged
// through LDS as whole rows (K % 8 == 0); written through the L2 (sc1, so the
// launch boundary has no dirty M to write back before the output transform
// starts) when M holds at most 32 MB. Measured on MI355X, whole forwards, us
// (direct b64 stores -> staged): ResNet-50 batch 32 128@28^2 28.9 -> 28.0,
// 256@14^2 30.2 -> 29.6, 512@7^2 28.6 -> 27.1, conv2_x three-pass 40.8 ->
// 36.4; batch 128 128@28^2 70.3 -> 64.1; batch 1 64@56^2 10.9 -> 10.4.
// Staged, write-back -> written through (with the V of the input transform
// written through as well; GEMM + output transform launches, event-timed):
// batch 16 256@14^2 7.22 + 6.75 -> 6.42 + 5.95; batch 64 128@28^2 11.69 +
// 11.69 -> 10.54 + 11.56; SDXL 320@128^2 (20 MB) 13.86 + 11.36 -> 12.81 +
// 11.52; above 32 MB it loses (batch 128 512@7^2, 34 MB: 26.59 + 12.77 ->
// 28.06 + 15.25). Streaming M with nt instead (4-16 MB) gained 0.4-1.2 us.
static int m_epilogue(int K, int BP) {
    const int64_t m_bytes = 2 * (int64_t)64 * BP * K;
    return m_bytes <= ((int64_t)32 << 20) ? 2 : 1;
}

template <int TK, int TB, int WK, int WB, int PF>
static hipError_t launch_lds(const uint16_t* U, const uint16_t* V, uint16_t* M, int K, int Cp,
                             int BP, hipStream_t s) {
    const unsigned grid = 64u * (unsigned)((BP + TB - 1) / TB) * (unsigned)((K + TK - 1) / TK);
    auto go = [&](auto kernel) {
        launch_n(kernel, dim3(grid), dim3(64 * WK * WB), s, reinterpret_cast<const _Float16*>(U),
               reinterpret_cast<const _Float16*>(V), reinterpret_cast<_Float16*>(M), K, Cp, BP);
    };
    if (m_epilogue(K, BP) == 2)
        go(wgemm_lds_kernel<TK, TB, WK, WB, PF, 2>);
    else
        go(wgemm_lds_kernel<TK, TB, WK, WB, PF, 1>);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GEMV-like shapes (BP <= 32, or 48 above K = 1024) on 1 KB operand blocks: U from the two-pass
// kernel's block copy (launch_u_wfrag: block (p, 16-row tile, 32-channel
// step), lane l = row l % 16, channels 8*(l / 16) .. +7) and V in the
// two-pass layout (launch_input_transform with vfrag = ceil(Cp / 32)), so
// every operand fragment is one contiguous 1 KB load per wave; the product
// layouts make it 16 rows x 64 bytes, two rows per 128-byte line with the
// line's other half fetched by the next step. Wave = MT 16-row tiles of K x
// all NT 16-tile blocks of BP; PD steps in flight; M leaves in the product
// layout [64][BP][K] for the output transform. Same lane layout and
// channel-step order as the other GEMM kernels: M is bit-identical. Measured
// on MI355X (back-to-back launches, us, product-layout kernel -> blocks):
// 512@7^2 batch 1 6.5 -> 4.6, batch 4 8.8 -> 4.7, batch 8 (32 tiles) 7.8 ->
// 6.5; 256@14^2 batch 1 3.1 -> 2.8, batch 3 4.1 -> 3.3; 128@28^2 batch 1 (25
// tiles) 3.1 -> 2.7; 1280@8^2 batch 1 33.4 -> 30.4, batch 2 35.1 -> 30.6 (U
// at 6.9 TB/s); 1280@16^2 batch 2 (18 tiles) 33.7 -> 31.3. Past 32 tiles
// (three blocks per wave) it won at 3 of 4 shapes (1280@32^2 batch 1, 36
// tiles, 35.2 -> 33.3; 512@7^2 batch 12 8.1 -> 7.3) and lost 7 % at 640@32^2
// batch 1, so it takes 33-48 tiles only above K = 1024 (whole forwards in a
// graph, us: 1280@32^2 batch 1 51.0 -> 49.0, 1280@36^2 51.7 -> 49.8; 1024@32^2
// batch 1 36.3 -> 36.5).
// ---------------------------------------------------------------------------
template <int MT, int NT, int PD, int WPB, int kPol>
__global__ __launch_bounds__(64 * WPB) void wgemm_block_kernel(
    const _Float16* __restrict__ Uw, const _Float16* __restrict__ Vb, _Float16* __restrict__ M,
    int K, int Cp, int BP, int u_bytes, int v_bytes, int m_bytes, int nwg) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int nkt = (K + 15) / 16;
    const int nkg = (nkt + MT - 1) / MT;
    // XCD-aware: each XCD takes a contiguous run of positions
    const int item = xcd_remap((int)blockIdx.x, nwg) * WPB + wave;
    if (item >= 64 * nkg) return;  // no barrier below: idle waves may leave
    const int p = item / nkg;
    const int kt0 = (item - p * nkg) * MT;
    const int nsteps = (Cp + 31) / 32;
    const int nbb = (BP + 15) / 16;  // <= NT
    const int r16 = lane & 15, g = lane >> 4;
    const __amdgpu_buffer_rsrc_t urs = make_rsrc(Uw, u_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(Vb, v_bytes);
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(M, m_bytes);
    // U blocks hold zeros past K and Cp; V slots of tiles past BP and of
    // channels past Cp are never written, so those lanes read through
    // out-of-range offsets
    int aoff[MT], boff[NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
        aoff[i] = kt0 + i < nkt ? (p * nkt + kt0 + i) * nsteps * 1024 + lane * 16 : kOob;
#pragma unroll
    for (int n = 0; n < NT; n++)
        boff[n] = 16 * n + r16 < BP ? ((p * nbb + n) * nsteps) * 1024 + lane * 16 : kOob;
    h8 a[PD][MT], b[PD][NT];
    auto load = [&](int j, h8 (&af)[MT], h8 (&bf)[NT]) {
        const bool cok = j < nsteps && 32 * j + 8 * g < Cp;  // Cp % 8 == 0: whole groups
#pragma unroll
        for (int i = 0; i < MT; i++)
            af[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
                                               urs, j < nsteps ? aoff[i] : kOob, j * 1024, 0));
#pragma unroll
        for (int n = 0; n < NT; n++)
            bf[n] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
                                               vrs, cok ? boff[n] : kOob, j * 1024, 0));
    };
    f4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int n = 0; n < NT; n++) acc[i][n] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < PD; j++) load(j, a[j], b[j]);
    for (int s0 = 0; s0 < nsteps; s0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; j++) {
            if (s0 + j >= nsteps) break;
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int n = 0; n < NT; n++)
                    acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j][i], b[j][n],
                                                                       acc[i][n], 0, 0, 0);
            if (s0 + PD + j < nsteps) load(s0 + PD + j, a[j], b[j]);
        }
    }
    const int mu = 2 * p * BP * K;  // uniform
    const bool vec_store = (K & 3) == 0;
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int k = (kt0 + i) * 16 + 4 * g;
            const int bp = 16 * n + r16;
            const int off = bp < BP ? 2 * (bp * K + k) : kOob;
            if (vec_store) {
                h4 v = {(_Float16)acc[i][n][0], (_Float16)acc[i][n][1], (_Float16)acc[i][n][2],
                        (_Float16)acc[i][n][3]};
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, v), mrs,
                                                      k < K ? off : kOob, mu, kPol);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    __builtin_amdgcn_raw_buffer_store_b16(
                        __builtin_bit_cast(uint16_t, (_Float16)acc[i][n][e]), mrs,
                        k + e < K ? off + 2 * e : kOob, mu, kPol);
            }
        }
}

bool wgemm_blocks(int K, int Cp, int BP) {
    return (BP <= 32 || (BP <= 48 && K > 1024)) && 2 * u_frag_elems(K, Cp) < ((int64_t)1 << 31) &&
           2 * (int64_t)64 * BP * K < ((int64_t)1 << 31);
}

hipError_t launch_wgemm_blocks(const uint16_t* Uw, const uint16_t* Vb, uint16_t* M, int K,
                               int Cp, int BP, hipStream_t s) {
    if (!wgemm_blocks(K, Cp, BP) || Cp % 8 != 0) return hipErrorInvalidValue;
    if (BP == 0) return hipSuccess;
    constexpr int kMT = 2, kPD = 4, kWPB = 2;
    const int nkg = ((K + 15) / 16 + kMT - 1) / kMT;
    const unsigned grid = (unsigned)((64 * nkg + kWPB - 1) / kWPB);
    auto go = [&](auto kernel) {
        launch_n(kernel, dim3(grid), dim3(64 * kWPB), s, reinterpret_cast<const _Float16*>(Uw),
               reinterpret_cast<const _Float16*>(Vb), reinterpret_cast<_Float16*>(M), K, Cp, BP,
               (int)(2 * u_frag_elems(K, Cp)), (int)(2 * gemm_out_v_elems(Cp, BP)),
               (int)(2 * (int64_t)64 * BP * K));
    };
    // M (32-byte pieces of lines) written through the L2 while it is small
    // (batch-1 layers, kWTSmallBytes)
    const bool wt = 2 * (int64_t)64 * BP * K <= kWTSmallBytes;
    auto by_tiles = [&](auto pol) {
        constexpr int P = decltype(pol)::value;
        if (BP <= 16)
            go(wgemm_block_kernel<kMT, 1, kPD, kWPB, P>);
        else if (BP <= 32)
            go(wgemm_block_kernel<kMT, 2, kPD, kWPB, P>);
        else
            go(wgemm_block_kernel<kMT, 3, kPD, kWPB, P>);
    };
    if (wt)
        by_tiles(std::integral_constant<int, kWT>());
    else
        by_tiles(std::integral_constant<int, 0>());
    return hipGetLastError();
}

const char* wgemm_blocks_name(int BP) {
    return BP <= 16   ? "wgemm_block_kernel<2, 1, 4, 2>"
           : BP <= 32 ? "wgemm_block_kernel<2, 2, 4, 2>"
                      : "wgemm_block_kernel<2, 3, 4, 2>";
}

// Kernel per shape on the product layouts (the operand-block kernel above
// takes GEMV-like shapes when the handle can hold U's block copy; this rule
// serves the rest, and the allocation-free forward). Register-direct 64 x 16
// for GEMV-like batch-1 deep layers (BP <= 16: few tiles; two 16-row tiles
// per wave, which halves the V fragment loads and doubles the U bytes each
// wave keeps in flight: 512@7^2 at batch 1 7.1 -> 6.5 us, 1280@8^2 at batch
// 2 39.2 -> 34.9 us); LDS-tiled otherwise, the tile chosen from a sweep of
// every tile shape on MI355X
// (GEMM launch alone, per-kernel events, min of 2 x 60 launches, us; the
// results are bit-identical across tile shapes):
//  * 128 x 128 for K >= 512 with BP >= 256 (512@7^2 B=64 17.1 vs 20.3-22.4
//    for the other shapes, B=128 31.4 vs 35.1-41.4);
//  * 128 x 64 (8 waves) for K >= 1024 below 128 tiles (1280@16^2 B=2 33.6 vs
//    36.4 for 64 x 64; 1280@32^2 B=1 34.0 vs 35.9; 640->1280@16^2 B=2 17.8 vs
//    19.5);
//  * 64 x 128, two stages in flight, for larger work: K >= 640 from 64 tiles,
//    K >= 512 from 128, K >= 256 from 200, K <= 128 from 1600 (ResNet-50
//    256@14^2 B=32 9.5 vs 11.0, B=128 24.6 vs 29.1; 512@7^2 B=32 10.8 vs
//    11.2 for 128 x 128; 128@28^2 B=128 23.0 vs 26.0; SD-1.5 640@32^2 B=2
//    14.4 vs 15.6, 320@64^2 B=2 8.8 vs 9.7; SDXL 640@64^2 14.5 vs 17.7;
//    1280->640@32^2 B=2 23.6 vs 30.4). A second sweep (back-to-back launches
//    of the GEMM alone) favoured it for K <= 128 from 200 tiles as well
//    (128@28^2 B=32 7.17 -> 6.38), but inside forwards, with V just written,
//    it lost there (batch 32 8.95 -> 9.41 us per GEMM), so 64 x 64 stays;
//  * 64 x 96 with four waves and one stage in flight where that tile width
//    fills its last tile 15 points better than 128 (GEMM alone, us:
//    256@14^2 B=32, 288 tiles, 6.98 -> 6.39; 640@32^2 B=2, 72 tiles, 13.9 ->
//    12.4, with 320 -> 640 channels 7.9 -> 7.3, 1280 -> 640 24.0 -> 21.2;
//    640@32^2 B=4 21.3 -> 19.9; inside forwards 640@32^2 B=2 13.2 -> 11.9,
//    whole forward 30.0 -> 28.5; 256@14^2 B=32 unchanged, 9.1 vs 9.0); where
//    the fills are close 64 x 128 stays ahead (256@14^2 B=64 12.5 vs 12.4,
//    128@28^2 B=64 11.9 vs 12.4);
//  * else 64 x 64: two stages in flight from 128 tiles (128@28^2 B=32 8.7,
//    128 x 128 8.7, 64 x 128 8.9; 256@14^2 B=16 7.5 vs 8.1 for 64 x 128),
//    8 waves up to K = 256, 4 waves beyond (512@7^2 B=8 7.7 vs 8.0 with 8
//    waves and 9.0 with 64 x 128; B=16 8.0 vs 9.3).
// Share of a row of bp tiles of width tb that holds real tiles.
static double bp_fill(int BP, int tb) { return (double)BP / (tb * ((BP + tb - 1) / tb)); }

static int wgemm_cfg(int K, int BP) {
    if (BP <= 16) return 0;
    if (K >= 512 && BP >= 256) return 2;
    if (K >= 1024 && BP < 128) return 5;
    if ((K >= 640 && BP >= 64) || (K >= 512 && BP >= 128) || (K >= 256 && BP >= 200) ||
        (K <= 128 && BP >= 1600))
        return bp_fill(BP, 96) >= bp_fill(BP, 128) + 0.15 ? 7 : 6;
    if (BP >= 128) return 3;
    return K <= 256 ? 4 : 1;
}

int wgemm_v_reads(int K, int BP) {
    const int cfg = wgemm_cfg(K, BP);
    const int tk = (cfg == 2 || cfg == 5) ? 128 : 64;  // output channels per workgroup tile
    return (K + tk - 1) / tk;
}

const char* wgemm_name(int K, int Cp, int BP) {
    (void)Cp;
    static const char* names[] = {"wgemm_kernel<2, 1, 2, 1, 4>", "wgemm_lds_kernel<64, 64, 2, 2, 1>",
                                  "wgemm_lds_kernel<128, 128, 2, 4, 1>",
                                  "wgemm_lds_kernel<64, 64, 2, 4, 2>",
                                  "wgemm_lds_kernel<64, 64, 2, 4, 1>",
                                  "wgemm_lds_kernel<128, 64, 2, 4, 1>",
                                  "wgemm_lds_kernel<64, 128, 2, 4, 2>",
                                  "wgemm_lds_kernel<64, 96, 2, 2, 1>"};
    return names[wgemm_cfg(K, BP)];
}

hipError_t launch_wgemm(const uint16_t* U, const uint16_t* V, uint16_t* M, int K, int Cp,
                        int BP, hipStream_t s) {
    switch (wgemm_cfg(K, BP)) {
        case 0: return launch_cfg<2, 1, 2, 1, 4>(U, V, M, K, Cp, BP, s);
        case 1: return launch_lds<64, 64, 2, 2, 1>(U, V, M, K, Cp, BP, s);
        case 2: return launch_lds<128, 128, 2, 4, 1>(U, V, M, K, Cp, BP, s);
        case 3: return launch_lds<64, 64, 2, 4, 2>(U, V, M, K, Cp, BP, s);
        case 5: return launch_lds<128, 64, 2, 4, 1>(U, V, M, K, Cp, BP, s);
        case 6: return launch_lds<64, 128, 2, 4, 2>(U, V, M, K, Cp, BP, s);
        case 7: return launch_lds<64, 96, 2, 2, 1>(U, V, M, K, Cp, BP, s);
        default: return launch_lds<64, 64, 2, 4, 1>(U, V, M, K, Cp, BP, s);
    }
}

}  // namespace nova
