// Internal interfaces between the translation units of libnova_winograd.so.
// Nothing here is exported; the public C-ABI is include/nova_winograd.h.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <cstdint>

namespace nova {

// Per-kernel timing hook. When a caller sets the calling thread's
// KernelEvents, the next kernel that thread launches records its own start
// and end (the timestamps of its dispatch packet, hipExtLaunchKernelGGL) into
// those events, which then time the kernel alone -- without the dispatch gap
// in front of it that events recorded between kernels would include. The
// events are consumed by that launch; either may be null (a span over two
// launches: the first records the start, the second the end). Unset (the
// default), launches are plain triple-chevron launches.
struct KernelEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
KernelEvents& kernel_events();

// lds: bytes of dynamic LDS (extern __shared__) per workgroup.
template <typename... KArgs, typename... Args>
inline void launch_lds(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds,
                       hipStream_t s, Args... args) {
    static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
    KernelEvents& ev = kernel_events();
    if (ev.start != nullptr || ev.stop != nullptr) {
        hipExtLaunchKernelGGL(kernel, grid, block, lds, s, ev.start, ev.stop, 0,
                              static_cast<KArgs>(args)...);
        ev = KernelEvents{};
    } else {
        kernel<<<grid, block, lds, s>>>(static_cast<KArgs>(args)...);
    }
}

template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t s,
                   Args... args) {
    launch_lds(kernel, grid, block, 0, s, args...);
}

// launch() for a kernel with a one-dimensional grid whose last parameter is
// its number of workgroups (grid.x, appended here). Kernels take that count
// as an argument instead of reading gridDim or blockDim: either read makes
// the compiler add 256 bytes of hidden kernel arguments, which the runtime
// writes to device memory on every launch -- 0.7-0.8 us of host time per
// launch on MI355X (2.8 us per launch without them, 3.5 with).
template <typename... KArgs, typename... Args>
inline void launch_n(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t s,
                     Args... args) {
    launch(kernel, grid, block, s, args..., (int)grid.x);
}
// launch_n() with dynamic LDS and the workgroup's thread count (block.x)
// appended before the workgroup count.
template <typename... KArgs, typename... Args>
inline void launch_n_lds(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds,
                         hipStream_t s, Args... args) {
    launch_lds(kernel, grid, block, lds, s, args..., (int)block.x, (int)grid.x);
}

// Error codes returned by nova_get_last_error().
enum Status : int {
    kOk = 0,
    kErrInvalidArgument = 1,
    kErrNotInitialized = 2,
    kErrHip = 3,
    kErrWorkspace = 4,
    kErrOutOfMemory = 5,
};

void set_error(int code, const char* fmt, ...);

// Fused output epilogue: optional per-output-channel fp16 bias (device
// pointer, K values) and ReLU, applied where the output transform stores y.
struct Epilogue {
    const uint16_t* bias = nullptr;
    int relu = 0;
    const uint16_t* residual = nullptr;  // fp16, the output's layout (added after the bias)
};

// Minimal tiling used by the product path: ceil(Ho/6) x ceil(Wo/6) tiles.
inline int tiles_min(int out) { return (out + 5) / 6; }

// Pad a channel count to the 8-element (16-byte) granule of the GEMM loads.
inline int pad8(int c) { return (c + 7) & ~7; }

// Size of a buffer resource over an fp16 tensor read with loads of 4 bytes or
// more: a raw buffer load returns zero for a whole dword that extends past
// the resource's size (measured on MI355X: with 2 mod 4 bytes the tensor's
// last element read as zero), so the size is rounded up to the dword that
// holds the last element. The bytes added share that dword, hence its page;
// the kernels mask the columns they land in.
inline int64_t dword_ceil(int64_t bytes) { return (bytes + 3) & ~(int64_t)3; }

// ---- filter transform ----------------------------------------------------
// Reference layout: U[p][c][k] (U[p*K*C + c*K + k]).
hipError_t launch_filter_transform_ref(const float* w, uint16_t* U, int K, int C,
                                       hipStream_t s);
// Product layout: U[p][k][Cp], zero for c >= C (Cp = pad8(C)).
hipError_t launch_filter_transform_gemm(const void* w, bool w_f16, uint16_t* U, int K, int C,
                                        int Cp, hipStream_t s);

// Fragment-ordered copy of U for the fused kernels: for each position p,
// 16-row output-channel tile kt and 32-channel chunk j, one
// v_mfma_f32_16x16x32_f16 A operand per lane, 64 lanes x 8 halves, so a wave
// reads it as 1024 contiguous bytes (16 per lane). Lane l holds row
// 16*kt + l % 16 and channels 32*j + 16*ks + 4*(l / 16) + e for ks = 0, 1
// and e = 0..3 in that order: the two 16-channel halves of the chunk that a
// 16x16x16 fragment would put in lane l, side by side (a B operand built the
// same way pairs every channel with itself). Rows >= K and channels >= Cp are
// zero. Uf[((p*nkt + kt)*nkp + j)*512 + l*8 + ks*4 + e], nkt = ceil(K/16),
// nkp = ceil(Cp/32).
inline int64_t u_frag_elems(int K, int Cp) {
    return (int64_t)64 * ((K + 15) / 16) * ((Cp + 31) / 32) * 512;
}
hipError_t launch_u_frag(const uint16_t* U, uint16_t* Uf, int K, int Cp, hipStream_t s);
// The two-pass kernel's U blocks (three-pass GEMM lane layout, contiguous;
// same size as the fused kernels' copy).
hipError_t launch_u_wfrag(const uint16_t* U, uint16_t* Uw, int K, int Cp, hipStream_t s);

// Cache-policy operands of buffer stores. kNt (non-temporal) marks the lines
// for early eviction, but they still reach the L2 dirty. kWT (sc1, device
// scope) writes through the L2 to the memory side: the kernel's end then has
// no dirty lines to write back before the next launch may start. Measured on
// MI355X (a kernel that only stores, then an empty kernel; us, the stores'
// span + the gap to the next kernel's first wave): 16.8 MB write-back 1.92 +
// 2.39, nt 1.92 + 2.40, write-through 2.92 + 1.01; 50 MB 5.72 + 3.36 against
// 7.45 + 1.00; with nothing written the gap is 1.0-1.1. It pays where every
// store instruction of a wave writes whole 128-byte lines and the stores
// overlap the kernel's arithmetic: the V of the tile-block transforms in the
// product layout and of the run form, and the staged M tiles of the GEMM.
// Partial lines written through reach memory piece by piece (the
// lane-parallel and two-pass-layout tile-block V: 64@56^2 batch 8 two-pass
// 13.8 -> 16.3 us in a graph, SD-1.5 640@32^2 batch 2 (5.9 MB of V) 27.9 ->
// 29.8; the fused kernels' y rows: conv2_x batch 32 21.5 -> 26.6), except
// when they are few: partial-line V and M of at most kWTSmallBytes (batch-1
// layers) are written through too.
constexpr int kNt = 2;
constexpr int kWT = 16;
constexpr int64_t kWTSmallBytes = (int64_t)2 << 20;

// ---- input transform -----------------------------------------------------
// V[p*pstride + bp*ldv + c], bp = (b*nh + th)*nw + tw, for th < nh, tw < nw.
// Channels c in [C, ldv) are written as zero. x is NCHW, or NHWC if nhwc.
// V store cache policy (results unchanged): the forms whose wave stores are
// whole 128-byte lines (the tile-block forms in the product layout with at
// least 64 channels per workgroup and ldv % 64 == 0, and the run form) write
// through the L2; otherwise stream_v asks for the non-temporal (nt) policy
// (see wgemm_v_reads for when it pays).
// vfrag: 0 = V in the product layout V[p][bp][ldv]; otherwise the number of
// 32-channel chunks of the two-pass layout (1 KB MFMA B-operand blocks of 16
// tiles x 32 channels; pstride = ceil(BP / 16) * vfrag * 512 halves).
hipError_t launch_input_transform(const uint16_t* x, uint16_t* V, int B, int C, int H, int W,
                                  int pad, int nh, int nw, int ldv, int64_t pstride,
                                  hipStream_t s, bool nhwc = false, bool stream_v = false,
                                  int vfrag = 0);

// ---- output transform ----------------------------------------------------
// Reads M[p*pstride + bp*ldm + k]; writes y[b][k][h][w] (y[b][h][w][k] if
// nhwc) for h < Ho, w < Wo.
hipError_t launch_output_transform(const uint16_t* M, uint16_t* y, int B, int K, int Ho,
                                   int Wo, int nh, int nw, int ldm, int64_t pstride,
                                   hipStream_t s, Epilogue ep = Epilogue(), bool nhwc = false);

// ---- Winograd-domain batched GEMM ------------------------------------------
// For p in 0..63: M_p[bp][k] = sum_c U_p[k][c] * V_p[bp][c]  (fp32 accumulate,
// fp16 result). U: [64][K][Cp], V: [64][BP][Cp] (pitch Cp, zero padded), M:
// [64][BP][K].
hipError_t launch_wgemm(const uint16_t* U, const uint16_t* V, uint16_t* M, int K, int Cp,
                        int BP, hipStream_t s);
// Times the GEMM reads each V element (its output-channel tiles). Measured on
// MI355X (whole forwards): streaming V past the L2 pays when this is at most 4
// (ResNet-50 at batch 32: 128@28^2 31.7 -> 28.9 us, 256@14^2 31.2 -> 30.3,
// 512@7^2 29.0 -> 28.4) and costs when V is re-read more often (320@128^2 at
// batch 1, five reads: 43.1 -> 45.1 us; 640@64^2, ten: 36.7 -> 39.1 us).
int wgemm_v_reads(int K, int BP);
// Kernel name (template configuration) launch_wgemm picks for this shape.
const char* wgemm_name(int K, int Cp, int BP);
// GEMV-like shapes (BP <= 32, or 48 above K = 1024; U block copy under
// 2^31 bytes): the GEMM on
// operand blocks, Uw from launch_u_wfrag and V in the two-pass layout
// (launch_input_transform with vfrag = ceil(Cp / 32)); M as launch_wgemm's,
// bit-identical.
bool wgemm_blocks(int K, int Cp, int BP);
hipError_t launch_wgemm_blocks(const uint16_t* Uw, const uint16_t* Vb, uint16_t* M, int K,
                               int Cp, int BP, hipStream_t s);
const char* wgemm_blocks_name(int BP);

// ---- fused transform + GEMM + transform ------------------------------------
// Launch plan of the fused kernel for one shape: tile block (tbh x tbw tiles),
// output-channel block (16*nm channels), staging geometry, grid and the
// scratch it needs (M in fp16 and one uint32 counter per (tile block,
// channel block), which must be zero before the first launch; every launch
// leaves them zero).
struct FusedPlan {
    int tbh, tbw, nm, nbh, nbw, n_kb;
    int rr, rp, cp, nj;
    int64_t n_tb, grid, ms_bytes, cnt_count;
};
// False when the shape is outside the fused kernel's envelope.
bool fused_plan(int B, int C, int K, int Cp, int H, int W, int nh, int nw, FusedPlan* p);
bool fused_fits(int64_t x_elems, int64_t u_elems, int64_t y_elems);
const char* fused_name(const FusedPlan& p);
hipError_t launch_fused(const uint16_t* x, const uint16_t* U, uint16_t* y, uint16_t* Ms,
                        unsigned* cnt, int B, int C, int K, int Cp, int H, int W, int pad,
                        int nh, int nw, int Ho, int Wo, const FusedPlan& p, hipStream_t s,
                        Epilogue ep = Epilogue());

// Block variant (16-tile runs x 64 output channels x all positions per
// workgroup, no scratch): layers with few channels at batch > 1.
struct FusedBlockPlan {
    int nruns, n_kblk, rp, cp, nj;
    int cols;   // NHWC: staged pixels per row
    bool nhwc;  // x and y channels-last
    int64_t grid;
};
bool fused_block_plan(int B, int C, int K, int Cp, int H, int W, int nh, int nw,
                      FusedBlockPlan* p, bool nhwc = false);
hipError_t launch_fused_block(const uint16_t* x, const uint16_t* U, uint16_t* y, int B, int C,
                              int K, int Cp, int H, int W, int pad, int nh, int nw, int Ho,
                              int Wo, const FusedBlockPlan& p, hipStream_t s,
                              Epilogue ep = Epilogue());

// Small-problem variant (2 tiles x 16 output channels x all positions per
// workgroup, every workgroup recomputing its tiles' input transform; no
// scratch, no hand-off): C, K <= 64 when the other kernels' grids cannot
// fill the chip (batch 1).
struct FusedSmallPlan {
    int tiles;  // tiles per workgroup
    int tfirst; // first tile of each image (tiles before it are left to another launch)
    int ntg;    // tile groups per image, from tfirst on
    int nkb;    // 16-channel output blocks
    int threads;  // workgroup size: 512 or 1024
    int nkp;      // 32-channel input chunks held in LDS: 2 (C <= 64) or 4 (C <= 128)
    int64_t grid;
};
bool fused_small_plan(int B, int C, int K, int Cp, int nh, int nw, int cus,
                      FusedSmallPlan* p, int tfirst = 0, int tiles = 2);
hipError_t launch_fused_small(const uint16_t* x, const uint16_t* U, uint16_t* y, int B, int C,
                              int K, int Cp, int H, int W, int pad, int nh, int nw, int Ho,
                              int Wo, const FusedSmallPlan& p, hipStream_t s,
                              Epilogue ep = Epilogue(), bool nhwc = false);

// Two-pass forward, second pass (path 6): the products and the output
// transform of 16 tiles x 16 kb output channels per workgroup, U from the
// launch_u_wfrag blocks and V in the two-pass layout (launch_input_transform
// with vfrag = ceil(Cp / 32)); M stays in LDS.
// kb: 16-row tiles of U per workgroup (2: 32 output channels, one workgroup
// per CU; 1: 16 output channels, two per CU)
int64_t gemm_out_grid(int K, int BP, int kb = 2);
int gemm_out_kb(int K, int BP, int cus);  // the kb launch_gemm_out takes on a chip of cus CUs
int64_t gemm_out_v_elems(int Cp, int64_t BP);  // V halves of the two-pass layout
hipError_t launch_gemm_out(const uint16_t* Uw, const uint16_t* V, uint16_t* y, int B, int K,
                           int Cp, int nh, int nw, int Ho, int Wo, hipStream_t s, Epilogue ep,
                           bool nhwc, int kb = 2);

// Input transform fused into the products (path 7), for GEMV-like shapes
// (few tiles, many channels): workgroup = position row x group of nt <= 16
// tiles x kr 16-row output-channel tiles; each builds the V slice its
// products need in LDS and writes M in the product layout [64][BP][K] (the
// output transform follows as its own launch). U from launch_u_wfrag's
// blocks. M equals the three-pass path's bit for bit.
struct InGemmPlan {
    int nt;      // tiles per workgroup
    int ntg;     // tile groups
    int kr;      // 16-row output-channel tiles per workgroup (1 or 2)
    int nkg;     // output-channel groups
    int nsteps;  // 32-channel steps
    int nsm;     // steps the kernel instantiation holds (4, 8 or 16)
    int64_t grid;
};
// False when the shape is outside the kernel's envelope (more than 64 tiles,
// more than 512 channels, pads above 4, 32-bit offsets).
bool in_gemm_plan(int B, int C, int K, int Cp, int nh, int nw, int pad, int cus,
                  InGemmPlan* p);
const char* in_gemm_name(const InGemmPlan& p);
hipError_t launch_in_gemm(const uint16_t* x, const uint16_t* Uw, uint16_t* M, int B, int C,
                          int K, int Cp, int H, int W, int pad, int nh, int nw,
                          const InGemmPlan& p, hipStream_t s, bool nhwc);

// ---- weight gradient (Winograd domain, fp32) --------------------------------
// Plan of a weight-gradient computation: images per sub-batch (the fp32
// transformed operands stay below 2^31 bytes each and 1 GiB together), the
// padded tile count of the largest sub-batch, the number of splits of the
// tile range in the products, the workspace it needs, and whether the shape
// fits the kernels' 32-bit offsets at all.
struct WgradPlan {
    int chunk_images;
    int nsplit;  // partial filters: ranges of the tile index
    int64_t BPp_max;
    int64_t ws_bytes;
    bool ok;
};
WgradPlan wgrad_plan(int B, int C, int K, int H, int W, int pad, int cus);
// dw[K][C][3][3] (fp32, overwritten) for x fp16 [B][C][H][W] and dY
// [B][K][Ho][Wo] (fp16, or fp32 if dy_f32); ws holds plan.ws_bytes.
hipError_t launch_wgrad(const uint16_t* x, const void* dy, bool dy_f32, float* dw, int B, int C,
                        int K, int H, int W, int pad, const WgradPlan& plan, void* ws,
                        hipStream_t s);

}  // namespace nova
