// Internal interfaces between the translation units of libnova_winograd.so.
// Nothing here is exported; the public C-ABI is include/nova_winograd.h.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace nova {

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

// Minimal tiling used by the product path: ceil(Ho/6) x ceil(Wo/6) tiles.
inline int tiles_min(int out) { return (out + 5) / 6; }

// Pad a channel count to the 8-element (16-byte) granule of the GEMM loads.
inline int pad8(int c) { return (c + 7) & ~7; }

// ---- filter transform ----------------------------------------------------
// Reference layout: U[p][c][k] (U[p*K*C + c*K + k]).
hipError_t launch_filter_transform_ref(const float* w, uint16_t* U, int K, int C,
                                       hipStream_t s);
// Product layout: U[p][k][Cp], zero for c >= C (Cp = pad8(C)).
hipError_t launch_filter_transform_gemm(const float* w, uint16_t* U, int K, int C, int Cp,
                                        hipStream_t s);

// ---- input transform -----------------------------------------------------
// V[p*pstride + bp*ldv + c], bp = (b*nh + th)*nw + tw, for th < nh, tw < nw.
// Channels c in [C, ldv) are written as zero.
hipError_t launch_input_transform(const uint16_t* x, uint16_t* V, int B, int C, int H, int W,
                                  int pad, int nh, int nw, int ldv, int64_t pstride,
                                  hipStream_t s);

// ---- output transform ----------------------------------------------------
// Reads M[p*pstride + bp*ldm + k]; writes y[b][k][h][w] for h < Ho, w < Wo.
hipError_t launch_output_transform(const uint16_t* M, uint16_t* y, int B, int K, int Ho,
                                   int Wo, int nh, int nw, int ldm, int64_t pstride,
                                   hipStream_t s);

// ---- Winograd-domain batched GEMM ------------------------------------------
// For p in 0..63: M_p[bp][k] = sum_c U_p[k][c] * V_p[bp][c]  (fp32 accumulate,
// fp16 result). U: [64][K][Cp], V: [64][BP][Cp] (pitch Cp, zero padded), M:
// [64][BP][K].
hipError_t launch_wgemm(const uint16_t* U, const uint16_t* V, uint16_t* M, int K, int Cp,
                        int BP, hipStream_t s);
// Kernel name (template configuration) launch_wgemm picks for this shape.
const char* wgemm_name(int K, int Cp, int BP);

// ---- fused transform + GEMM + transform ------------------------------------
// Returns false when the shape is outside the fused kernel's envelope.
bool fused_supported(int K, int C);
bool fused_fits(int64_t x_elems, int64_t u_elems, int64_t y_elems);
const char* fused_name(int K, int C, int64_t BP);
hipError_t launch_fused(const uint16_t* x, const uint16_t* U, uint16_t* y, int B, int C,
                        int K, int Cp, int H, int W, int pad, int nh, int nw, int Ho,
                        int Wo, hipStream_t s);

}  // namespace nova
