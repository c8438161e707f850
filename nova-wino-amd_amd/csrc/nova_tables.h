// NOVA F(6,3) transform tables for the points {0, 3/5, -3/5, 1, -1, 7/6, -7/6, inf}.
//
// Values: the exact Cook-Toom rationals for those points rounded to fp32 (they
// equal the reference's fp32 tables bit for bit,
// /root/reference/csrc/nova_winograd.hip:68-97). As in the reference's
// constant upload (/root/reference/csrc/nova_winograd.hip:103-131), A and B
// enter the transforms rounded to fp16 (kAh, kBh, stored here as the fp32
// value of that fp16), while G stays fp32 (kG).
//
//   A (6x8): A[r][i] = a_i^r, infinity column = e_5
//   B (8x8): column i = coefficients of prod_{j != i} (x - a_j), infinity
//            column = coefficients of prod_j (x - a_j)
//   G (8x3): row i = [1, a_i, a_i^2] / prod_{j != i} (a_i - a_j), infinity
//            row = [0, 0, 1]
//
// Transforms: V = B^T d B (8x8 input patch d), U = G w G^T (3x3 filter w),
// Y = A M A^T (6x6 output tile). The arrays are constexpr so that fully
// unrolled transform loops see compile-time coefficients (zero terms vanish).
#pragma once

namespace nova {

constexpr float kG[8][3] = {
    {-0x1.053978p+1f, 0x0p+0f, 0x0p+0f},
    {0x1.15783p+1f, 0x1.4cf6ap+0f, 0x1.8f8e5ap-1f},
    {0x1.15783p+1f, -0x1.4cf6ap+0f, 0x1.8f8e5ap-1f},
    {-0x1.14ec4ep+1f, -0x1.14ec4ep+1f, -0x1.14ec4ep+1f},
    {-0x1.14ec4ep+1f, 0x1.14ec4ep+1f, -0x1.14ec4ep+1f},
    {0x1.0421b6p+0f, 0x1.2f7caap+0f, 0x1.62117p+0f},
    {0x1.0421b6p+0f, -0x1.2f7caap+0f, 0x1.62117p+0f},
    {0x0p+0f, 0x0p+0f, 0x1p+0f}};

// fp16(A) as fp32
constexpr float kAh[6][8] = {
    {0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.334p-1f, -0x1.334p-1f, 0x1p+0f, -0x1p+0f, 0x1.2acp+0f, -0x1.2acp+0f, 0x0p+0f},
    {0x0p+0f, 0x1.70cp-2f, 0x1.70cp-2f, 0x1p+0f, 0x1p+0f, 0x1.5c8p+0f, 0x1.5c8p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.ba4p-3f, -0x1.ba4p-3f, 0x1p+0f, -0x1p+0f, 0x1.968p+0f, -0x1.968p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.098p-3f, 0x1.098p-3f, 0x1p+0f, 0x1p+0f, 0x1.da4p+0f, 0x1.da4p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.3e8p-4f, -0x1.3e8p-4f, 0x1p+0f, -0x1p+0f, 0x1.14cp+1f, -0x1.14cp+1f, 0x1p+0f}};

// fp16(B) as fp32
constexpr float kBh[8][8] = {
    {-0x1.f5cp-2f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.a24p-1f, -0x1.a24p-1f, 0x1.f5cp-2f, -0x1.f5cp-2f, 0x1.aep-2f, -0x1.aep-2f, -0x1.f5cp-2f},
    {0x1.1bp+1f, 0x1.5c8p+0f, 0x1.5c8p+0f, 0x1.f5cp-2f, 0x1.f5cp-2f, 0x1.70cp-2f, 0x1.70cp-2f, 0x0p+0f},
    {0x0p+0f, -0x1.6acp+0f, 0x1.6acp+0f, -0x1.b88p+0f, 0x1.b88p+0f, -0x1.964p+0f, 0x1.964p+0f, 0x1.1bp+1f},
    {-0x1.5c4p+1f, -0x1.2e4p+1f, -0x1.2e4p+1f, -0x1.b88p+0f, -0x1.b88p+0f, -0x1.5c4p+0f, -0x1.5c4p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.334p-1f, -0x1.334p-1f, 0x1p+0f, -0x1p+0f, 0x1.2acp+0f, -0x1.2acp+0f, -0x1.5c4p+1f},
    {0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x0p+0f},
    {0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x1p+0f}};

}  // namespace nova
