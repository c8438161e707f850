// Per-tile NOVA F(6,3) transform arithmetic, shared by the standalone
// transform kernels and the fused kernel.
//
// Order of operations (the contract the CPU oracle restates):
//   input : t[r][j] = fma-chain_i  Bh[i][r] * d[i][j]        (i = 0..7)
//           v[r][s] = fma-chain_j  t[r][j]  * Bh[j][s]        (j = 0..7)
//   output: t[r][j] = fma-chain_i  Ah[r][i] * m[i][j]         (r < 6)
//           y[r][s] = fma-chain_j  t[r][j]  * Ah[s][j]        (s < 6)
//   filter: u[r][s] = fma-chain_{p,q} (G[r][p]*w[p][q]) * G[s][q]
// Chains start at +0 and skip terms whose table coefficient is zero (input
// and output only). Loops are fully unrolled so that the constexpr tables fold
// into immediates and the zero tests disappear at compile time.
#pragma once

#include "nova_tables.h"

namespace nova {

// Round an fp32 value to fp16 (nearest even) *as an fp32 value*. The empty asm
// pins v in a register, which stops the compiler from fusing the producing
// fma with the conversion into v_fma_mix{lo,hi}_f16 -- that instruction rounds
// the exact fma result straight to fp16 (one rounding) and differs from
// fp32-then-fp16 when the fp32 result lands on an fp16 tie.
__device__ __forceinline__ _Float16 to_f16(float v) {
    asm("" : "+v"(v));
    return (_Float16)v;
}

// Two fp32 values rounded to fp16 (nearest even) and packed, lo in the low
// half: one v_cvt_pk_f16_f32, the same bits as two to_f16 calls (the empty
// asm keeps each value a separate fp32 rounding, as in to_f16).
__device__ __forceinline__ unsigned pack_f16x2(float lo, float hi) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    asm("" : "+v"(lo));
    asm("" : "+v"(hi));
    return __builtin_bit_cast(unsigned, __builtin_convertvector(f2{lo, hi}, h2));
}

// Output epilogue for channel k: the convolution value rounded to fp16, then
// the reference's separate bias add (`y + bias.half()`: fp16 + fp16 summed in
// fp32, rounded once) and an optional ReLU (negative values -> 0). bias is a
// device array of K fp16 values, or null.
__device__ __forceinline__ _Float16 epilogue(float v, const _Float16* bias, int k, int relu) {
    _Float16 h = to_f16(v);
    if (bias != nullptr) h = to_f16((float)h + (float)bias[k]);
    if (relu && (float)h < 0.0f) h = (_Float16)0.0f;
    return h;
}

// epilogue() for one output channel, with the channel's bias read once. With
// kEpi false the kernel was launched without bias and without a ReLU at this
// stage (none, or one that follows a residual add), and the value is only
// rounded to fp16: no per-value bias or ReLU code at all.
template <bool kEpi>
struct ChannelEpilogue {
    bool hb = false;
    float bk = 0.0f;
    int relu = 0;
    __device__ ChannelEpilogue(const _Float16* bias, int k, int relu_) {
        if constexpr (kEpi) {
            hb = bias != nullptr;
            bk = hb ? (float)bias[k] : 0.0f;
            relu = relu_;
        }
    }
    __device__ _Float16 operator()(float v) const {
        _Float16 h = to_f16(v);
        if constexpr (kEpi) {
            if (hb) h = to_f16((float)h + bk);
            if (relu && (float)h < 0.0f) h = (_Float16)0.0f;
        }
        return h;
    }
};

// Whether a launch needs ChannelEpilogue<true>: a bias, or a ReLU that is not
// deferred to a residual add.
inline bool epilogue_needed(const void* bias, int relu, const void* residual) {
    return bias != nullptr || (relu != 0 && residual == nullptr);
}

// Residual stage of the epilogue, after the bias: h plus the residual value
// r (fp16 + fp16 summed in fp32, rounded once -- a separate `y + residual` on
// fp16 tensors), then the optional ReLU. With a residual the ReLU is applied
// here and not in epilogue().
__device__ __forceinline__ _Float16 add_residual(_Float16 h, _Float16 r, int relu) {
    _Float16 o = to_f16((float)h + (float)r);
    if (relu && (float)o < 0.0f) o = (_Float16)0.0f;
    return o;
}

// add_residual on two packed halves (low half = lower address).
__device__ __forceinline__ unsigned add_residual2(unsigned h2, unsigned r2, int relu) {
    const _Float16 lo = add_residual(__builtin_bit_cast(_Float16, (unsigned short)(h2 & 0xffffu)),
                                     __builtin_bit_cast(_Float16, (unsigned short)(r2 & 0xffffu)),
                                     relu);
    const _Float16 hi = add_residual(__builtin_bit_cast(_Float16, (unsigned short)(h2 >> 16)),
                                     __builtin_bit_cast(_Float16, (unsigned short)(r2 >> 16)), relu);
    return (unsigned)__builtin_bit_cast(unsigned short, lo) |
           ((unsigned)__builtin_bit_cast(unsigned short, hi) << 16);
}

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own
// L2. This bijection maps the dispatch index L (0..N-1) to a work index such
// that every XCD receives one contiguous range of work items, so spatial
// neighbours (overlapping input strips, shared cache lines) meet in the same
// L2. Correctness does not depend on the dispatch order.
__device__ __forceinline__ int xcd_remap(int L, int N) {
    constexpr int kXcds = 8;
    const int q = N / kXcds, r = N % kXcds;
    const int xcd = L % kXcds, slot = L / kXcds;
    const int start = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
    return start + slot;
}

// An SGPR holding 1.0 that the optimizer cannot see through. A first-pass
// term multiplies a table coefficient by an fp16 value widened to fp32; with a
// coefficient of +-1 the compiler folds fma(c, x, acc) into acc +- x, which
// needs x converted to fp32 by an instruction of its own, while fma(c, x, acc)
// is one v_fma_mix_f32 that reads the fp16 operand in place. Both round once,
// to the same value.
__device__ __forceinline__ float opaque_one() {
    float one = 1.0f;
    asm("" : "+s"(one));
    return one;
}

// Table coefficient c of a first-pass fma (see opaque_one).
__device__ __forceinline__ float mix_coef(float c, float one) {
    return c == 1.0f ? one : c == -1.0f ? -one : c;
}

// Input tile: ld(i, j) returns d[i][j] as fp32. Processes one input column j
// at a time, which keeps every v[r][s] chain in j order.
template <typename Load>
__device__ __forceinline__ void input_tile(Load ld, float v[8][8]) {
    const float one = opaque_one();
#pragma unroll
    for (int r = 0; r < 8; r++)
#pragma unroll
        for (int s = 0; s < 8; s++) v[r][s] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float d[8];
#pragma unroll
        for (int i = 0; i < 8; i++) d[i] = ld(i, j);
        float t[8];
#pragma unroll
        for (int r = 0; r < 8; r++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (kBh[i][r] != 0.0f)
                    acc = __builtin_fmaf(mix_coef(kBh[i][r], one), d[i], acc);
            t[r] = acc;
        }
#pragma unroll
        for (int r = 0; r < 8; r++)
#pragma unroll
            for (int s = 0; s < 8; s++)
                if (kBh[j][s] != 0.0f) v[r][s] = __builtin_fmaf(t[r], kBh[j][s], v[r][s]);
    }
}

// Input tile evaluated row by row (same per-element chains as input_tile):
// row r of T = B^T d needs all of d, row r of V needs only row r of T, so
// only d plus two 8-vectors are live. ld(i, j) returns d[i][j] as fp32 and
// st(r, s, v) consumes each V value.
template <typename Load, typename Store>
__device__ __forceinline__ void input_tile_rows(Load ld, Store st) {
    const float one = opaque_one();
#pragma unroll
    for (int r = 0; r < 8; r++) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (kBh[i][r] != 0.0f)
                    acc = __builtin_fmaf(mix_coef(kBh[i][r], one), ld(i, j), acc);
            t[j] = acc;
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (kBh[j][s] != 0.0f) acc = __builtin_fmaf(t[j], kBh[j][s], acc);
            st(r, s, acc);
        }
    }
}

// Row I of V = B^T d B for one patch (positions 8*I .. 8*I+7), with the same
// per-element chains as input_tile_rows: t[j] over i ascending, then
// v[I][s] over j ascending. Only the input rows i with B[i][I] != 0 are read.
template <int I, typename Load>
__device__ __forceinline__ void input_row(Load ld, float out[8]) {
    const float one = opaque_one();
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (kBh[i][I] != 0.0f)
                acc = __builtin_fmaf(mix_coef(kBh[i][I], one), ld(i, j), acc);
        t[j] = acc;
    }
#pragma unroll
    for (int s = 0; s < 8; s++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (kBh[j][s] != 0.0f) acc = __builtin_fmaf(t[j], kBh[j][s], acc);
        out[s] = acc;
    }
}

// input_row with the columns outside the image zeroed after the first pass
// (bit j of cols clear: t[j] = +0, what all-zero inputs give, since the chain
// starts at +0), so ld(i, j) may return anything for such a column.
template <int I, typename Load>
__device__ __forceinline__ void input_row_masked(Load ld, unsigned cols, float out[8]) {
    const float one = opaque_one();
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (kBh[i][I] != 0.0f)
                acc = __builtin_fmaf(mix_coef(kBh[i][I], one), ld(i, j), acc);
        t[j] = ((cols >> j) & 1u) ? acc : 0.0f;
    }
#pragma unroll
    for (int s = 0; s < 8; s++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (kBh[j][s] != 0.0f) acc = __builtin_fmaf(t[j], kBh[j][s], acc);
        out[s] = acc;
    }
}

// True when input row i enters row I of V (B[i][I] != 0).
constexpr bool input_row_uses(int I, int i) { return kBh[i][I] != 0.0f; }

// Output tile: ld(i, j) returns m[i][j] (position 8*i+j) as fp32.
template <typename Load>
__device__ __forceinline__ void output_tile(Load ld, float y[6][6]) {
    const float one = opaque_one();
#pragma unroll
    for (int r = 0; r < 6; r++)
#pragma unroll
        for (int s = 0; s < 6; s++) y[r][s] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float m[8];
#pragma unroll
        for (int i = 0; i < 8; i++) m[i] = ld(i, j);
        float t[6];
#pragma unroll
        for (int r = 0; r < 6; r++) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (kAh[r][i] != 0.0f)
                    acc = __builtin_fmaf(mix_coef(kAh[r][i], one), m[i], acc);
            t[r] = acc;
        }
#pragma unroll
        for (int r = 0; r < 6; r++)
#pragma unroll
            for (int s = 0; s < 6; s++)
                if (kAh[s][j] != 0.0f) y[r][s] = __builtin_fmaf(t[r], kAh[s][j], y[r][s]);
    }
}

// Filter tile: all 9 terms, t = G[r][p]*w[p][q] rounded to fp32 first.
__device__ __forceinline__ void filter_tile(const float w[3][3], float u[8][8]) {
#pragma unroll
    for (int r = 0; r < 8; r++)
#pragma unroll
        for (int s = 0; s < 8; s++) {
            float acc = 0.0f;
#pragma unroll
            for (int p = 0; p < 3; p++)
#pragma unroll
                for (int q = 0; q < 3; q++) {
                    const float t = kG[r][p] * w[p][q];
                    acc = __builtin_fmaf(t, kG[s][q], acc);
                }
            u[r][s] = acc;
        }
}

}  // namespace nova
