/*
 * NOVA F(6,3) Winograd convolution: CPU oracle (TEST INFRASTRUCTURE ONLY).
 *
 * This file is the checker, not the product. Only tests/, the smoke() entry
 * point and bench.py's cpu_baseline leg may load it. The product library in
 * nova-wino-amd_amd/ never links or calls it.
 *
 * It restates, in plain C, the arithmetic of the reference's 3-pass NOVA path:
 *   tables       /root/reference/csrc/nova_winograd.hip:68-97 (values),
 *                :103-131 (A, B rounded to fp16, G kept fp32)
 *   tiling       /root/reference/csrc/nova_winograd.hip:617-631
 *   filter       /root/reference/csrc/nova_winograd.hip:214-255
 *   input        /root/reference/csrc/nova_winograd.hip:336-392 (and :141-205)
 *   batched GEMM /root/reference/csrc/nova_winograd.hip:589-601 (rocBLAS:
 *                fp16 operands, fp32 accumulate, fp16 result)
 *   output       /root/reference/csrc/nova_winograd.hip:398-450 (and :264-328)
 *   direct conv  /root/reference/csrc/nova_winograd.hip:637-669 (truth; here
 *                accumulated in double)
 *
 * Layouts are the reference's GEMM layouts:
 *   x  fp16 [B][C][H][W]            w  fp32 [K][C][3][3]
 *   U  fp16 [64][C][K]   (U[p*K*C + c*K + k])
 *   V  fp16 [64][BP][C]  (V[p*C*BP + bp*C + c]),  bp = b*nh*nw + th*nw + tw
 *   M  fp16 [64][BP][K]  (M[p*K*BP + bp*K + k])
 *   y  fp16 [B][K][Ho][Wo]
 *
 * Canonical arithmetic (what "bit-exact" means for this path):
 *   - every fp32 dot product is a chain of fused multiply-adds in the
 *     reference's loop order, starting from +0;
 *   - in the input and output transforms, terms whose table coefficient is
 *     zero are skipped (for finite operands fma(0, x, acc) == acc exactly,
 *     because acc is never -0 when the chain starts at +0);
 *   - the filter transform keeps all 9 terms: t = G[r][p]*w[p][q] rounded to
 *     fp32, then acc = fma(t, G[s][q], acc);
 *   - V, U, Y are rounded once to fp16 (round to nearest even);
 *   - the Winograd-domain GEMM has no specified order in the reference
 *     (rocBLAS); here it is accumulated in double and rounded once to fp16,
 *     i.e. it is the correctly rounded M. GPU results are compared with it
 *     under an explicit error bound, never bit-for-bit.
 * Stage 1 of both transforms multiplies fp16 values by fp16 constants; those
 * products are exact in fp32, so FMA and separate multiply+add agree there.
 * For non-finite inputs the NaN pattern may differ from the reference, which
 * also multiplies the zero coefficients.
 *
 * Parity pins (tests/test_oracle.py): tables derived exactly from the points;
 * exact-arithmetic Winograd == direct correlation; fp16 conversion against
 * numpy; tiling law by brute force; zero / delta / constant / linearity
 * special cases; whole-path error vs fp64 direct conv at the reference's
 * published level (rel-L2 ~5e-2); committed golden fixtures.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* Tables: fp32 values of the exact rationals for the points                */
/* {0, 3/5, -3/5, 1, -1, 7/6, -7/6, inf} (derived in derive_tables.py).      */
/* ------------------------------------------------------------------------ */
static const float kA[6][8] = {
    {0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.333334p-1f, -0x1.333334p-1f, 0x1p+0f, -0x1p+0f, 0x1.2aaaaap+0f, -0x1.2aaaaap+0f, 0x0p+0f},
    {0x0p+0f, 0x1.70a3d8p-2f, 0x1.70a3d8p-2f, 0x1p+0f, 0x1p+0f, 0x1.5c71c8p+0f, 0x1.5c71c8p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.ba5e36p-3f, -0x1.ba5e36p-3f, 0x1p+0f, -0x1p+0f, 0x1.9684bep+0f, -0x1.9684bep+0f, 0x0p+0f},
    {0x0p+0f, 0x1.096bbap-3f, 0x1.096bbap-3f, 0x1p+0f, 0x1p+0f, 0x1.da4588p+0f, 0x1.da4588p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.3e8146p-4f, -0x1.3e8146p-4f, 0x1p+0f, -0x1p+0f, 0x1.14a89p+1f, -0x1.14a89p+1f, 0x1p+0f}};

static const float kB[8][8] = {
    {-0x1.f5c29p-2f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.a22222p-1f, -0x1.a22222p-1f, 0x1.f5c29p-2f, -0x1.f5c29p-2f, 0x1.ae147ap-2f, -0x1.ae147ap-2f, -0x1.f5c29p-2f},
    {0x1.1b05bp+1f, 0x1.5c71c8p+0f, 0x1.5c71c8p+0f, 0x1.f5c29p-2f, 0x1.f5c29p-2f, 0x1.70a3d8p-2f, 0x1.70a3d8p-2f, 0x0p+0f},
    {0x0p+0f, -0x1.6aaaaap+0f, 0x1.6aaaaap+0f, -0x1.b89abcp+0f, 0x1.b89abcp+0f, -0x1.962fcap+0f, 0x1.962fcap+0f, 0x1.1b05bp+1f},
    {-0x1.5c4d5ep+1f, -0x1.2e38e4p+1f, -0x1.2e38e4p+1f, -0x1.b89abcp+0f, -0x1.b89abcp+0f, -0x1.5c28f6p+0f, -0x1.5c28f6p+0f, 0x0p+0f},
    {0x0p+0f, 0x1.333334p-1f, -0x1.333334p-1f, 0x1p+0f, -0x1p+0f, 0x1.2aaaaap+0f, -0x1.2aaaaap+0f, -0x1.5c4d5ep+1f},
    {0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x1p+0f, 0x0p+0f},
    {0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x0p+0f, 0x1p+0f}};

static const float kG[8][3] = {
    {-0x1.053978p+1f, 0x0p+0f, 0x0p+0f},
    {0x1.157830p+1f, 0x1.4cf6ap+0f, 0x1.8f8e5ap-1f},
    {0x1.157830p+1f, -0x1.4cf6ap+0f, 0x1.8f8e5ap-1f},
    {-0x1.14ec4ep+1f, -0x1.14ec4ep+1f, -0x1.14ec4ep+1f},
    {-0x1.14ec4ep+1f, 0x1.14ec4ep+1f, -0x1.14ec4ep+1f},
    {0x1.0421b6p+0f, 0x1.2f7caap+0f, 0x1.62117p+0f},
    {0x1.0421b6p+0f, -0x1.2f7caap+0f, 0x1.62117p+0f},
    {0x0p+0f, 0x0p+0f, 0x1p+0f}};

/* ------------------------------------------------------------------------ */
/* IEEE binary16 conversions (round to nearest even, subnormals, inf, NaN)   */
/* ------------------------------------------------------------------------ */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) { /* inf / nan */
        if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    if (e <= 0) {                                   /* subnormal or zero */
        if (e < -10) return (uint16_t)sign;         /* below half the smallest subnormal */
        man |= 0x800000u;
        int shift = 14 - e; /* 14..24 */
        uint32_t q = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q); /* q may carry into the exponent: still correct */
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* carry may reach inf: correct */
    return (uint16_t)(sign | q);
}

static uint16_t f64_to_f16(double d) {
    /* exact single rounding from double: scale into an integer grid */
    if (isnan(d)) return 0x7e00u;
    uint16_t sign = signbit(d) ? 0x8000u : 0u;
    double a = fabs(d);
    if (isinf(a)) return (uint16_t)(sign | 0x7c00u);
    if (a == 0.0) return sign;
    int e;
    frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) -> unbiased exponent e-1 */
    int ue = e - 1;
    if (ue < -14) ue = -14;              /* subnormal quantum 2^-24 */
    double quantum = ldexp(1.0, ue - 10);
    double q = a / quantum;              /* exact: power-of-two scaling */
    double fl = floor(q);
    double rem = q - fl;
    if (rem > 0.5 || (rem == 0.5 && fmod(fl, 2.0) == 1.0)) fl += 1.0;
    double v = fl * quantum;
    if (v >= 65520.0 || v > 65504.0) return (uint16_t)(sign | 0x7c00u);
    /* v is exactly representable in fp16; convert through float (exact) */
    return (uint16_t)(sign | (f32_to_f16((float)v) & 0x7fffu));
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        x = sign | 0x7f800000u | (man << 13);
    } else {
        x = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* fp16-rounded A and B, as the reference uploads them */
static float Ah[6][8], Bh[8][8];
static int tables_ready = 0;

static void init_tables(void) {
    if (tables_ready) return;
    for (int i = 0; i < 6; i++)
        for (int j = 0; j < 8; j++) Ah[i][j] = f16_to_f32(f32_to_f16(kA[i][j]));
    for (int i = 0; i < 8; i++)
        for (int j = 0; j < 8; j++) Bh[i][j] = f16_to_f32(f32_to_f16(kB[i][j]));
    tables_ready = 1;
}

/* ------------------------------------------------------------------------ */
/* Exported API (ctypes)                                                     */
/* ------------------------------------------------------------------------ */
void nvo_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int nvo_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void nvo_tables(float* A, float* B, float* G, float* Ah_out, float* Bh_out) {
    init_tables();
    memcpy(A, kA, sizeof(kA));
    memcpy(B, kB, sizeof(kB));
    memcpy(G, kG, sizeof(kG));
    memcpy(Ah_out, Ah, sizeof(Ah));
    memcpy(Bh_out, Bh, sizeof(Bh));
}

void nvo_f32_to_f16(const float* in, uint16_t* out, long n) {
    for (long i = 0; i < n; i++) out[i] = f32_to_f16(in[i]);
}

void nvo_f64_to_f16(const double* in, uint16_t* out, long n) {
    for (long i = 0; i < n; i++) out[i] = f64_to_f16(in[i]);
}

void nvo_f16_to_f32(const uint16_t* in, float* out, long n) {
    for (long i = 0; i < n; i++) out[i] = f16_to_f32(in[i]);
}

/* Tiling law (/root/reference/csrc/nova_winograd.hip:617-631). */
void nvo_tiling(int H, int W, int pad, int* nh, int* nw, int* Ho, int* Wo) {
    const int m = 6, n = 8;
    *Ho = H + 2 * pad - 2;
    *Wo = W + 2 * pad - 2;
    int hp = *Ho + n - 1, wp = *Wo + n - 1;
    hp += (m - (hp - n) % m) % m;
    wp += (m - (wp - n) % m) % m;
    *nh = (hp - n) / m + 1;
    *nw = (wp - n) / m + 1;
}

/* Filter transform (/root/reference/csrc/nova_winograd.hip:214-255). */
void nvo_filter(const float* w, int K, int C, uint16_t* U) {
    long KC = (long)K * C;
#pragma omp parallel for schedule(static)
    for (long kc = 0; kc < KC; kc++) {
        int k = (int)(kc / C), c = (int)(kc % C);
        const float* wp = w + kc * 9;
        for (int r = 0; r < 8; r++)
            for (int s = 0; s < 8; s++) {
                float acc = 0.0f;
                for (int p = 0; p < 3; p++)
                    for (int q = 0; q < 3; q++) {
                        float t = kG[r][p] * wp[p * 3 + q];
                        acc = fmaf(t, kG[s][q], acc);
                    }
                U[(long)(r * 8 + s) * KC + (long)c * K + k] = f32_to_f16(acc);
            }
    }
}

/* V = B^T d B for one 8x8 patch (d already fp32), canonical order. */
static void input_tile(const float d[8][8], float v[8][8]) {
    float t[8][8];
    for (int r = 0; r < 8; r++)
        for (int j = 0; j < 8; j++) {
            float acc = 0.0f;
            for (int i = 0; i < 8; i++)
                if (Bh[i][r] != 0.0f) acc = fmaf(Bh[i][r], d[i][j], acc);
            t[r][j] = acc;
        }
    for (int r = 0; r < 8; r++)
        for (int s = 0; s < 8; s++) {
            float acc = 0.0f;
            for (int j = 0; j < 8; j++)
                if (Bh[j][s] != 0.0f) acc = fmaf(t[r][j], Bh[j][s], acc);
            v[r][s] = acc;
        }
}

/* Input transform (/root/reference/csrc/nova_winograd.hip:336-392). */
void nvo_input(const uint16_t* x, int B, int C, int H, int W, int pad, int nh, int nw,
               uint16_t* V) {
    init_tables();
    long P = (long)nh * nw, BP = (long)B * P;
    long total = BP * C;
#pragma omp parallel for schedule(static)
    for (long idx = 0; idx < total; idx++) {
        long bp = idx / C;
        int c = (int)(idx % C);
        int b = (int)(bp / P);
        int tile = (int)(bp % P);
        int th = tile / nw, tw = tile % nw;
        float d[8][8], v[8][8];
        for (int i = 0; i < 8; i++)
            for (int j = 0; j < 8; j++) {
                int h = th * 6 - pad + i, ww = tw * 6 - pad + j;
                d[i][j] = (h >= 0 && h < H && ww >= 0 && ww < W)
                              ? f16_to_f32(x[(((long)b * C + c) * H + h) * W + ww])
                              : 0.0f;
            }
        input_tile(d, v);
        for (int r = 0; r < 8; r++)
            for (int s = 0; s < 8; s++)
                V[(long)(r * 8 + s) * C * BP + bp * C + c] = f32_to_f16(v[r][s]);
    }
}

/* Winograd-domain batched GEMM (/root/reference/csrc/nova_winograd.hip:589-601):
 * M[p] = U[p] (K x C) * V[p] (C x BP).  Accumulated in double, rounded once.
 * Mabs (optional) receives sum_c |U||V| in fp32 for error bounds. */
void nvo_gemm(const uint16_t* U, const uint16_t* V, int K, int C, long BP, uint16_t* M,
              float* Mabs) {
    long KC = (long)K * C;
#pragma omp parallel for schedule(static)
    for (long pb = 0; pb < 64 * BP; pb++) {
        int p = (int)(pb / BP);
        long bp = pb % BP;
        const uint16_t* Up = U + p * KC;
        const uint16_t* Vp = V + (long)p * C * BP + bp * C;
        float vf[4096];
        double* acc = (double*)malloc(sizeof(double) * K);
        double* aab = Mabs ? (double*)malloc(sizeof(double) * K) : NULL;
        for (int k = 0; k < K; k++) { acc[k] = 0.0; if (aab) aab[k] = 0.0; }
        for (int c0 = 0; c0 < C; c0 += 4096) {
            int cn = C - c0 < 4096 ? C - c0 : 4096;
            for (int c = 0; c < cn; c++) vf[c] = f16_to_f32(Vp[c0 + c]);
            for (int c = 0; c < cn; c++) {
                const uint16_t* Uc = Up + (long)(c0 + c) * K;
                double vv = vf[c];
                for (int k = 0; k < K; k++) {
                    double prod = (double)f16_to_f32(Uc[k]) * vv;
                    acc[k] += prod;
                    if (aab) aab[k] += fabs(prod);
                }
            }
        }
        uint16_t* Mp = M + (long)p * K * BP + bp * K;
        for (int k = 0; k < K; k++) {
            Mp[k] = f64_to_f16(acc[k]);
            if (Mabs) Mabs[(long)p * K * BP + bp * K + k] = (float)aab[k];
        }
        free(acc);
        free(aab);
    }
}

/* Y = A M A^T for one tile (m fp32 8x8), canonical order; returns 6x6. */
static void output_tile(const float m[8][8], float y[6][6]) {
    float t[6][8];
    for (int r = 0; r < 6; r++)
        for (int j = 0; j < 8; j++) {
            float acc = 0.0f;
            for (int i = 0; i < 8; i++)
                if (Ah[r][i] != 0.0f) acc = fmaf(Ah[r][i], m[i][j], acc);
            t[r][j] = acc;
        }
    for (int r = 0; r < 6; r++)
        for (int s = 0; s < 6; s++) {
            float acc = 0.0f;
            for (int j = 0; j < 8; j++)
                if (Ah[s][j] != 0.0f) acc = fmaf(t[r][j], Ah[s][j], acc);
            y[r][s] = acc;
        }
}

/* Output transform (/root/reference/csrc/nova_winograd.hip:398-450). */
void nvo_output(const uint16_t* M, int B, int K, int Ho, int Wo, int nh, int nw, uint16_t* y) {
    init_tables();
    long P = (long)nh * nw, BP = (long)B * P;
    long total = BP * K;
#pragma omp parallel for schedule(static)
    for (long idx = 0; idx < total; idx++) {
        long bp = idx / K;
        int k = (int)(idx % K);
        int b = (int)(bp / P);
        int tile = (int)(bp % P);
        int th = tile / nw, tw = tile % nw;
        float m[8][8], out[6][6];
        for (int i = 0; i < 8; i++)
            for (int j = 0; j < 8; j++)
                m[i][j] = f16_to_f32(M[(long)(i * 8 + j) * K * BP + bp * K + k]);
        output_tile(m, out);
        for (int r = 0; r < 6; r++)
            for (int s = 0; s < 6; s++) {
                int h = th * 6 + r, w = tw * 6 + s;
                if (h < Ho && w < Wo) y[(((long)b * K + k) * Ho + h) * Wo + w] = f32_to_f16(out[r][s]);
            }
    }
}

/* Whole path with the reference tiling: filter, input, GEMM, output. */
int nvo_conv(const uint16_t* x, const float* w, int B, int C, int K, int H, int W, int pad,
             uint16_t* y) {
    int nh, nw, Ho, Wo;
    nvo_tiling(H, W, pad, &nh, &nw, &Ho, &Wo);
    if (Ho <= 0 || Wo <= 0) return -1;
    long BP = (long)B * nh * nw;
    uint16_t* U = (uint16_t*)malloc(sizeof(uint16_t) * 64 * (size_t)K * C);
    uint16_t* V = (uint16_t*)malloc(sizeof(uint16_t) * 64 * (size_t)C * BP);
    uint16_t* M = (uint16_t*)malloc(sizeof(uint16_t) * 64 * (size_t)K * BP);
    if (!U || !V || !M) { free(U); free(V); free(M); return -2; }
    nvo_filter(w, K, C, U);
    nvo_input(x, B, C, H, W, pad, nh, nw, V);
    nvo_gemm(U, V, K, C, BP, M, NULL);
    nvo_output(M, B, K, Ho, Wo, nh, nw, y);
    free(U);
    free(V);
    free(M);
    return 0;
}

/* Direct correlation in double (/root/reference/csrc/nova_winograd.hip:637-669). */
void nvo_direct(const uint16_t* x, const float* w, int B, int C, int K, int H, int W, int pad,
                double* y) {
    int Ho = H + 2 * pad - 2, Wo = W + 2 * pad - 2;
    long total = (long)B * K * Ho * Wo;
#pragma omp parallel for schedule(static)
    for (long idx = 0; idx < total; idx++) {
        int ow = (int)(idx % Wo);
        int oh = (int)((idx / Wo) % Ho);
        int k = (int)((idx / ((long)Wo * Ho)) % K);
        int b = (int)(idx / ((long)Wo * Ho * K));
        double s = 0.0;
        for (int c = 0; c < C; c++)
            for (int fh = 0; fh < 3; fh++) {
                int ih = oh - pad + fh;
                if (ih < 0 || ih >= H) continue;
                for (int fw = 0; fw < 3; fw++) {
                    int iw = ow - pad + fw;
                    if (iw < 0 || iw >= W) continue;
                    s += (double)f16_to_f32(x[(((long)b * C + c) * H + ih) * W + iw]) *
                         (double)w[(((long)k * C + c) * 3 + fh) * 3 + fw];
                }
            }
        y[idx] = s;
    }
}

/*
 * Weight gradient of the 3x3 correlation (truth for the GPU's Winograd-domain
 * gradient), accumulated in double:
 *   gw[k][c][a][b] = sum_{n,oh,ow} dy[n][k][oh][ow] * x[n][c][oh-pad+a][ow-pad+b]
 * (x outside the image is zero). This is the gradient the reference computes
 * in fp32 with its per-sample unfold loop
 * (/root/reference/nova_winograd/conv2d.py:121-147); dy is fp32 here.
 */
void nvo_weight_grad(const uint16_t* x, const float* dy, int B, int C, int K, int H, int W,
                     int pad, double* gw) {
    int Ho = H + 2 * pad - 2, Wo = W + 2 * pad - 2;
    long total = (long)K * C * 9;
#pragma omp parallel for schedule(static)
    for (long idx = 0; idx < total; idx++) {
        int fb = (int)(idx % 3);
        int fa = (int)((idx / 3) % 3);
        int c = (int)((idx / 9) % C);
        int k = (int)(idx / (9L * C));
        double s = 0.0;
        for (int n = 0; n < B; n++)
            for (int oh = 0; oh < Ho; oh++) {
                int ih = oh - pad + fa;
                if (ih < 0 || ih >= H) continue;
                const float* g = dy + (((long)n * K + k) * Ho + oh) * Wo;
                const uint16_t* xr = x + (((long)n * C + c) * H + ih) * W;
                for (int ow = 0; ow < Wo; ow++) {
                    int iw = ow - pad + fb;
                    if (iw < 0 || iw >= W) continue;
                    s += (double)g[ow] * (double)f16_to_f32(xr[iw]);
                }
            }
        gw[idx] = s;
    }
}
