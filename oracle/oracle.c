/*
 * phobos leaf-kernel ORACLE -- test infrastructure only.
 *
 * A CPU restatement of the arithmetic the reference's leaf kernels and its
 * host-side verifiers perform.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline.  The product path (libphobos_hip + the gfx950
 * code objects) never calls into it.
 *
 * Reference anchors (all paths under the reference tree):
 *   Lcg                 phobos-base/src/rng.rs:1-26 (KAT at rng.rs:50-63)
 *   saxpy               examples/saxpy_fp32.ph:1-5; mul/add not contracted,
 *                       phobos-lang/src/codegen/tile.rs:1786-1794;
 *                       verifier phobos-bench/src/main.rs:1176-1188
 *   gemm epilogue       phobos-lang/src/codegen/matmul.rs:384-403
 *                       fl(fl(alpha*acc) + fl(beta*c))
 *   gemm check          phobos-bench/src/main.rs:386-445 (f64 dot, xorshift64
 *                       sampler seeded 0x243F6A8885A308D3, (0,0), (M-1,N-1))
 *   f16 rounding        main.rs:447-449 (half 2.7.1 from_f32 = IEEE RNE)
 *   fp16-acc model      main.rs:638-679 (informational)
 *   flash replay        main.rs:869-920 (f64 online softmax)
 *   cluster chain       phobos-cluster/src/clustergen.rs:1292-1399
 *                       init: C = fl(beta*C); step: C = fl(fl(alpha*acc)+C)
 *
 * Parity pins (tests/test_oracle.py): Lcg KAT recomputed with Python
 * integers; f16 RNE against numpy.float16 incl. ties/subnormals/overflow;
 * saxpy against numpy float32 mul-then-add; GEMM against numpy float64
 * matmul and the exact-integer fixture (masking.rs:108-110 style inputs);
 * flash against the closed-form softmax(QK^T*s)V in float64 plus the
 * one-key / permutation / convexity invariants; the cluster chain against a
 * direct f64 evaluation.  The Box-Muller normal generator is this build's own
 * input convention (the reference has none) and is pinned only statistically.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- Lcg */
/* rng.rs:9-20: s = s*6364136223846793005 + 1442695040888963407 (mod 2^64);
 * unit = (s >> 33) as f32 / 2^31 - 1.0  (both steps rounded in f32). */
static inline uint64_t lcg_step(uint64_t *s) {
    *s = *s * 6364136223846793005ULL + 1442695040888963407ULL;
    return *s;
}

void orc_lcg_fill_f32(uint64_t seed, size_t n, float *out) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) {
        uint64_t v = lcg_step(&s) >> 33;           /* < 2^31, exact in f32? no: rounded */
        float f = (float)v;                        /* `as f32` rounds to nearest even */
        out[i] = f / 2147483648.0f - 1.0f;
    }
}

void orc_lcg_u64(uint64_t seed, size_t n, uint64_t *out) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) out[i] = lcg_step(&s);
}

/* Seeded N(0,1) by Box-Muller on Lcg draws (this build's convention; the
 * reference has no normal generator).  Pair i uses two successive Lcg
 * states a, b: u1 = ((a>>11)+1)*2^-53 in (0,1], u2 = (b>>11)*2^-53 in [0,1);
 * z0 = r*cos(2*pi*u2), z1 = r*sin(2*pi*u2), r = sqrt(-2 ln u1); all in f64,
 * multiplied by `scale`, then cast to f32. */
void orc_normal_fill_f32(uint64_t seed, size_t n, double scale, float *out) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        uint64_t a = lcg_step(&s), b = lcg_step(&s);
        double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;
        double u2 = (double)(b >> 11) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(two_pi * u2) * scale);
        if (i + 1 < n) out[i + 1] = (float)(r * sin(two_pi * u2) * scale);
    }
}

/* ---------------------------------------------------------------- f16 */
/* IEEE binary32 -> binary16, round to nearest even (half 2.7.1 from_f32). */
uint16_t orc_f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {                         /* inf / nan */
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);   /* overflow -> inf */
    if (e <= 0) {                                     /* subnormal / zero */
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;                 /* 24-bit significand */
        uint32_t shift = (uint32_t)(14 - e);          /* 14..24 */
        uint32_t half_m = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m += 1;
        return (uint16_t)(sign | half_m);            /* may carry into exp=1: correct */
    }
    uint32_t half_m = man >> 13;
    uint32_t rem = man & 0x1fffu;
    uint32_t out = sign | ((uint32_t)e << 10) | half_m;
    if (rem > 0x1000u || (rem == 0x1000u && (half_m & 1u))) out += 1;  /* carry ok */
    return (uint16_t)out;
}

float orc_f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else {                                  /* subnormal: man * 2^-24 */
            float f = (float)man * 0x1.0p-24f;
            memcpy(&x, &f, 4);
            x |= sign;
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

float orc_f16_round(float f) { return orc_f16_bits_to_f32(orc_f32_to_f16_bits(f)); }

void orc_f16_round_array(size_t n, const float *in, float *out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f16_round(in[i]);
}
void orc_f32_to_f16_array(size_t n, const float *in, uint16_t *out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16_bits(in[i]);
}
void orc_f16_to_f32_array(size_t n, const uint16_t *in, float *out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f16_bits_to_f32(in[i]);
}

/* -------------------------------------------------------------- saxpy */
/* out[i] = fl(fl(alpha*x[i]) + y[i]); volatile temporaries keep gcc from
 * contracting (the file is also built with -ffp-contract=off). */
void orc_saxpy(size_t n, float alpha, const float *x, const float *y, float *out) {
    for (size_t i = 0; i < n; ++i) {
        volatile float p = alpha * x[i];
        out[i] = p + y[i];
    }
}

/* The same, split over the host cores (OpenMP): the timed CPU baseline of
 * the saxpy config. */
void orc_saxpy_mt(size_t n, float alpha, const float *x, const float *y, float *out) {
#pragma omp parallel for schedule(static)
    for (long i = 0; i < (long)n; ++i) {
        volatile float p = alpha * x[i];
        out[i] = p + y[i];
    }
}

/* --------------------------------------------------------------- gemm */
/* xorshift64 point sampler of main.rs:399-410: (0,0), (M-1,N-1), then
 * (sample(M), sample(N)) with sample(l) = state % l after each step. */
void orc_sample_points(size_t M, size_t N, size_t count, uint64_t *rows, uint64_t *cols) {
    uint64_t st = 0x243F6A8885A308D3ULL;
    for (size_t s = 0; s < count; ++s) {
        if (s == 0) { rows[s] = 0; cols[s] = 0; continue; }
        if (s == 1) { rows[s] = M - 1; cols[s] = N - 1; continue; }
        st ^= st << 13; st ^= st >> 7; st ^= st << 17;
        rows[s] = st % M;
        st ^= st << 13; st ^= st >> 7; st ^= st << 17;
        cols[s] = st % N;
    }
}

/* want(i,j) = alpha * sum_k A[i,k]*B[k,j] + beta * Cin[i,j], all in f64
 * (main.rs:411-436).  round16 rounds A and B to f16 first (main.rs:417-427).
 * Row strides lda/ldb/ldc are in elements. */
double orc_gemm_point_f64(size_t i, size_t j, size_t K, const float *A, size_t lda,
                          const float *B, size_t ldb, const float *Cin, size_t ldc,
                          double alpha, double beta, int round16) {
    double dot = 0.0;
    for (size_t k = 0; k < K; ++k) {
        double a = round16 ? orc_f16_round(A[i * lda + k]) : A[i * lda + k];
        double b = round16 ? orc_f16_round(B[k * ldb + j]) : B[k * ldb + j];
        dot += a * b;
    }
    double c = Cin ? (double)Cin[i * ldc + j] : 0.0;
    return alpha * dot + beta * c;
}

void orc_gemm_points_f64(size_t npts, const uint64_t *rows, const uint64_t *cols, size_t K,
                         const float *A, size_t lda, const float *B, size_t ldb,
                         const float *Cin, size_t ldc, double alpha, double beta, int round16,
                         double *out) {
#pragma omp parallel for schedule(dynamic, 1)
    for (long p = 0; p < (long)npts; ++p)
        out[p] = orc_gemm_point_f64(rows[p], cols[p], K, A, lda, B, ldb, Cin, ldc, alpha, beta,
                                    round16);
}

/* Full f64 product, for shapes the CPU finishes in seconds. */
void orc_gemm_full_f64(size_t M, size_t N, size_t K, const float *A, const float *B,
                       const float *Cin, double alpha, double beta, int round16, double *out) {
#pragma omp parallel for schedule(static)
    for (long i = 0; i < (long)M; ++i) {
        double *row = out + (size_t)i * N;
        for (size_t j = 0; j < N; ++j) row[j] = 0.0;
        for (size_t k = 0; k < K; ++k) {
            double a = round16 ? orc_f16_round(A[(size_t)i * K + k]) : A[(size_t)i * K + k];
            const float *b = B + k * N;
            if (round16) {
                for (size_t j = 0; j < N; ++j) row[j] += a * (double)orc_f16_round(b[j]);
            } else {
                for (size_t j = 0; j < N; ++j) row[j] += a * (double)b[j];
            }
        }
        for (size_t j = 0; j < N; ++j)
            row[j] = alpha * row[j] + beta * (Cin ? (double)Cin[(size_t)i * N + j] : 0.0);
    }
}

/* The reference's sequential fp16-accumulate model (main.rs:659-672):
 * acc = f16(acc + f16(a)*f16(b)) per k (product and sum in f32), then
 * f16(alpha*acc + beta*c).  Informational: MFMA accumulates in f32. */
float orc_gemm_fp16acc_point(size_t i, size_t j, size_t K, const float *A, const float *B,
                             size_t N, const float *Cin, float alpha, float beta) {
    float acc = 0.0f;
    for (size_t k = 0; k < K; ++k) {
        float af = orc_f16_round(A[i * K + k]);
        float bf = orc_f16_round(B[k * N + j]);
        volatile float p = af * bf;
        acc = orc_f16_round(acc + p);
    }
    volatile float t0 = alpha * acc;
    volatile float t1 = beta * (Cin ? Cin[i * N + j] : 0.0f);
    return orc_f16_round(t0 + t1);
}

/* -------------------------------------------------------------- flash */
/* main.rs:894-911: f64 online softmax over all keys for one (row, d).
 * Here the whole output row is produced at once (same recurrence, all d). */
void orc_flash_row_f64(size_t i, size_t Nk, size_t D, const float *q, const float *k,
                       const float *v, double scale, double *orow) {
    double m = -INFINITY, l = 0.0;
    for (size_t d = 0; d < D; ++d) orow[d] = 0.0;
    for (size_t j = 0; j < Nk; ++j) {
        double s = 0.0;
        for (size_t e = 0; e < D; ++e) s += (double)q[i * D + e] * (double)k[j * D + e];
        s *= scale;
        double mnew = m > s ? m : s;
        double corr = exp(m - mnew);
        double p = exp(s - mnew);
        l = l * corr + p;
        for (size_t d = 0; d < D; ++d) orow[d] = orow[d] * corr + p * (double)v[j * D + d];
        m = mnew;
    }
    for (size_t d = 0; d < D; ++d) orow[d] /= l;
}

/* rows[] subset of one head; out is [nrows, D]. */
void orc_flash_rows_f64(size_t nrows, const uint64_t *rows, size_t Nk, size_t D, const float *q,
                        const float *k, const float *v, double scale, double *out) {
#pragma omp parallel for schedule(dynamic, 1)
    for (long r = 0; r < (long)nrows; ++r)
        orc_flash_row_f64(rows[r], Nk, D, q, k, v, scale, out + (size_t)r * D);
}

/* All rows of `heads` independent heads laid out [heads, N, D]. */
void orc_flash_heads_f64(size_t heads, size_t Nq, size_t Nk, size_t D, const float *q,
                         const float *k, const float *v, double scale, double *out) {
#pragma omp parallel for schedule(dynamic, 4)
    for (long t = 0; t < (long)(heads * Nq); ++t) {
        size_t h = (size_t)t / Nq, i = (size_t)t % Nq;
        orc_flash_row_f64(i, Nk, D, q + h * Nq * D, k + h * Nk * D, v + h * Nk * D, scale,
                          out + ((size_t)h * Nq + i) * D);
    }
}

/* -------------------------------------------------------- cluster chain */
/* matmul_init (clustergen.rs:1292-1360): C = fl(beta * C). */
void orc_matmul_init(size_t n, float beta, float *c) {
    for (size_t i = 0; i < n; ++i) {
        volatile float t = beta * c[i];
        c[i] = t;
    }
}

/* matmul step leaf (clustergen.rs:1369-1399): C = fl(fl(alpha*acc) + C)
 * where acc is supplied (the f32 dot over one K supertile). */
void orc_matmul_step_epilogue(size_t n, float alpha, const float *acc, float *c) {
    for (size_t i = 0; i < n; ++i) {
        volatile float t = alpha * acc[i];
        c[i] = t + c[i];
    }
}

/* ------------------------------------------------------- CPU baselines */
/* Blocked f32 GEMM, C = fl(fl(alpha*acc) + fl(beta*C)), OpenMP over row
 * blocks.  This is the timed CPU baseline, not a parity reference. */
void orc_sgemm_f32(size_t M, size_t N, size_t K, float alpha, const float *A, const float *B,
                   float beta, float *C) {
    const size_t BM = 64, BN = 256, BK = 256;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
    for (long ib = 0; ib < (long)((M + BM - 1) / BM); ++ib) {
        for (long jb = 0; jb < (long)((N + BN - 1) / BN); ++jb) {
            size_t i0 = (size_t)ib * BM, j0 = (size_t)jb * BN;
            size_t i1 = i0 + BM < M ? i0 + BM : M, j1 = j0 + BN < N ? j0 + BN : N;
            float acc[64][256];
            for (size_t i = i0; i < i1; ++i)
                for (size_t j = j0; j < j1; ++j) acc[i - i0][j - j0] = 0.0f;
            for (size_t k0 = 0; k0 < K; k0 += BK) {
                size_t k1 = k0 + BK < K ? k0 + BK : K;
                for (size_t i = i0; i < i1; ++i) {
                    float *arow = acc[i - i0];
                    for (size_t k = k0; k < k1; ++k) {
                        float a = A[i * K + k];
                        const float *b = B + k * N;
                        for (size_t j = j0; j < j1; ++j) arow[j - j0] += a * b[j];
                    }
                }
            }
            for (size_t i = i0; i < i1; ++i)
                for (size_t j = j0; j < j1; ++j) {
                    float t0 = alpha * acc[i - i0][j - j0];
                    float t1 = beta * C[i * N + j];
                    C[i * N + j] = t0 + t1;
                }
        }
    }
}

/* f32 flash attention over [heads, N, D] (two-pass softmax per row), the
 * timed CPU baseline for the flash kernels. */
void orc_flash_f32(size_t heads, size_t Nq, size_t Nk, size_t D, const float *q, const float *k,
                   const float *v, float scale, float *o) {
#pragma omp parallel
    {
        float *s = (float *)malloc(Nk * sizeof(float));
#pragma omp for schedule(dynamic, 8)
        for (long t = 0; t < (long)(heads * Nq); ++t) {
            size_t h = (size_t)t / Nq, i = (size_t)t % Nq;
            const float *qi = q + (h * Nq + i) * D;
            const float *kh = k + h * Nk * D, *vh = v + h * Nk * D;
            float m = -INFINITY;
            for (size_t j = 0; j < Nk; ++j) {
                float acc = 0.0f;
                for (size_t e = 0; e < D; ++e) acc += qi[e] * kh[j * D + e];
                s[j] = acc * scale;
                if (s[j] > m) m = s[j];
            }
            float l = 0.0f;
            float *oi = o + (h * Nq + i) * D;
            for (size_t e = 0; e < D; ++e) oi[e] = 0.0f;
            for (size_t j = 0; j < Nk; ++j) {
                float p = expf(s[j] - m);
                l += p;
                for (size_t e = 0; e < D; ++e) oi[e] += p * vh[j * D + e];
            }
            for (size_t e = 0; e < D; ++e) oi[e] /= l;
        }
        free(s);
    }
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
