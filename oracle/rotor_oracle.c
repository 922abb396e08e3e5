/*
 * CPU oracle for the rotor ternary-linear path, plain C restatement.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker; never by the product library.
 *
 * Each function restates a reference function (paths are relative to the
 * reference repository BikerSam86/rotor-RAG).  It is a second, independent
 * statement of what oracle/rotor_oracle.py computes; tests check the two
 * against each other and against the reference's own C core (oracle/_ref).
 *
 * Build: see oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off, no fast-math,
 * so fp32 division and rintf are IEEE round-to-nearest-even).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

/* Field f = (byte >> 2j) & 3 of element j; value = bit0 - bit1 = (f >> 1) - (f & 1).
 * 00 -> 0, 10 -> +1, 01 -> -1, 11 -> 0 (reserved/error).
 * src/rotor/core.py:99-108 (layout), native/c/rotor_core.c:240-256 (decode rule). */
static inline int8_t field_value(unsigned f) { return (int8_t)((int)(f >> 1) - (int)(f & 1u)); }

/* W int8 [N][K] in {-1,0,1} -> rotor bytes [N][ceil(K/4)]; rows packed on their own,
 * missing elements of the last byte are zero codes.  src/rotor/core.py:75-110. */
void orc_pack_rotor(const int8_t* W, size_t N, size_t K, uint8_t* out) {
    size_t kb = (K + 3) / 4;
    for (size_t n = 0; n < N; n++) {
        for (size_t b = 0; b < kb; b++) {
            unsigned byte = 0;
            for (unsigned j = 0; j < 4; j++) {
                size_t k = b * 4 + j;
                int8_t v = k < K ? W[n * K + k] : 0;
                unsigned bit0 = v == 1, bit1 = v == -1;
                byte |= (bit0 << (2 * j + 1)) | (bit1 << (2 * j));
            }
            out[n * kb + b] = (uint8_t)byte;
        }
    }
}

/* rotor bytes [N][ceil(K/4)] -> int8 [N][K].  src/rotor/core.py:113-141 + :56-72. */
void orc_unpack_rotor(const uint8_t* p, size_t N, size_t K, int8_t* W) {
    size_t kb = (K + 3) / 4;
    for (size_t n = 0; n < N; n++)
        for (size_t k = 0; k < K; k++)
            W[n * K + k] = field_value((p[n * kb + k / 4] >> (2 * (k % 4))) & 3u);
}

/* 4/byte codes -> LSB-first planes [rows][ceil(cols/8)].  native/c/rotor_core.c:202-260. */
void orc_bitnet_to_rotor(const uint8_t* src, size_t rows, size_t cols, uint8_t* bit0, uint8_t* bit1) {
    size_t cb = (cols + 3) / 4, ob = (cols + 7) / 8;
    memset(bit0, 0, rows * ob);
    memset(bit1, 0, rows * ob);
    for (size_t r = 0; r < rows; r++)
        for (size_t k = 0; k < cols; k++) {
            unsigned f = (src[r * cb + k / 4] >> (2 * (k % 4))) & 3u;
            if (f == 2u) bit0[r * ob + k / 8] |= (uint8_t)(1u << (k % 8));
            if (f == 1u) bit1[r * ob + k / 8] |= (uint8_t)(1u << (k % 8));
        }
}

/* planes -> int8 w = bit0 - bit1.  native/c/rotor_core.c:270-299. */
void orc_unpack_planes(const uint8_t* bit0, const uint8_t* bit1, size_t rows, size_t cols, int8_t* W) {
    size_t ob = (cols + 7) / 8;
    for (size_t r = 0; r < rows; r++)
        for (size_t k = 0; k < cols; k++) {
            int v0 = (bit0[r * ob + k / 8] >> (k % 8)) & 1, v1 = (bit1[r * ob + k / 8] >> (k % 8)) & 1;
            W[r * cols + k] = (int8_t)(v0 - v1);
        }
}

/* Per-row absmax int8: s = max|x|/127 (1 if 0), q = clip(rint(x/s), -128, 127), all fp32.
 * src/rotor/quantization.py:137-149 applied per row. */
void orc_quant_rows(const float* x, size_t M, size_t K, int8_t* q, float* s) {
    for (size_t m = 0; m < M; m++) {
        const float* xr = x + m * K;
        float amax = 0.0f;
        for (size_t k = 0; k < K; k++) {
            float a = fabsf(xr[k]);
            if (a > amax) amax = a;
        }
        float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
        s[m] = sc;
        for (size_t k = 0; k < K; k++) {
            float r = rintf(xr[k] / sc);
            if (r < -128.0f) r = -128.0f;
            if (r > 127.0f) r = 127.0f;
            q[m * K + k] = (int8_t)r;
        }
    }
}

/* acc[m][n] = sum_k q[m][k] * W[n][k], exact in int64. */
void orc_linear_i64(const int8_t* q, const int8_t* W, size_t M, size_t N, size_t K, int64_t* acc) {
#pragma omp parallel for schedule(static)
    for (long long n = 0; n < (long long)N; n++) {
        const int8_t* w = W + (size_t)n * K;
        for (size_t m = 0; m < M; m++) {
            const int8_t* qr = q + m * K;
            int64_t a = 0;
            for (size_t k = 0; k < K; k++) a += (int64_t)qr[k] * (int64_t)w[k];
            acc[m * N + (size_t)n] = a;
        }
    }
}

/* Same accumulators straight from the packed rotor bytes (decode on the fly): the
 * CPU statement of what the GPU kernels compute before the fp32 epilogue. */
void orc_linear_i64_packed(const int8_t* q, const uint8_t* Wp, size_t M, size_t N, size_t K, int64_t* acc) {
    size_t kb = (K + 3) / 4;
#pragma omp parallel for schedule(static)
    for (long long n = 0; n < (long long)N; n++) {
        const uint8_t* w = Wp + (size_t)n * kb;
        for (size_t m = 0; m < M; m++) {
            const int8_t* qr = q + m * K;
            int64_t a = 0;
            for (size_t k = 0; k < K; k++) a += (int64_t)qr[k] * field_value((w[k / 4] >> (2 * (k % 4))) & 3u);
            acc[m * N + (size_t)n] = a;
        }
    }
}
