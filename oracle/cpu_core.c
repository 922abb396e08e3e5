/*
 * CPU baseline kernels: this build's own C restatement of the reference's AVX2 C core
 * (native/c/rotor_core.c), built single-threaded with -O3 -mavx2 like the reference's
 * native/build.py builds its core.
 *
 * TEST INFRASTRUCTURE ONLY: the cpu_baseline leg of bench.py times these on the GPU box's
 * host, and tests/test_oracle.py checks them against the NumPy oracle and the reference's
 * own core (oracle/_ref).  The product library never loads this file.
 */
#include <stddef.h>
#include <stdint.h>

/* Bit planes (8 weights per byte, LSB first, rows of ceil(cols/8) bytes) -> int8 weights
 * [rows][cols], w = bit0 - bit1.  The load path of the reference's int8 weights_cache:
 * rotor_unpack_weights, native/c/rotor_core.c:270-299. */
void cb_unpack_planes(const uint8_t* bit0, const uint8_t* bit1, size_t rows, size_t cols, int8_t* w) {
    const size_t rb = (cols + 7) / 8;
    for (size_t r = 0; r < rows; r++) {
        const uint8_t* p0 = bit0 + r * rb;
        const uint8_t* p1 = bit1 + r * rb;
        int8_t* dst = w + r * cols;
        const size_t full = cols / 8;
        for (size_t b = 0; b < full; b++) {
            const unsigned b0 = p0[b], b1 = p1[b];
            for (int j = 0; j < 8; j++) dst[8 * b + j] = (int8_t)((int)((b0 >> j) & 1u) - (int)((b1 >> j) & 1u));
        }
        for (size_t k = full * 8; k < cols; k++) {  /* ragged last byte */
            const size_t b = k / 8;
            const int j = (int)(k % 8);
            dst[k] = (int8_t)((int)((p0[b] >> j) & 1u) - (int)((p1[b] >> j) & 1u));
        }
    }
}

/* The reference's sign-activation ternary mat-vec: x is quantised to {-1, 0, +1} by its
 * sign (threshold 0: rotor_quantize_ternary, native/c/rotor_core.c:186-196), encoded as
 * two byte planes (one element per byte: rotor_encode, :25-30), and each output is the
 * plane product pp - pn - np + nn of rotor_dot (:102-162) against the weight planes
 * W_bit0 / W_bit1 [m][n] (one element per byte): rotor_matvec, :305-331.  Different
 * numerics from the W2A8 path (1-bit activations): reported, never compared with it.
 * xq0 / xq1: caller scratch of n bytes each.  Sums are kept in int32 (the reference's
 * 8-bit lane accumulators agree while n <= 8160). */
void cb_sign_matvec(const uint8_t* wb0, const uint8_t* wb1, const float* x, size_t m, size_t n, uint8_t* xq0,
                    uint8_t* xq1, int32_t* y) {
    for (size_t k = 0; k < n; k++) {
        xq0[k] = x[k] > 0.0f ? 1 : 0;
        xq1[k] = x[k] < -0.0f ? 1 : 0;
    }
    for (size_t i = 0; i < m; i++) {
        const uint8_t* a0 = wb0 + i * n;
        const uint8_t* a1 = wb1 + i * n;
        int32_t pp = 0, pn = 0, np_ = 0, nn = 0;
        for (size_t k = 0; k < n; k++) {
            pp += a0[k] & xq0[k];
            pn += a0[k] & xq1[k];
            np_ += a1[k] & xq0[k];
            nn += a1[k] & xq1[k];
        }
        y[i] = pp - pn - np_ + nn;
    }
}
