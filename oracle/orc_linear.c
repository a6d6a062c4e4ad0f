/*
 * orc_linear.c -- restatement of the reference dense layer (linear.rs:44-96).
 * Test infrastructure only (see orc.h).
 */
#include <stdlib.h>

#include "orc.h"

/* Linear::forward (linear.rs:44-63). */
void orc_linear_forward(size_t rows, size_t fin, size_t fout, const float *x, const float *w,
                        const float *b, float *y) {
    orc_matmul(rows, fout, fin, x, 0, w, 1, y, 0);
    if (b)
        for (size_t r = 0; r < rows; r++)
            for (size_t o = 0; o < fout; o++) y[r * fout + o] += b[o];
}

/* Linear::backward (linear.rs:66-96). */
void orc_linear_backward(size_t rows, size_t fin, size_t fout, const float *dy, const float *x,
                         const float *w, float *dw, float *db, float *dx) {
    /* dW[fout, fin] += dY^T[fout, rows] X[rows, fin] */
    orc_matmul_dw(fout, fin, rows, dy, x, dw);
    if (db) {
        /* fold over rows of dy, reduce, then b.g += acc (linear.rs:70-89) */
        size_t lo[256], hi[256];
        size_t nl = orc_fold_leaves(rows, orc_get_threads(), lo, hi, 256);
        float *accs = (float *)calloc(nl * fout + 1, sizeof(float));
        for (size_t l = 0; l < nl; l++)
            for (size_t r = lo[l]; r < hi[l]; r++)
                for (size_t o = 0; o < fout; o++) accs[l * fout + o] += dy[r * fout + o];
        float *red = (float *)calloc(fout, sizeof(float));
        for (size_t l = 0; l < nl; l++)
            for (size_t o = 0; o < fout; o++) red[o] += accs[l * fout + o];
        for (size_t o = 0; o < fout; o++) db[o] += red[o];
        free(red);
        free(accs);
    }
    /* dX[rows, fin] = dY[rows, fout] W[fout, fin] */
    orc_matmul(rows, fin, fout, dy, 0, w, 0, dx, 0);
}
