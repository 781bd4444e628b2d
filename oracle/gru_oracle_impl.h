/*
 * CPU restatement of the reference's fp32 GRU training path (one layer).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load the
 * library built from it.  The product path (rnn_kernel_amd) never calls it.
 *
 * It is compiled twice by gru_oracle.c, once with REAL=double and once with
 * REAL=float, giving the *_f64 and *_f32 entry points.  Every sum is taken
 * left to right in increasing index order (there is no blocking, splitting or
 * threading of a sum), so the fp32 variant's summation order is the naive one
 * and the fp64 variant bounds its rounding error.  The loops over a sum's
 * index are arranged so that inner loops run over contiguous memory (a
 * transposed copy of the weights in the forward, arrays of running sums in
 * the backward); that reorders independent sums against one another, never
 * the terms of one sum.
 *
 * Equations follow the reference:
 *   input projection  Gx = x W_ih^T + b_ih
 *       src/rnn_kernel/a100/prod/gru.py:519-523
 *   recurrence (gate order r, z, n in rows [0,H), [H,2H), [2H,3H))
 *       a   = W_hh h_{t-1} + b_hh
 *       r   = sigmoid(Gx_r + a_r), z = sigmoid(Gx_z + a_z)
 *       n   = tanh(Gx_n + r * a_n)
 *       h_t = n + z * (h_{t-1} - n)
 *       src/rnn_kernel/a100/prod/kernels/a100_gru_h256_kernels.cu:756-771
 *       src/rnn_kernel/custom_gru.py:112-117
 *   gate cache (r, z, n, a_n) per step
 *       src/rnn_kernel/a100/prod/kernels/a100_gru_h256_kernels.cu:772-775
 *   h_n = output[:, T-1]
 *       src/rnn_kernel/a100/prod/gru.py:525
 *   backward (g = dh_t + dy_t), reverse time
 *       dz = g (h_{t-1} - n), dn = g (1 - z), dn^ = dn (1 - n^2)
 *       dr = dn^ a_n, da_n = dn^ r, dr^ = dr r (1 - r), dz^ = dz z (1 - z)
 *       G_i = (dr^, dz^, dn^), G_h = (dr^, dz^, da_n)
 *       dh_{t-1} = g z + G_h W_hh
 *       src/rnn_kernel/a100/prod/kernels/a100_gru_h256_kernels.cu:842-866,915-932
 *       src/rnn_kernel/triton_gru_pointwise.py:78-94
 *   weight / input gradients
 *       dW_hh = sum_t G_h^T h_{t-1}, db_hh = sum G_h,
 *       dx = G_i W_ih, dW_ih = sum_t G_i^T x_t, db_ih = sum G_i
 *       src/rnn_kernel/a100/prod/gru.py:569-578
 *
 * Layouts: x [B,T,I], y [B,T,H], h0/hn [B,H], W_ih [3H,I], W_hh [3H,H],
 * biases [3H], cache [B,T,4H] holding (r, z, n, a_n) blocks of H.
 */

#ifndef REAL
#error "define REAL before including gru_oracle_impl.h"
#endif
#ifndef SUF
#error "define SUF before including gru_oracle_impl.h"
#endif

#define ORC_CAT2(a, b) a##b
#define ORC_CAT(a, b) ORC_CAT2(a, b)
#define ORC_FN(name) ORC_CAT(name, SUF)

static REAL ORC_FN(orc_sigmoid)(REAL v) { return (REAL)1 / ((REAL)1 + EXPF(-v)); }

/* One layer forward.  cache may be NULL (inference).  Returns 0. */
int ORC_FN(oracle_gru_forward)(int B, int T, int I, int H,
                               const REAL* x, const REAL* h0,
                               const REAL* w_ih, const REAL* w_hh,
                               const REAL* b_ih, const REAL* b_hh,
                               REAL* y, REAL* hn, REAL* cache)
{
    const int G3 = 3 * H;
    REAL* gx = (REAL*)malloc(sizeof(REAL) * (size_t)G3);
    REAL* ah = (REAL*)malloc(sizeof(REAL) * (size_t)G3);
    REAL* hprev = (REAL*)malloc(sizeof(REAL) * (size_t)H);
    /* W_ih^T [I][3H] and W_hh^T [H][3H]: row k holds the k-th term's weights
     * of every gate row j, so the running sums of all j advance together */
    REAL* wiT = (REAL*)malloc(sizeof(REAL) * (size_t)I * G3);
    REAL* whT = (REAL*)malloc(sizeof(REAL) * (size_t)H * G3);
    if (!gx || !ah || !hprev || !wiT || !whT) {
        free(gx); free(ah); free(hprev); free(wiT); free(whT);
        return 1;
    }
    for (int j = 0; j < G3; ++j) {
        for (int k = 0; k < I; ++k) wiT[(size_t)k * G3 + j] = w_ih[(size_t)j * I + k];
        for (int k = 0; k < H; ++k) whT[(size_t)k * G3 + j] = w_hh[(size_t)j * H + k];
    }
    for (int b = 0; b < B; ++b) {
        for (int k = 0; k < H; ++k) hprev[k] = h0[(size_t)b * H + k];
        for (int t = 0; t < T; ++t) {
            const REAL* xt = x + ((size_t)b * T + t) * I;
            /* gx[j] = (sum_k W_ih[j][k] x_t[k], k = 0, 1, ...) + b_ih[j] */
            for (int j = 0; j < G3; ++j) gx[j] = 0;
            for (int k = 0; k < I; ++k) {
                const REAL* w = wiT + (size_t)k * G3;
                const REAL xk = xt[k];
                for (int j = 0; j < G3; ++j) gx[j] += w[j] * xk;
            }
            for (int j = 0; j < G3; ++j) gx[j] += b_ih[j];
            /* ah[j] = (sum_k W_hh[j][k] h_{t-1}[k]) + b_hh[j] */
            for (int j = 0; j < G3; ++j) ah[j] = 0;
            for (int k = 0; k < H; ++k) {
                const REAL* w = whT + (size_t)k * G3;
                const REAL hk = hprev[k];
                for (int j = 0; j < G3; ++j) ah[j] += w[j] * hk;
            }
            for (int j = 0; j < G3; ++j) ah[j] += b_hh[j];
            REAL* yt = y + ((size_t)b * T + t) * H;
            REAL* ct = cache ? cache + ((size_t)b * T + t) * 4 * H : NULL;
            for (int u = 0; u < H; ++u) {
                const REAL r = ORC_FN(orc_sigmoid)(gx[u] + ah[u]);
                const REAL z = ORC_FN(orc_sigmoid)(gx[H + u] + ah[H + u]);
                const REAL n = TANHF(gx[2 * H + u] + r * ah[2 * H + u]);
                yt[u] = n + z * (hprev[u] - n);
                if (ct) {
                    ct[u] = r;
                    ct[H + u] = z;
                    ct[2 * H + u] = n;
                    ct[3 * H + u] = ah[2 * H + u];
                }
            }
            for (int u = 0; u < H; ++u) hprev[u] = yt[u];
        }
        if (hn) {
            for (int u = 0; u < H; ++u) hn[(size_t)b * H + u] = hprev[u];
        }
    }
    free(gx); free(ah); free(hprev); free(wiT); free(whT);
    return 0;
}

/*
 * One layer backward.  dy may be NULL (treated as zeros, gru.py:534-535);
 * dhn may be NULL (no gradient on h_n, gru.py:552-554).  dx may be NULL
 * (input gradient not needed).  Gradients are written, not accumulated.
 */
int ORC_FN(oracle_gru_backward)(int B, int T, int I, int H,
                                const REAL* x, const REAL* h0,
                                const REAL* w_ih, const REAL* w_hh,
                                const REAL* y, const REAL* cache,
                                const REAL* dy, const REAL* dhn,
                                REAL* dx, REAL* dh0,
                                REAL* dw_ih, REAL* dw_hh,
                                REAL* db_ih, REAL* db_hh)
{
    const int G3 = 3 * H;
    REAL* dh = (REAL*)malloc(sizeof(REAL) * (size_t)H);
    REAL* gi = (REAL*)malloc(sizeof(REAL) * (size_t)G3);
    REAL* gh = (REAL*)malloc(sizeof(REAL) * (size_t)G3);
    REAL* dhp = (REAL*)malloc(sizeof(REAL) * (size_t)H);
    REAL* sh = (REAL*)malloc(sizeof(REAL) * (size_t)H);  /* running sums of G_h W_hh */
    REAL* sx = (REAL*)malloc(sizeof(REAL) * (size_t)I);  /* running sums of G_i W_ih */
    if (!dh || !gi || !gh || !dhp || !sh || !sx) {
        free(dh); free(gi); free(gh); free(dhp); free(sh); free(sx);
        return 1;
    }
    memset(dw_ih, 0, sizeof(REAL) * (size_t)G3 * I);
    memset(dw_hh, 0, sizeof(REAL) * (size_t)G3 * H);
    memset(db_ih, 0, sizeof(REAL) * (size_t)G3);
    memset(db_hh, 0, sizeof(REAL) * (size_t)G3);

    for (int b = 0; b < B; ++b) {
        for (int u = 0; u < H; ++u) dh[u] = dhn ? dhn[(size_t)b * H + u] : (REAL)0;
        for (int t = T - 1; t >= 0; --t) {
            const REAL* ct = cache + ((size_t)b * T + t) * 4 * H;
            const REAL* hp = (t == 0) ? h0 + (size_t)b * H : y + ((size_t)b * T + t - 1) * H;
            const REAL* dyt = dy ? dy + ((size_t)b * T + t) * H : NULL;
            for (int u = 0; u < H; ++u) {
                const REAL r = ct[u], z = ct[H + u], n = ct[2 * H + u], an = ct[3 * H + u];
                const REAL g = dh[u] + (dyt ? dyt[u] : (REAL)0);
                const REAL dz = g * (hp[u] - n);
                const REAL dn = g * ((REAL)1 - z);
                const REAL dnh = dn * ((REAL)1 - n * n);
                const REAL dr = dnh * an;
                const REAL dan = dnh * r;
                const REAL drh = dr * r * ((REAL)1 - r);
                const REAL dzh = dz * z * ((REAL)1 - z);
                gi[u] = drh;     gi[H + u] = dzh;     gi[2 * H + u] = dnh;
                gh[u] = drh;     gh[H + u] = dzh;     gh[2 * H + u] = dan;
                dhp[u] = g * z;
            }
            /* dh_{t-1}[k] = g z + (sum_j G_h[j] W_hh[j][k], j = 0, 1, ...) */
            for (int k = 0; k < H; ++k) sh[k] = 0;
            for (int j = 0; j < G3; ++j) {
                const REAL* w = w_hh + (size_t)j * H;
                const REAL gj = gh[j];
                for (int k = 0; k < H; ++k) sh[k] += gj * w[k];
            }
            for (int k = 0; k < H; ++k) dh[k] = dhp[k] + sh[k];
            /* parameter gradients */
            const REAL* xt = x + ((size_t)b * T + t) * I;
            for (int j = 0; j < G3; ++j) {
                REAL* wi = dw_ih + (size_t)j * I;
                REAL* wh = dw_hh + (size_t)j * H;
                for (int k = 0; k < I; ++k) wi[k] += gi[j] * xt[k];
                for (int k = 0; k < H; ++k) wh[k] += gh[j] * hp[k];
                db_ih[j] += gi[j];
                db_hh[j] += gh[j];
            }
            if (dx) {
                /* dx_t[k] = sum_j G_i[j] W_ih[j][k], j = 0, 1, ... */
                REAL* dxt = dx + ((size_t)b * T + t) * I;
                for (int k = 0; k < I; ++k) sx[k] = 0;
                for (int j = 0; j < G3; ++j) {
                    const REAL* w = w_ih + (size_t)j * I;
                    const REAL gj = gi[j];
                    for (int k = 0; k < I; ++k) sx[k] += gj * w[k];
                }
                for (int k = 0; k < I; ++k) dxt[k] = sx[k];
            }
        }
        for (int u = 0; u < H; ++u) dh0[(size_t)b * H + u] = dh[u];
    }
    free(dh); free(gi); free(gh); free(dhp); free(sh); free(sx);
    return 0;
}

#undef ORC_FN
#undef ORC_CAT
#undef ORC_CAT2
