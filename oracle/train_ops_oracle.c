/*
 * CPU restatement of the training-step operations on either side of the GRU
 * in the reference's benchmark harness, in float64.
 *
 * TEST INFRASTRUCTURE ONLY: only tests/ load it (through gru_oracle.py); the
 * product path never calls it.
 *
 * The reference uses PyTorch for these (torch==2.6.0, requirements.txt:3):
 *   head   self.head = nn.Linear(hidden_size, 1); pred = head(out).squeeze(-1)
 *          rnn_benchmark.py:510,525
 *   loss   F.mse_loss(pred, y) (reduction 'mean')      rnn_benchmark.py:636
 *   update torch.optim.AdamW(..., weight_decay=1e-4)   rnn_benchmark.py:722
 * and the formulas below are the published definitions of those operations
 * (AdamW: decoupled weight decay p *= 1 - lr*wd, then Adam with bias
 * correction, in torch's order of operations).
 */
#include <math.h>
#include <stddef.h>

/* pred[r] = sum_h out[r,h] w[h] + b */
void oracle_head_forward_f64(int rows, int hidden, const double* out, const double* w, double b, double* pred) {
    for (int r = 0; r < rows; ++r) {
        double s = 0.0;
        for (int h = 0; h < hidden; ++h) s += out[(size_t)r * hidden + h] * w[h];
        pred[r] = s + b;
    }
}

/* dout[r,h] = dpred[r] w[h]; dw[h] = sum_r dpred[r] out[r,h]; db = sum_r dpred[r] */
void oracle_head_backward_f64(int rows, int hidden, const double* out, const double* w, const double* dpred,
                              double* dout, double* dw, double* db) {
    for (int h = 0; h < hidden; ++h) dw[h] = 0.0;
    double sb = 0.0;
    for (int r = 0; r < rows; ++r) {
        const double g = dpred[r];
        sb += g;
        for (int h = 0; h < hidden; ++h) {
            dw[h] += g * out[(size_t)r * hidden + h];
            if (dout) dout[(size_t)r * hidden + h] = g * w[h];
        }
    }
    *db = sb;
}

/* mean of (pred - target)^2 */
double oracle_mse_forward_f64(size_t n, const double* pred, const double* target) {
    double s = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double d = pred[i] - target[i];
        s += d * d;
    }
    return s / (double)n;
}

/* grad_pred = g * 2 (pred - target) / n */
void oracle_mse_backward_f64(size_t n, const double* pred, const double* target, double g, double* grad) {
    for (size_t i = 0; i < n; ++i) grad[i] = 2.0 * (pred[i] - target[i]) / (double)n * g;
}

/* One AdamW step (step = 1, 2, ...) on n elements, in place on p, m, v. */
void oracle_adamw_step_f64(size_t n, double* p, const double* g, double* m, double* v, double lr, double beta1,
                           double beta2, double eps, double weight_decay, int step) {
    const double bc1 = 1.0 - pow(beta1, step);
    const double bc2 = 1.0 - pow(beta2, step);
    for (size_t i = 0; i < n; ++i) {
        p[i] *= 1.0 - lr * weight_decay;
        m[i] = beta1 * m[i] + (1.0 - beta1) * g[i];
        v[i] = beta2 * v[i] + (1.0 - beta2) * g[i] * g[i];
        const double mhat = m[i] / bc1;
        const double vhat = v[i] / bc2;
        p[i] -= lr * mhat / (sqrt(vhat) + eps);
    }
}
