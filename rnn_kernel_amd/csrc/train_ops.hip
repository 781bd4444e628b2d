// Training-step operations on either side of the GRU in the reference's
// benchmark harness: the Linear(H, 1) head, the mean-squared-error loss and
// the AdamW update (rnn_benchmark.py:510,526,618-639).  All of them are
// HBM-bound elementwise passes or reductions; every reduction runs in a
// fixed order (per-block partial sums, then one ordered pass over the
// partials), so results are bitwise reproducible run to run.
#include "rka_internal.h"

#include <algorithm>
#include <cmath>

namespace rka {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxReduceBlocks = 2048;   // partial sums of a loss reduction
constexpr int kHeadBlocks = 512;         // row ranges of the head's dw reduction

// Sum over the block's threads in a fixed order: each wavefront's 64 values
// by a butterfly of lane exchanges, then the four wavefront sums in order
// (one barrier instead of a tree of eight); valid in every thread.
// `scratch` holds kThreads / 64 floats.
__device__ __forceinline__ float block_sum_waves(float v, float* scratch) {
    static_assert(kThreads == 256, "four wavefronts");
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    return (scratch[0] + scratch[1]) + (scratch[2] + scratch[3]);
}

// Sum over the block's threads in a fixed tree order; the result is valid in
// thread 0.  `scratch` holds kThreads floats.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    scratch[threadIdx.x] = v;
    __syncthreads();
#pragma unroll
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) scratch[threadIdx.x] += scratch[threadIdx.x + s];
        __syncthreads();
    }
    return scratch[0];
}

// ------------------------------------------------------------------ MSE ---
// The target is read with streaming loads: it is not needed again in the
// step, and keeping it out of the MALL leaves room there for the activations
// the backward recurrence reads next (backward recurrence ~2 us faster at c2).
__device__ __forceinline__ float4 load_streaming(const float4* p) {
    typedef float v4 __attribute__((ext_vector_type(4)));
    const v4 v = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// Block b sums (pred - target)^2 over its contiguous range of `chunk`
// elements.  Vector form (chunk a multiple of 4, both operands 16-byte
// aligned): thread t takes float4 t, t + 256, ... of the range into four
// running sums (one per component), combined as (s0 + s1) + (s2 + s3);
// scalar form: elements t, t + 256, ... into one sum.
__global__ __launch_bounds__(kThreads) void mse_partial_kernel(const float* __restrict__ pred,
                                                               const float* __restrict__ target, size_t n,
                                                               size_t chunk, int vec, float* __restrict__ partial) {
    __shared__ float scratch[kThreads / 64];
    const size_t beg = (size_t)blockIdx.x * chunk;
    const size_t end = beg + chunk < n ? beg + chunk : n;
    float acc = 0.f;
    if (vec) {
        const float4* p4 = reinterpret_cast<const float4*>(pred + beg);
        const float4* t4 = reinterpret_cast<const float4*>(target + beg);
        const size_t n4 = (end - beg) / 4;
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll 4
        for (size_t i = threadIdx.x; i < n4; i += kThreads) {
            const float4 a = p4[i], b = load_streaming(t4 + i);
            const float dx = a.x - b.x, dy = a.y - b.y, dz = a.z - b.z, dw = a.w - b.w;
            s0 = fmaf(dx, dx, s0);
            s1 = fmaf(dy, dy, s1);
            s2 = fmaf(dz, dz, s2);
            s3 = fmaf(dw, dw, s3);
        }
        // the last range may end inside a float4
        for (size_t i = beg + 4 * n4 + threadIdx.x; i < end; i += kThreads) {
            const float d = pred[i] - target[i];
            s0 = fmaf(d, d, s0);
        }
        acc = (s0 + s1) + (s2 + s3);
    } else {
        for (size_t i = beg + threadIdx.x; i < end; i += kThreads) {
            const float d = pred[i] - target[i];
            acc = fmaf(d, d, acc);
        }
    }
    const float s = block_sum_waves(acc, scratch);
    if (threadIdx.x == 0) partial[blockIdx.x] = s;
}

// loss[0] = (sum of the nb <= kMaxReduceBlocks partials, thread t summing
// t, t + 256, ... in order, then the fixed tree) / n.  The thread's loads are
// all issued before the additions (one memory latency instead of eight).
__global__ __launch_bounds__(kThreads) void mse_finish_kernel(const float* __restrict__ partial, int nb, size_t n,
                                                              float* __restrict__ loss) {
    __shared__ float scratch[kThreads];
    constexpr int kPer = kMaxReduceBlocks / kThreads;
    float v[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int i = (int)threadIdx.x + r * kThreads;
        v[r] = i < nb ? partial[i] : 0.f;
    }
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < kPer; ++r) acc += v[r];
    const float s = block_sum(acc, scratch);
    if (threadIdx.x == 0) loss[0] = s / (float)n;
}

// grad_pred = grad_loss * 2 (pred - target) / n  (torch's mse_loss backward
// for reduction='mean': norm = 2 / n, grad = norm * (pred - target) * grad);
// float4 per thread when all three arrays are 16-byte aligned.
__global__ __launch_bounds__(kThreads) void mse_backward_kernel(const float* __restrict__ pred,
                                                                const float* __restrict__ target,
                                                                const float* __restrict__ grad_loss, size_t n,
                                                                int vec, float* __restrict__ grad_pred) {
    const float norm = 2.0f / (float)n;
    const float g = grad_loss[0];
    const size_t stride = (size_t)gridDim.x * kThreads;
    size_t first = 0;
    if (vec) {
        const size_t n4 = n / 4;
        const float4* p4 = reinterpret_cast<const float4*>(pred);
        const float4* t4 = reinterpret_cast<const float4*>(target);
        float4* g4 = reinterpret_cast<float4*>(grad_pred);
        for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
            const float4 a = p4[i], b = load_streaming(t4 + i);
            g4[i] = make_float4(norm * (a.x - b.x) * g, norm * (a.y - b.y) * g, norm * (a.z - b.z) * g,
                                norm * (a.w - b.w) * g);
        }
        first = 4 * n4;
    }
    for (size_t i = first + (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        grad_pred[i] = norm * (pred[i] - target[i]) * g;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Blocks of the loss reduction and the range of each (a multiple of 4).
int mse_blocks(size_t n, size_t* chunk) {
    const size_t nb = std::min<size_t>(kMaxReduceBlocks, (n + 4095) / 4096);
    const size_t b = nb < 1 ? 1 : nb;
    *chunk = ((n + b - 1) / b + 3) / 4 * 4;
    return (int)((n + *chunk - 1) / *chunk);
}

// ----------------------------------------------------------------- head ---
// pred[r] = sum_h out[r, h] w[h] + b[0]; one wavefront per row, lane l
// summing h = l, l + 64, ... in order, then a fixed butterfly across lanes.
__global__ __launch_bounds__(kThreads) void head_forward_kernel(const float* __restrict__ out,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ b, int rows, int hidden,
                                                                float* __restrict__ pred) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* o = out + (size_t)row * hidden;
    float acc = 0.f;
    for (int h = lane; h < hidden; h += 64) acc = fmaf(o[h], w[h], acc);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) pred[row] = acc + b[0];
}

// dout[r, h] = dpred[r] w[h] (if dout), and per row range of block k:
// partial[k][h] = sum_r dpred[r] out[r, h], partial[k][hidden] = sum_r dpred[r]
// (rows in order, thread t owning h = t, t + 256, ...).
__global__ __launch_bounds__(kThreads) void head_backward_partial_kernel(
    const float* __restrict__ out, const float* __restrict__ w, const float* __restrict__ dpred, int rows,
    int hidden, int rows_per_block, float* __restrict__ dout, float* __restrict__ partial) {
    const int r0 = blockIdx.x * rows_per_block;
    const int r1 = min(rows, r0 + rows_per_block);
    float* part = partial + (size_t)blockIdx.x * (hidden + 1);
    for (int h = threadIdx.x; h <= hidden; h += kThreads) {
        const bool bias = h == hidden;
        const float wh = bias ? 0.f : w[h];
        float acc = 0.f;
#pragma unroll 8
        for (int r = r0; r < r1; ++r) {
            const float g = dpred[r];
            if (bias) {
                acc += g;
            } else {
                const size_t idx = (size_t)r * hidden + h;
                acc = fmaf(g, out[idx], acc);
                if (dout) dout[idx] = g * wh;
            }
        }
        part[h] = acc;
    }
}

// dw[h] = sum_k partial[k][h] (k in order); db[0] = sum_k partial[k][hidden]
__global__ __launch_bounds__(kThreads) void head_backward_finish_kernel(const float* __restrict__ partial, int nb,
                                                                        int hidden, float* __restrict__ dw,
                                                                        float* __restrict__ db) {
    const int h = blockIdx.x * kThreads + threadIdx.x;
    if (h > hidden) return;
    float acc = 0.f;
    for (int k = 0; k < nb; ++k) acc += partial[(size_t)k * (hidden + 1) + h];
    if (h < hidden)
        dw[h] = acc;
    else
        db[0] = acc;
}

int head_blocks(int rows, int* rows_per_block) {
    const int nb = std::max(1, std::min(kHeadBlocks, rows));
    *rows_per_block = (rows + nb - 1) / nb;
    return (rows + *rows_per_block - 1) / *rows_per_block;
}

// ---------------------------------------------------------------- AdamW ---
constexpr int kAdamMaxTensors = 16;

struct AdamTensor {
    float* p;
    const float* g;
    float* m;
    float* v;
    size_t n;
};

struct AdamArgs {
    AdamTensor t[kAdamMaxTensors];
    int count;
    float beta2, eps;
    // scalars formed in double on the host and rounded once, as torch forms
    // them from Python floats (1 - beta2 is not 1 - (float)beta2)
    float decay;           // 1 - lr * weight_decay
    float w1, w2;          // 1 - beta1, 1 - beta2
    float step_size;       // lr / (1 - beta1^step)
    float bc2_sqrt;        // sqrt(1 - beta2^step)
};

// torch.optim.AdamW's update (decoupled weight decay), in its order:
//   p *= 1 - lr wd;  m = lerp(m, g, 1 - beta1);  v = beta2 v + (1 - beta2) g^2
//   p -= step_size * m / (sqrt(v) / sqrt(1 - beta2^step) + eps)
// grid.y = tensor, grid.x strides over its elements.
__global__ __launch_bounds__(kThreads) void adamw_kernel(AdamArgs a) {
    const AdamTensor t = a.t[blockIdx.y];
    const float decay = a.decay, w1 = a.w1, w2 = a.w2;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < t.n; i += (size_t)gridDim.x * kThreads) {
        const float g = t.g[i];
        float p = t.p[i] * decay;
        // lerp(m, g, w) with w < 0.5: m + w (g - m)
        const float m = t.m[i] + w1 * (g - t.m[i]);
        const float v = t.v[i] * a.beta2 + w2 * g * g;
        const float denom = sqrtf(v) / a.bc2_sqrt + a.eps;
        p = p - a.step_size * (m / denom);
        t.p[i] = p;
        t.m[i] = m;
        t.v[i] = v;
    }
}

}  // namespace
}  // namespace rka

using namespace rka;

extern "C" {

size_t rka_mse_workspace_bytes(size_t n) {
    size_t chunk = 0;
    return (size_t)mse_blocks(n, &chunk) * sizeof(float);
}

int rka_mse_forward(const float* pred, const float* target, float* loss, void* workspace, size_t workspace_bytes,
                    size_t n, void* stream) {
    if (n == 0 || !pred || !target || !loss) return fail(RKA_ERR_INVALID_ARGUMENT, "mse_forward: bad arguments");
    size_t chunk = 0;
    const int nb = mse_blocks(n, &chunk);
    if (!workspace || workspace_bytes < (size_t)nb * sizeof(float))
        return fail(RKA_ERR_WORKSPACE_TOO_SMALL, "mse_forward: workspace too small");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    float* partial = reinterpret_cast<float*>(workspace);
    const int vec = (aligned16(pred) && aligned16(target)) ? 1 : 0;
    hipLaunchKernelGGL(mse_partial_kernel, dim3(nb), dim3(kThreads), 0, s, pred, target, n, chunk, vec, partial);
    RKA_RETURN_IF_HIP(hipGetLastError());
    hipLaunchKernelGGL(mse_finish_kernel, dim3(1), dim3(kThreads), 0, s, partial, nb, n, loss);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

int rka_mse_backward(const float* pred, const float* target, const float* grad_loss, float* grad_pred, size_t n,
                     void* stream) {
    if (n == 0 || !pred || !target || !grad_loss || !grad_pred)
        return fail(RKA_ERR_INVALID_ARGUMENT, "mse_backward: bad arguments");
    const int vec = (aligned16(pred) && aligned16(target) && aligned16(grad_pred)) ? 1 : 0;
    const size_t blocks = std::min<size_t>((n / (vec ? 4 : 1) + kThreads - 1) / kThreads, 4096);
    hipLaunchKernelGGL(mse_backward_kernel, dim3((unsigned)std::max<size_t>(blocks, 1)), dim3(kThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), pred, target, grad_loss, n, vec, grad_pred);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

int rka_head_forward(const float* out, const float* w, const float* b, float* pred, int rows, int hidden,
                     void* stream) {
    if (rows < 1 || hidden < 1 || !out || !w || !b || !pred)
        return fail(RKA_ERR_INVALID_ARGUMENT, "head_forward: bad arguments");
    const int per_block = kThreads / 64;
    hipLaunchKernelGGL(head_forward_kernel, dim3((rows + per_block - 1) / per_block), dim3(kThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), out, w, b, rows, hidden, pred);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

size_t rka_head_backward_workspace_bytes(int rows, int hidden) {
    if (rows < 1 || hidden < 1) return 0;
    int rpb = 0;
    const int nb = head_blocks(rows, &rpb);
    return (size_t)nb * (hidden + 1) * sizeof(float);
}

int rka_head_backward(const float* out, const float* w, const float* dpred, float* dout, float* dw, float* db,
                      void* workspace, size_t workspace_bytes, int rows, int hidden, void* stream) {
    if (rows < 1 || hidden < 1 || !out || !w || !dpred || !dw || !db)
        return fail(RKA_ERR_INVALID_ARGUMENT, "head_backward: bad arguments");
    int rpb = 0;
    const int nb = head_blocks(rows, &rpb);
    if (!workspace || workspace_bytes < (size_t)nb * (hidden + 1) * sizeof(float))
        return fail(RKA_ERR_WORKSPACE_TOO_SMALL, "head_backward: workspace too small");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    float* partial = reinterpret_cast<float*>(workspace);
    hipLaunchKernelGGL(head_backward_partial_kernel, dim3(nb), dim3(kThreads), 0, s, out, w, dpred, rows, hidden, rpb,
                       dout, partial);
    RKA_RETURN_IF_HIP(hipGetLastError());
    hipLaunchKernelGGL(head_backward_finish_kernel, dim3((hidden + 1 + kThreads - 1) / kThreads), dim3(kThreads), 0,
                       s, partial, nb, hidden, dw, db);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

int rka_adamw_step(float* const* params, const float* const* grads, float* const* exp_avgs,
                   float* const* exp_avg_sqs, const size_t* numels, int count, double lr, double beta1,
                   double beta2, double eps, double weight_decay, int step, void* stream) {
    if (count < 0 || (count > 0 && (!params || !grads || !exp_avgs || !exp_avg_sqs || !numels)) || step < 1)
        return fail(RKA_ERR_INVALID_ARGUMENT, "adamw_step: bad arguments");
    // bias corrections in double, as torch computes them from Python floats
    const double bc1 = 1.0 - std::pow(beta1, (double)step);
    const double bc2 = 1.0 - std::pow(beta2, (double)step);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    for (int first = 0; first < count; first += kAdamMaxTensors) {
        AdamArgs a{};
        a.count = std::min(kAdamMaxTensors, count - first);
        size_t max_n = 0;
        for (int i = 0; i < a.count; ++i) {
            const int j = first + i;
            if (!params[j] || !grads[j] || !exp_avgs[j] || !exp_avg_sqs[j])
                return fail(RKA_ERR_INVALID_ARGUMENT, "adamw_step: null tensor pointer");
            a.t[i] = AdamTensor{params[j], grads[j], exp_avgs[j], exp_avg_sqs[j], numels[j]};
            max_n = std::max(max_n, numels[j]);
        }
        if (max_n == 0) continue;
        a.beta2 = (float)beta2;
        a.eps = (float)eps;
        a.decay = (float)(1.0 - lr * weight_decay);
        a.w1 = (float)(1.0 - beta1);
        a.w2 = (float)(1.0 - beta2);
        a.step_size = (float)(lr / bc1);
        a.bc2_sqrt = (float)std::sqrt(bc2);
        const unsigned gx = (unsigned)std::min<size_t>((max_n + kThreads - 1) / kThreads, 1024);
        hipLaunchKernelGGL(adamw_kernel, dim3(gx, a.count), dim3(kThreads), 0, s, a);
        RKA_RETURN_IF_HIP(hipGetLastError());
    }
    return 0;
}

}  // extern "C"
