// Measurements of the two hardware rates the persistent recurrences' step is
// built from (bench.py reports both beside each recurrence's step time):
//
// - the cross-workgroup exchange: a ping-pong between pairs of workgroups on
//   one XCD, each side publishing a 64-bit tagged word with a plain store and
//   polling its partner's with agent-scope loads, exactly as the recurrence
//   kernels exchange h_t / G_h,t.  Every workgroup has eight wavefronts that
//   all poll (as the recurrences' do), and `pairs` pairs run at once (128
//   pairs: every CU of an MI355X busy).  Waits are bounded; a wait that gives
//   up is reported, not hidden;
// - the issue rate of non-packed fp32 FMAs (v_fmac_f32 with VGPR operands,
//   the recurrences' W_hh products): every CU runs 512-thread workgroups whose
//   lanes each advance independent FMA chains.
#include "rka_internal.h"

#include <algorithm>
#include <vector>

namespace rka {
namespace {

__device__ __forceinline__ unsigned long long poll_word(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block b plays side (b / 8) % 2 of pair 8 (b / 16) + b % 8: the two sides
// are eight block ids apart, so the round-robin dispatch puts them on one
// XCD (each side records its XCD so that the host can check).  The words of
// a pair sit on their own 256-byte block.  out[b] = elapsed 100 MHz ticks
// of `iters` round trips, xcc[b] = XCD, failed[b] = 1 if a wait gave up.
__global__ __launch_bounds__(512) void pingpong_kernel(unsigned long long* __restrict__ words, int iters, int pairs,
                                                       int spin_limit, long long* __restrict__ out,
                                                       int* __restrict__ xcc, int* __restrict__ failed) {
    const int b = blockIdx.x;
    const int pair = 8 * (b / 16) + b % 8;
    if (pair >= pairs) return;
    const bool first = (b / 8) % 2 == 0;
    unsigned long long* mine = words + (size_t)pair * 32 + (first ? 0 : 16);
    const unsigned long long* theirs = words + (size_t)pair * 32 + (first ? 16 : 0);
    __shared__ int s_fail;
    if (threadIdx.x == 0) s_fail = 0;
    __syncthreads();
    int fail = 0;
    const long long t0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < iters; ++i) {
        const unsigned long long want = first ? 2ull * i + 2 : 2ull * i + 1;
        if (!first) {
            int spins = 0;
            while (poll_word(theirs) != want && !fail)
                if (++spins >= spin_limit) fail = 1;
        }
        __syncthreads();
        if (threadIdx.x < 64 && !fail)
            __hip_atomic_store(mine, first ? 2ull * i + 1 : 2ull * i + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
        if (first) {
            int spins = 0;
            while (poll_word(theirs) != want && !fail)
                if (++spins >= spin_limit) fail = 1;
        }
        if (fail) s_fail = 1;
        __syncthreads();
        if (s_fail) break;
    }
    const long long t1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        out[b] = t1 - t0;
        unsigned v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
        xcc[b] = (int)(v & 0xfu);
        failed[b] = s_fail;
    }
}

__global__ void zero_words_kernel(unsigned long long* __restrict__ w, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) w[i] = 0;
}

// C independent accumulators a <- h * w + a per lane (v_fmac_f32, every
// operand a VGPR, as in the recurrences' W_hh products), 8 C FMAs per
// iteration; h and w are per-lane values near 1e-3 and 0.5, so no sum
// overflows or goes subnormal.  ticks[2 b] / ticks[2 b + 1] = 100 MHz clock
// at the start and end of block b, each taken after a barrier; out keeps the
// sums live.
template <int C>
__global__ __launch_bounds__(512) void fma_rate_kernel(float* __restrict__ out, long long* __restrict__ ticks,
                                                       int iters, float w0, float h0) {
    const float lanef = (float)(threadIdx.x & 63);
    const float w = w0 + 1e-6f * lanef;
    float h[4], a[C];
#pragma unroll
    for (int q = 0; q < 4; ++q) h[q] = h0 * (float)(q + 1) + 1e-7f * lanef;
#pragma unroll
    for (int c = 0; c < C; ++c) a[c] = 0.f;
    __syncthreads();
    const long long t0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int c = 0; c < C; ++c) a[c] = fmaf(h[(r + c) & 3], w, a[c]);
    }
    __syncthreads();
    const long long t1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) s += a[c];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        ticks[2 * blockIdx.x] = t0;
        ticks[2 * blockIdx.x + 1] = t1;
    }
}

}  // namespace
}  // namespace rka

using namespace rka;

extern "C" size_t rka_exchange_probe_workspace_bytes(int pairs) {
    if (pairs < 1 || pairs > 2048) return 0;
    const size_t blocks = (size_t)(pairs + 7) / 8 * 16;
    return (size_t)pairs * 32 * 8 + blocks * (8 + 4 + 4) + 256;
}

extern "C" int rka_measure_exchange_latency(int pairs, int iters, void* workspace, size_t workspace_bytes,
                                            double* round_trip_ns, int* same_xcd) {
    clear_error();
    if (pairs < 1 || pairs > 2048 || iters < 1 || iters > (1 << 20) || !round_trip_ns || !same_xcd)
        return fail(RKA_ERR_INVALID_ARGUMENT, "rka_measure_exchange_latency: pairs 1..2048, iters 1..2^20, outputs");
    const size_t need = rka_exchange_probe_workspace_bytes(pairs);
    if (!workspace || workspace_bytes < need)
        return fail(RKA_ERR_WORKSPACE_TOO_SMALL, "rka_measure_exchange_latency: workspace needs " +
                                                     std::to_string(need) + " bytes");
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    const int blocks = (pairs + 7) / 8 * 16;
    if (blocks > dev->num_cus)
        return fail(RKA_ERR_TOO_LARGE_FOR_RESIDENT_LAUNCH, "rka_measure_exchange_latency: more workgroups than CUs");
    char* base = reinterpret_cast<char*>(workspace);
    auto* words = reinterpret_cast<unsigned long long*>(base);
    auto* out = reinterpret_cast<long long*>(base + (size_t)pairs * 32 * 8);
    auto* xcc = reinterpret_cast<int*>(out + blocks);
    auto* failed = xcc + blocks;
    hipLaunchKernelGGL(zero_words_kernel, dim3(16), dim3(256), 0, nullptr, words, (size_t)pairs * 32);
    RKA_RETURN_IF_HIP(hipGetLastError());
    hipLaunchKernelGGL(pingpong_kernel, dim3(blocks), dim3(512), 0, nullptr, words, iters, pairs, 1 << 22, out, xcc,
                       failed);
    RKA_RETURN_IF_HIP(hipGetLastError());
    RKA_RETURN_IF_HIP(hipDeviceSynchronize());
    std::vector<long long> t(blocks);
    std::vector<int> x(blocks), f(blocks);
    RKA_RETURN_IF_HIP(hipMemcpy(t.data(), out, sizeof(long long) * blocks, hipMemcpyDeviceToHost));
    RKA_RETURN_IF_HIP(hipMemcpy(x.data(), xcc, sizeof(int) * blocks, hipMemcpyDeviceToHost));
    RKA_RETURN_IF_HIP(hipMemcpy(f.data(), failed, sizeof(int) * blocks, hipMemcpyDeviceToHost));
    double sum = 0;
    int n = 0, same = 1;
    for (int b = 0; b < blocks; ++b) {
        const int pair = 8 * (b / 16) + b % 8;
        if (pair >= pairs) continue;
        if (f[b]) return fail(RKA_ERR_INVALID_ARGUMENT, "rka_measure_exchange_latency: a wait gave up");
        if ((b / 8) % 2 == 0) {
            sum += (double)t[b];
            ++n;
            if (x[b] != x[b + 8]) same = 0;
        }
    }
    // s_memrealtime counts at 100 MHz: 10 ns per tick
    *round_trip_ns = n ? sum / n * 10.0 / iters : 0.0;
    *same_xcd = same;
    return 0;
}

namespace {

constexpr int kFmaProbeMaxBlocksPerCu = 2;
constexpr int kFmaProbeIters = 2000;

// One launch of fma_rate_kernel<C> with `per_cu` 512-thread workgroups per
// CU (2 per_cu wavefronts per SIMD); ns per wave64 FMA instruction per SIMD.
template <int C>
int time_fma(const DeviceInfo& dev, int per_cu, float* out, long long* ticks, double* ns) {
    const int blocks = dev.num_cus * per_cu;
    hipLaunchKernelGGL(fma_rate_kernel<C>, dim3(blocks), dim3(512), 0, nullptr, out, ticks, kFmaProbeIters, 0.5f,
                       1e-3f);
    RKA_RETURN_IF_HIP(hipGetLastError());
    RKA_RETURN_IF_HIP(hipDeviceSynchronize());
    std::vector<long long> t(2 * (size_t)blocks);
    RKA_RETURN_IF_HIP(hipMemcpy(t.data(), ticks, sizeof(long long) * t.size(), hipMemcpyDeviceToHost));
    long long first = t[0], last = t[1];
    for (int b = 0; b < blocks; ++b) {
        first = std::min(first, t[2 * b]);
        last = std::max(last, t[2 * b + 1]);
    }
    // per SIMD: 2 per_cu wavefronts x iters x 8 C instructions; 10 ns per tick
    const double insts = 2.0 * per_cu * kFmaProbeIters * 8.0 * C;
    *ns = (double)(last - first) * 10.0 / insts;
    return 0;
}

}  // namespace

extern "C" size_t rka_fma_probe_workspace_bytes(void) {
    const DeviceInfo* dev = nullptr;
    if (current_device_info(&dev) != 0) return 0;
    const size_t blocks = (size_t)dev->num_cus * kFmaProbeMaxBlocksPerCu;
    return blocks * 512 * sizeof(float) + blocks * 2 * sizeof(long long);
}

extern "C" int rka_measure_fma_rate(void* workspace, size_t workspace_bytes, double* ns_per_instruction,
                                    double* tflops) {
    clear_error();
    if (!ns_per_instruction || !tflops)
        return fail(RKA_ERR_INVALID_ARGUMENT, "rka_measure_fma_rate: null output");
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    const size_t need = rka_fma_probe_workspace_bytes();
    if (!workspace || workspace_bytes < need)
        return fail(RKA_ERR_WORKSPACE_TOO_SMALL, "rka_measure_fma_rate: workspace needs " + std::to_string(need) +
                                                     " bytes");
    const size_t blocks = (size_t)dev->num_cus * kFmaProbeMaxBlocksPerCu;
    auto* out = reinterpret_cast<float*>(workspace);
    auto* ticks = reinterpret_cast<long long*>(out + blocks * 512);
    double ns = 0, best = 0;
    RKA_RETURN_IF_ERR(time_fma<12>(*dev, 1, out, ticks, &ns));  // warm-up, not counted
    for (int per_cu = 1; per_cu <= kFmaProbeMaxBlocksPerCu; ++per_cu) {
        RKA_RETURN_IF_ERR(time_fma<12>(*dev, per_cu, out, ticks, &ns));
        if (best == 0 || ns < best) best = ns;
        RKA_RETURN_IF_ERR(time_fma<24>(*dev, per_cu, out, ticks, &ns));
        if (ns < best) best = ns;
    }
    *ns_per_instruction = best;
    // 64 lanes x 2 FLOP per instruction on each of the 4 SIMDs of every CU
    *tflops = best > 0 ? 4.0 * dev->num_cus * 128.0 / best * 1e-3 : 0.0;
    return 0;
}
