// Device-side pieces shared by the persistent recurrence kernels.
//
// Cross-workgroup exchange is flag-in-data: a published value is a 64-bit
// word {fp32 bits, step tag} written with one agent-scope atomic store
// (global_store ... sc1) and read with agent-scope atomic loads, so a reader
// needs one round trip per step and no separate barrier counter.  Two slots
// (step parity) suffice because a writer can only reach step t+2 after every
// reader of its group has published step t+1, i.e. finished reading step t.
// Spins are bounded: on time-out a device flag is raised, every workgroup
// leaves its time loop and writes its final state as NaN.
#pragma once

#include "rka_internal.h"

namespace rka {
namespace rec {

constexpr int NW = 8;          // wavefronts per workgroup
constexpr int NTH = NW * 64;   // threads per workgroup
constexpr int SPIN_LIMIT = 1 << 21;

// Host-side argument bundle of one recurrence launch.
struct Args {
    // forward
    const float* gx = nullptr;
    const float* b_hh = nullptr;
    float* hn = nullptr;
    // backward
    const float* dy = nullptr;
    const float* dhn = nullptr;
    float* gout = nullptr;
    float* dh0 = nullptr;
    // both
    const float* h0 = nullptr;
    const float* w_hh = nullptr;
    float* y = nullptr;              // written by forward, read by backward
    float* reserve = nullptr;        // written by forward (nullable), read by backward
    unsigned long long* exch = nullptr;
    int* abort_flag = nullptr;
    int B = 0, T = 0, H = 0;
};

// Gate nonlinearities from their definitions, on the hardware transcendental
// units: v_exp_f32 (2^x) and v_rcp_f32 (reciprocal, 1 ulp).
//   sigmoid(v) = 1 / (1 + e^-v),  tanh(v) = 1 - 2 / (1 + e^{2v})
// Saturation is exact: e^x overflows to +inf (rcp -> 0) or underflows to 0.
// Errors against float64 (measured by the gate-function test through
// rka_eval_gate_functions): sigmoid <= 1.2e-7 absolute, tanh <= 2.4e-7
// absolute, far inside the 1e-4 output tolerance of the path.  This keeps the
// owner wavefront's dependent chain short: the IEEE division sequence and the
// branchy library tanh cost ~0.3 us per step on the critical path.
__device__ __forceinline__ float exp_f(float v) { return __builtin_amdgcn_exp2f(v * 1.4426950408889634f); }
__device__ __forceinline__ float sigmoid_f(float v) { return __builtin_amdgcn_rcpf(1.0f + exp_f(-v)); }
__device__ __forceinline__ float tanh_f(float v) { return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + exp_f(2.0f * v)); }

// Sum of the 8 wavefront partials p(0..7) as a fixed tree (depth 3).
template <typename F>
__device__ __forceinline__ float tree8(F p) {
    return ((p(0) + p(1)) + (p(2) + p(3))) + ((p(4) + p(5)) + (p(6) + p(7)));
}

__device__ __forceinline__ unsigned long long pack_word(float v, unsigned tag) {
    return ((unsigned long long)tag << 32) | (unsigned long long)__float_as_uint(v);
}

__device__ __forceinline__ unsigned long long load_word(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_word(unsigned long long* p, unsigned long long w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Re-reads *p until its tag equals `tag` (w holds the first read).  Two
// loads are kept in flight (each check waits only for the older one), so a
// word that becomes visible between polls is seen about half a round trip
// later instead of a full one.  Returns the value; clears `ok` when the spin
// budget ran out or another workgroup raised the abort flag.
__device__ __forceinline__ float wait_word(const unsigned long long* p, unsigned long long w, unsigned tag,
                                           int* abort_flag, bool& ok) {
    if ((unsigned)(w >> 32) == tag || !ok) return __uint_as_float((unsigned)w);
    unsigned long long a = load_word(p);
    int spins = 0;
    for (;;) {
        const unsigned long long b = load_word(p);
        if ((unsigned)(a >> 32) == tag) {
            w = a;
            break;
        }
        a = load_word(p);
        if ((unsigned)(b >> 32) == tag) {
            w = b;
            break;
        }
        spins += 2;
        if (spins > SPIN_LIMIT) {
            __hip_atomic_store(abort_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = false;
            break;
        }
        if ((spins & 1023) == 0 &&
            __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
            ok = false;
            break;
        }
    }
    return __uint_as_float((unsigned)w);
}

__device__ __forceinline__ float bcast(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

}  // namespace rec

// Tiled kernels (W_hh slice in LDS; any hidden size that fits LDS).
int tiled_choose(int dir, int B, int H, const DeviceInfo& dev, int fixed_units, int fixed_pw, RecConfig* cfg);
int tiled_launch(int dir, const RecConfig& c, const rec::Args& a, hipStream_t stream);

// Register-resident kernels (W_hh slice in VGPRs; hidden size <= 256).
int reg_choose(int dir, int B, int H, const DeviceInfo& dev, int fixed_units, int fixed_rows, RecConfig* cfg);
int reg_launch(int dir, const RecConfig& c, const rec::Args& a, hipStream_t stream);

}  // namespace rka
