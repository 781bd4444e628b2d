// Device-side pieces shared by the persistent recurrence kernels.
//
// Cross-workgroup exchange is flag-in-data: a published value is a 64-bit
// word {fp32 bits, step tag} written with one store and read with
// agent-scope atomic loads (global_load ... sc1), so a reader needs one round
// trip per step and no separate barrier counter.  The store is a plain one
// when every workgroup of the exchange group runs on one XCD (checked at
// start-up through the XCC_ID register), else an agent-scope one.  Two slots
// (step parity) suffice because a writer can only reach step t+2 after every
// reader of its group has published step t+1, i.e. finished reading step t.
//
// Waits are bounded by a poll count (default 2^24 rounds, about 2 s at the
// fastest poll rate; tests lower it from the host).  A wait that gives up
// raises the launch's abort flag and
// counts the launch in a per-device abort counter the host can read; every
// workgroup then leaves its time loop, writes NaN into each output row it
// did not store and NaN final states, so an aborted launch can only leave
// values that are either NaN or the ones a complete run computes.
#pragma once

#include "rka_internal.h"

namespace rka {
namespace rec {

constexpr int NW = 8;          // wavefronts per workgroup
constexpr int NTH = NW * 64;   // threads per workgroup
constexpr int MAX_XCC_BLOCKS = 4096;  // workgroups covered by the start-up XCD check

// How a launch's waits give up.  `flag` is the call's abort flag
// (workspace; shared by the launches of one call: batch slices, time
// ranges), `count` the per-device counter of aborted calls; a wait
// gives up after `spin_limit` poll rounds, or when it sees (every 1024
// rounds) that another workgroup has raised the flag.  The bound is a poll
// count rather than a clock: on MI355X a wall-clock check on the same
// once-per-1024-rounds branch of the poll loop made a c2 backward launch 6 %
// slower although the branch is never taken in a normal run.  Every grid is
// resident (batch slices), so a wait lasts about one step unless other
// kernels hold CUs the grid needs.
struct WaitCtl {
    int* flag;
    unsigned long long* count;
    int spin_limit;
};

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
    unsigned long long* abort_count = nullptr;  // per-device counter of aborted launches
    // one {xcc, tag} word per workgroup (nullptr: grid too large, exchange
    // through memory); tag distinct per launch on one workspace
    unsigned long long* xcc_words = nullptr;
    unsigned xcc_tag = 0;
    int spin_limit = 1 << 24;                 // poll rounds before a wait gives up
    // Forward: added to every step tag of the launch's exchange words.  Calls
    // that share exchange memory across calls (the allocation-free forward)
    // take a different base per call, so a word left or written by another
    // call never matches; with a private, freshly zeroed workspace it is 0
    // (the backward, which has no allocation-free entry point, ignores it).
    unsigned tag_base = 0;
    // Failure injection for tests (-1: off): the workgroup with this block
    // index publishes every word into the other step-parity slot, where its
    // partners never look for it, so their waits give up deterministically.
    int stall_block = -1;
    int B = 0, T = 0, H = 0;
    // backward: steps t_end-1 down to t_begin of a sequence of T (strides and
    // exchange tags use the global step, so consecutive ranges continue one
    // another on the same, once-zeroed workspace)
    int t_begin = 0, t_end = 0;
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

// Publishing store for readers that all run on the writer's XCD.  A plain
// store (global_store without scope bits) leaves the line dirty in the XCD's
// L2, where the agent-scope loads of the readers hit it; the agent-scope
// store (sc1) writes through to memory and the readers' loads then fetch it
// from there.  Measured on MI355X, ping-pong between two CUs of one XCD:
// 1.00 us round trip against 1.39 us; across XCDs only the agent-scope
// store is ever seen.
__device__ __forceinline__ void store_word_xcd(unsigned long long* p, unsigned long long w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

__device__ __forceinline__ void publish_word(unsigned long long* p, unsigned long long w, bool xcd_local) {
    if (xcd_local)
        store_word_xcd(p, w);
    else
        store_word(p, w);
}

// Publishes N words computed before the call: one branch on the (uniform)
// locality around all N stores, and every value fixed ahead of the first
// store.  A value computed between two stores would make the compiler wait
// for the whole vector-memory counter (the earlier store included) before
// it, since stores and loads retire through the same in-order counter.
template <int N>
__device__ __forceinline__ void publish_words(unsigned long long* const (&p)[N], const unsigned long long (&w)[N],
                                             bool xcd_local) {
#pragma unroll
    for (int v = 0; v < N; ++v) asm volatile("" ::"v"(w[v]));
    if (xcd_local) {
#pragma unroll
        for (int v = 0; v < N; ++v) store_word_xcd(p[v], w[v]);
    } else {
#pragma unroll
        for (int v = 0; v < N; ++v) store_word(p[v], w[v]);
    }
}

// Raises the abort flag; the lane that raises it first counts the call in
// the per-device abort counter (read by rka_recurrence_abort_count).
__device__ __forceinline__ void raise_abort(const WaitCtl& wc) {
    if (__hip_atomic_exchange(wc.flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0 && wc.count != nullptr)
        __hip_atomic_fetch_add(wc.count, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool abort_raised(const WaitCtl& wc) {
    return __hip_atomic_load(wc.flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Index of the XCD (accelerator complex die) this wavefront runs on.
__device__ __forceinline__ unsigned xcc_id() {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xfu;
}

// Placement of this workgroup in a grid of G exchange groups of S
// workgroups (batch-row group g, slice s).  The launch needs no
// co-residency guarantee: workgroups are dispatched to the 8 XCDs round
// robin (block b to XCD (b + c) mod 8) and, within an XCD, in increasing
// block order, so a mapping in which every group precedes every later group
// in each XCD's dispatch order always makes progress (the earliest group
// that is not fully resident has its missing members at the heads of their
// XCDs' queues, behind groups that can finish).
// The grid holds GX = gridDim.x / S groups, GX >= G:
//   GX a multiple of 8: the S members of group g are consecutive in the
//     dispatch order of one XCD: blocks x + 8 (l S + k), x = g mod 8,
//     l = g / 8, k < S, so the group also shares that XCD's L2.  A grid
//     of G groups rounded up to whole multiples of 8 (GX > G) has padding
//     workgroups, g >= G, which the kernels end before their first barrier;
//   otherwise (GX = G): consecutive block ids g S .. g S + S - 1.
struct GroupCoords {
    int g, s;           // group and slice of this workgroup
    int first, stride;  // the group's blocks: first + k stride, k < S
};
__device__ __forceinline__ GroupCoords group_coords(int S) {
    const int b = blockIdx.x;
    const int GX = (int)gridDim.x / S;
    if (GX % 8 == 0) {
        const int x = b % 8, q = b / 8, l = q / S, k = q % S;
        return {x + 8 * l, k, x + 8 * l * S, 8};
    }
    return {b / S, b % S, (b / S) * S, 1};
}

// Whether every member of this workgroup's exchange group (blocks first +
// k * stride, k < count, this one included) runs on this workgroup's XCD.
// Each workgroup publishes {xcc, tag} at words[blockIdx.x] with an
// agent-scope store and reads the members' words (bounded spin); all members
// read the same words and reach the same answer.  `tag` must differ from
// any value the words may still hold from an earlier launch on the same
// workspace.  Called by every thread of the workgroup (always contains a
// barrier); words == nullptr answers false without an exchange.
__device__ __forceinline__ bool group_on_one_xcd(unsigned long long* words, int first, int stride, int count,
                                                 unsigned tag, const WaitCtl& wc, int* s_flag) {
    if (words == nullptr) {
        __syncthreads();
        return false;
    }
    const unsigned me = xcc_id();
    if (threadIdx.x == 0) {
        *s_flag = 1;
        store_word(words + blockIdx.x, ((unsigned long long)tag << 32) | me);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        bool same = true;
        for (int k = (int)threadIdx.x; k < count; k += 64) {
            const unsigned long long* p = words + first + (size_t)k * stride;
            unsigned long long w = load_word(p);
            int spins = 0;
            while ((unsigned)(w >> 32) != tag) {
                if (++spins >= wc.spin_limit || ((spins & 1023) == 0 && abort_raised(wc))) {
                    raise_abort(wc);
                    break;
                }
                w = load_word(p);
            }
            same = same && (unsigned)(w >> 32) == tag && (unsigned)w == me;
        }
        if (!__all(same) && threadIdx.x == 0) *s_flag = 0;
    }
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(*s_flag) != 0;
}

// Waits for N words of this lane at once: every poll round re-reads all N,
// so words published together cost one round trip however many there are.
// One round is in flight at a time: measured between two CUs of one XCD on
// MI355X, a ping-pong round trip is 680 ns with one polling load in flight
// and 705-920 ns with two to four staggered ones (an L2-hit load takes
// ~100 ns; the rest is the store becoming visible).  Every word is waited
// for and tested in each round (no short-circuit), so no load is still
// pending on return: the in-order vector-memory counter would otherwise
// make the next wait on anything issued after the poll cover it too.  w[]
// holds the first reads on entry and the matching words on return; a word
// with valid[v] false counts as ready.  Every p[v] is loaded
// unconditionally (no exec-mask branches in the loop), so an invalid lane
// must point at a word that a valid lane of the same instruction loads: the
// duplicate costs no request, whereas one stand-in address polled by every
// wave of the grid would be a hot spot.
// UNIFORM: the wavefront polls as one (every lane reloads its words each
// round until no lane is missing one; a tagged word does not change before
// its reader has passed the step, so ready lanes reload the same value).
// Otherwise each lane leaves the loop when its own words are in, which
// costs some thirty scalar instructions of exec-mask bookkeeping per round.
// Measured at c2 (same box, alternating pairs, µs per launch): forward (one
// word per lane) 445.6-446.4 uniform vs 451.8-453.2 per lane; the backward
// (several words per lane) 453.5 / 454.7 uniform vs 448.4 / 450.1, and the
// four-row forward spills with it, so both keep the per-lane loop.
// LIKELY: the first test is marked as the expected outcome, so that the
// compiler lays the path on which every word is in as straight-line code
// (one-row forward at c2: 410 -> 404 us per launch; the one-row backward
// and the four-row forward measured slower with it, 5 and 55 us).
template <int N, bool UNIFORM = false, bool LIKELY = false>
__device__ __forceinline__ void wait_words(const unsigned long long* const (&p)[N], const bool (&valid)[N],
                                           unsigned long long (&w)[N], unsigned tag, const WaitCtl& wc, bool& ok) {
    auto ready = [&]() {
        bool r = true;
#pragma unroll
        for (int v = 0; v < N; ++v) asm volatile("" : "+v"(w[v]));
#pragma unroll
        for (int v = 0; v < N; ++v) r &= (!valid[v] || (unsigned)(w[v] >> 32) == tag);
        return r;
    };
    // Giving up: a word that never came would enter the caller's sums with
    // a stale value; NaN instead, so that whatever this step publishes from
    // it is NaN too and no workgroup still running can turn it into a
    // finite, wrong state.
    auto give_up = [&]() {
        ok = false;
#pragma unroll
        for (int v = 0; v < N; ++v)
            if (valid[v] && (unsigned)(w[v] >> 32) != tag) w[v] = ((unsigned long long)tag << 32) | 0x7fc00000ull;
    };
    // wave-uniform: no lane is missing a word
    auto all_ready = [&]() { return __builtin_amdgcn_ballot_w64(!ready()) == 0; };
    if (!ok) return;
    // With one word per lane the first test is a wave-wide vote in both forms:
    // it passes in nearly every step, and a vote takes no exec-mask branch
    // (c2 backward 431 -> 424 us per launch; with two words per lane, the
    // four-row backward, the per-lane test stays faster: 4.46 vs 4.52 ms)
    const bool first_ok = UNIFORM || N == 1 ? all_ready() : ready();
    if (LIKELY ? __builtin_expect(first_ok, 1) : first_ok) return;
    int spins = 0;
    for (;;) {
#pragma unroll
        for (int v = 0; v < N; ++v) w[v] = load_word(p[v]);
        if (UNIFORM ? all_ready() : ready()) break;
        ++spins;
        if (spins >= wc.spin_limit) {
            raise_abort(wc);
            give_up();
            break;
        }
        if ((spins & 1023) == 0 && abort_raised(wc)) {
            give_up();
            break;
        }
    }
}

}  // namespace rec

// Tiled kernels (W_hh slice in LDS; any hidden size that fits LDS).
int tiled_choose(int dir, int B, int H, const DeviceInfo& dev, int fixed_units, int fixed_pw, RecConfig* cfg);
int tiled_launch(int dir, const RecConfig& c, const rec::Args& a, hipStream_t stream);

// Register-resident kernels (W_hh slice in VGPRs; hidden size <= 256).
int reg_choose(int dir, int B, int H, const DeviceInfo& dev, int fixed_units, int fixed_rows, RecConfig* cfg);
int reg_launch(int dir, const RecConfig& c, const rec::Args& a, hipStream_t stream);

}  // namespace rka
