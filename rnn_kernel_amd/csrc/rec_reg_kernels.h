// Register-resident persistent GRU recurrences (hidden size <= 256).
//
// Workgroup (g, s) owns hidden units [64 s, 64 s + 64) of batch rows
// [R g, R g + R) (R = 1, 2 or 4 rows per workgroup, S = ceil(H / 64)
// slices); lane l of a row's owner wavefront is unit 64 s + l.  The W_hh
// entries the workgroup needs live in VGPRs for the whole sequence, every
// wavefront holding an equal share of each slice's k (forward) or j
// (backward) values, so the FMAs of the workgroup's own slice can run from
// LDS while the other slices' words are in flight.  The S workgroups of a
// group exchange one word per value and step (h_t forward, G_h,t backward)
// and sit on one XCD when the group count allows.
//
// Measured on MI355X (same box, alternating runs) against the designs this
// one replaced:
//   * wavefronts holding contiguous k (j) chunks with the exchanged words
//     replicated into 16-lane rows (v_permlane16/32_swap) and broadcast into
//     the FMAs by DPP row_newbcast, one barrier per step: at B=64, H=256,
//     T=512 forward 0.570 -> 0.529 ms, backward 0.615 -> 0.567 ms for the
//     local-slice form, and at H <= 192 (c3) steps 0.94 -> 0.80 ms (H = 64)
//     to 1.61 -> 1.35 ms (H = 192); with several rows per workgroup (c4,
//     B = 256) forward 2 rows in two waves of workgroups plus backward 4
//     rows resident: 5.4 vs 5.8 ms per layer;
//   * readlane broadcasts into scalar FMA operands instead of DPP: forward
//     0.726 vs 0.706 ms, backward 1.182 vs 0.934 ms;
//   * backward owner issuing its G stores and the loads of its next inputs
//     before the poll instead of after it: 0.943 vs 0.848 ms; the same in
//     the forward: 0.825 vs 0.782 ms;
//   * 128 units per workgroup (2 exchanging workgroups, twice the FMAs on
//     the owner's critical path): forward 1.67 vs 1.29 us/step;
//   * a ninth, non-polling wavefront for the gate math (it shares a SIMD with
//     two polling wavefronts): forward 1.6 vs 1.29 us/step;
//   * a poller wavefront relaying the exchanged words through LDS to the
//     others: forward 2.48 vs 1.54 us/step, backward 3.16 vs 2.21 us/step;
//   * backward exchanging per-slice partial sums of dh (forward-sized
//     exchange, one polling wavefront, but a second barrier and the FMAs
//     ahead of the publish): 2.56 vs ~2.3 us/step.
//
// Forward maths (src/rnn_kernel/a100/prod/kernels/a100_gru_h256_kernels.cu:756-776):
//   a = W_hh h_{t-1} + b_hh; r = sigmoid(gx_r + a_r); z = sigmoid(gx_z + a_z);
//   n = tanh(gx_n + r a_n); h_t = n + z (h_{t-1} - n); reserve[b, t, u] = (r, z, n, a_n)
// Backward maths (a100_gru_h256_kernels.cu:842-866,915-932), g = dh_t + dy_t:
//   dz = g (h_{t-1} - n), dn^ = g (1 - z)(1 - n^2), dr^ = dn^ a_n r (1 - r),
//   dz^ = dz z (1 - z), da_n = dn^ r; dh_{t-1} = g z + G_h W_hh;
//   g_out[b,t] = (da_n, dr^, dz^, dn^).
#pragma once

#include "rec_common.h"

#include <algorithm>
#include <type_traits>

namespace rka {
namespace {


using rec::NTH;
using rec::NW;

struct RegParams {
    int B, T, H;
    int G, S;      // groups of R rows, slices of 64 units
    int chunk;     // units per workgroup (64)
    int wvec;      // forward: W_hh rows may be read as aligned float4
    int t_begin, t_end;  // backward: time range processed
    unsigned long long* xcc_words;  // start-up XCD check (nullable)
    unsigned xcc_tag;
    unsigned tag_base;                    // forward: added to every step tag (rec::Args::tag_base)
    int spin_limit;                       // poll rounds before a wait gives up
    unsigned long long* abort_count;      // per-device count of aborted launches
    int stall_block;                      // test failure injection (rec::Args::stall_block)
};

// Forward recurrence, S = ceil(H / 64) slices of 64 units (one workgroup
// each) and R batch rows per workgroup, with the workgroup's own slice of
// h_{t-1} taken from LDS (S = 1: no exchange at all).  Every wavefront runs
// the FMAs of all R rows with the same weights; wavefront r < R owns row r
// (its gate math, outputs and exchange words).  The description below is
// for one row.
// Wavefront w takes units 32 (w / 4) + l % 32 of the slice and k quarter
// Q = w % 4: its half hf = l / 32 holds, for each slot j (slot 0 = its own
// slice, slots 1..S-1 = the others in rotation), the eight k =
// 64 ((s + j) mod S) + 16 Q + 8 hf + i of the unit's three W_hh rows.  The
// two halves' sums are added with a permlane swap, so each unit and gate
// has four wave partials to reduce (eight when every wave took all 64
// units: forward 0.481 vs 0.472 ms per launch).  After the owner publishes h_t it also writes
// it to LDS; a second barrier follows and every wavefront runs the own
// slot's 24 FMAs of step t+1 while the other slices' words are still on
// their way, leaving 72 FMAs per lane after they arrive (96 with the whole
// chunk polled; at S = 4).  The h values reach the FMAs as wave-uniform VGPRs read
// from LDS (broadcast ds_read_b128): the polled words are written to a
// wave-private LDS row first.  Measured on MI355X, a VGPR-operand v_fmac_f32
// issues at ~1.2 ns per SIMD with two waves per SIMD against ~2.0 ns for
// the row-broadcast DPP form and ~2.1 ns with an SGPR operand.
//
// IO (one row per workgroup): a ninth wavefront, which never polls, stores
// the outputs of each step from LDS, so the owner's per-step stores no
// longer sit in its vector-memory counter ahead of its next poll (the
// counter retires in issue order).  Same-box A/B at c2: 0.466 vs 0.488 ms
// per launch.  The owner still loads the input gates one step ahead, after
// its poll: loads that miss to HBM delay the return of every later load of
// the CU, the polls of all wavefronts included, so moving them to the I/O
// wavefront (registers or LDS-DMA, one to three steps ahead) measured 0.53
// to 0.57 ms, while the same copies from L2-resident addresses measured
// 0.455 ms.
template <int S, int R, bool IO, int NWF = NW, bool FULL = false>
__global__ __launch_bounds__(IO ? NWF * 64 + 64 : NWF * 64) void gru_fwd_local_kernel(
    const float* __restrict__ gx, const float* __restrict__ h0, const float* __restrict__ w_hh,
    const float* __restrict__ b_hh, float* __restrict__ y, float* __restrict__ hn,
    float* __restrict__ reserve, unsigned long long* __restrict__ exch, int* __restrict__ abort_flag,
    RegParams p) {
    static_assert(R == 1 || R == 2 || R == 4, "rows per workgroup");
    static_assert(!IO || R == 1, "the I/O wavefront serves one row");
    static_assert(NWF == 8 || (NWF == 16 && R == 1), "eight compute wavefronts, or sixteen at one row");
    constexpr int NR = S - 1;                 // remote slots
    constexpr int NQ = NWF / 2;               // k parts of a slot (a wave takes one for 32 units)
    constexpr int KP = 64 / NQ, KH = KP / 2;  // k per part, per wave half
    constexpr int NP = NR > 0 ? KH * NR : 4;  // polled h values per wave half and row
    static_assert(2 * NP <= 64, "a wave's polled words fit its 64 LDS entries");
    // [step parity][k part][gate][row][unit]; gate 3 takes the upper half's
    // copy of the n sum, so both halves store without a branch
    __shared__ float part[2][NQ][4][R][64];
    __shared__ __attribute__((aligned(16))) float hloc[2][R][64];
    // per wave and row: the polled h values, half h's NP at [h NP, h NP + NP)
    // (lane l's word at l; lanes past 2 NP write unread entries, so no lane
    // needs a branch)
    __shared__ __attribute__((aligned(16))) float hrem[NWF][R][64];
    __shared__ float io_out[IO ? 2 : 1][5][64];  // IO: outputs (h, r, z, n, a_n) of a step, by step parity
    __shared__ int s_abort;
    __shared__ int s_local;

    // FULL: H = 64 S (every slice whole), a compile-time constant; every
    // lane's unit exists, so the owner test is the same for the whole
    // wavefront and its branches need no lane masks
    const int B = p.B, T = p.T, H = FULL ? 64 * S : p.H;
    const int lane = threadIdx.x & 63;
    const int wave = FULL ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : threadIdx.x >> 6;
    const rec::GroupCoords gc = rec::group_coords(p.S);
    if (gc.g >= p.G) return;  // padding workgroup of a grid rounded up to whole XCDs
    const int s = gc.s;
    const int row0 = gc.g * R;    // the group's first batch row
    const int u = s * 64 + lane;  // the owner lane's unit
    const bool uvalid = FULL || u < H;
    // FMA layout: wave w takes units 32 (w / NQ) + l % 32 of the slice and k
    // part Q = w % NQ; half hf = l / 32 of the wave the KH k
    // 64 ((s + j) mod S) + KP Q + KH hf + i of slot j (for every row)
    const int hf = lane >> 5, uu = lane & 31, Q = wave % NQ;
    const int fu = 32 * (wave / NQ) + uu;  // the lane's FMA unit within the slice
    const int uf = s * 64 + fu;
    const bool ufvalid = uf < H;
    auto kofh = [&](int half, int j, int i) { return 64 * ((s + j) % S) + KP * Q + KH * half + i; };
    auto kof = [&](int j, int i) { return kofh(hf, j, i); };

    if constexpr (IO) {
        if (wave == NWF) {
            // The I/O wavefront: lane l is unit u of row row0.  Per step t,
            // before the step's first barrier, it stores the outputs of step
            // t-1 (written to io_out by the owner before the second barrier
            // of step t-1).  It takes both barriers of every step and leaves
            // the loop when the compute wavefronts do.
            if (threadIdx.x == NWF * 64) s_abort = 0;
            const bool valid = uvalid && row0 < B;
            float* yp = y + (size_t)row0 * T * H + u;
            float* rp = reserve ? reserve + (size_t)row0 * T * 4 * H + 4 * u : nullptr;
            auto store_step = [&](int t, const float (&o)[5]) {
                if (!valid) return;
                yp[(size_t)t * H] = o[0];
                if (reserve) *reinterpret_cast<float4*>(rp + (size_t)t * 4 * H) = make_float4(o[1], o[2], o[3], o[4]);
            };
            auto read_out = [&](int t, float (&o)[5]) {
#pragma unroll
                for (int c = 0; c < 5; ++c) o[c] = io_out[t & 1][c][lane];
            };
            const rec::WaitCtl wc{abort_flag, p.abort_count, p.spin_limit};
            (void)rec::group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, wc, &s_local);
            int t_stop = T;
            for (int t = 0; t < T; ++t) {
                if (t >= 1) {
                    float o[5];
                    read_out(t - 1, o);
                    store_step(t - 1, o);
                }
                __syncthreads();
                const bool abort_now = s_abort != 0;
                __syncthreads();
                if (abort_now) {
                    t_stop = t;
                    break;
                }
            }
            if (t_stop == T) {
                float o[5];
                read_out(T - 1, o);
                store_step(T - 1, o);
            } else {
                const float nan = __builtin_nanf("");
                const float o[5] = {nan, nan, nan, nan, nan};
                for (int t = t_stop; t < T; ++t) store_step(t, o);
            }
            return;
        }
    }

    // slot j's W_hh entries in w?[KH j .. KH j + KH - 1]
    float wr[KH * S], wz[KH * S], wn[KH * S];
    const bool vec = p.wvec != 0;
#pragma unroll
    for (int j = 0; j < S; ++j) {
#pragma unroll
        for (int i = 0; i < KH; i += 4) {
            const int k = kof(j, i);
            const float* pr = w_hh + (size_t)uf * H + k;
            const float* pz = pr + (size_t)H * H;
            const float* pn = pz + (size_t)H * H;
            if (vec) {
                const bool ok = ufvalid && k < H;
                const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
                const float4 a = ok ? *reinterpret_cast<const float4*>(pr) : z4;
                const float4 b = ok ? *reinterpret_cast<const float4*>(pz) : z4;
                const float4 c = ok ? *reinterpret_cast<const float4*>(pn) : z4;
                const int e = KH * j + i;
                wr[e] = a.x; wr[e + 1] = a.y; wr[e + 2] = a.z; wr[e + 3] = a.w;
                wz[e] = b.x; wz[e + 1] = b.y; wz[e + 2] = b.z; wz[e + 3] = b.w;
                wn[e] = c.x; wn[e + 1] = c.y; wn[e + 2] = c.z; wn[e + 3] = c.w;
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const bool ok = ufvalid && k + c < H;
                    wr[KH * j + i + c] = ok ? pr[c] : 0.f;
                    wz[KH * j + i + c] = ok ? pz[c] : 0.f;
                    wn[KH * j + i + c] = ok ? pn[c] : 0.f;
                }
            }
        }
    }

    // wave r < R owns row row0 + r: its gate math, outputs and exchange words
    const int orow = row0 + (wave < R ? wave : 0);
    const bool owner = wave < R && uvalid && orow < B;
    float h_prev = 0.f, bias_r = 0.f, bias_z = 0.f, bias_n = 0.f;
    float gxs[2][3];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int c = 0; c < 3; ++c) gxs[e][c] = 0.f;
    const float* gx_row = gx + (size_t)orow * T * 3 * H + u;
    auto load_gx = [&](float (&d)[3], int t) {
        const float* gp = gx_row + (unsigned)t * (unsigned)(3 * H);  // 32-bit: B T H < 2^29
        d[0] = gp[0];
        d[1] = gp[H];
        d[2] = gp[2 * H];
    };
    if (owner) {
        h_prev = h0[(size_t)orow * H + u];
        bias_r = b_hh[u];
        bias_z = b_hh[H + u];
        bias_n = b_hh[2 * H + u];
        load_gx(gxs[0], 0);
    }
    if (!IO && threadIdx.x == 0) s_abort = 0;
    const rec::WaitCtl wc{abort_flag, p.abort_count, p.spin_limit};
    const bool xlocal = rec::group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, wc, &s_local);

    // Lane l < 2 NP polls half l / NP, slot 1 + (l % NP) / 8, entry l % 8 of
    // every row; other lanes, and lanes of a k past H, re-read the wave's
    // first valid remote word (word 0 when it has none); a row past B reads
    // the group's first row.
    auto pkof = [&](int l) { return kofh(l / NP, 1 + (l % NP) / KH, l % KH); };
    int fallback = -1;
#pragma unroll
    for (int l = 0; l < 2 * NP * (NR > 0); ++l) {
        const int k = pkof(l);
        if (fallback < 0 && k < H) fallback = k;
    }
    const int pk = NR > 0 && lane < 2 * NP ? pkof(lane) : H;
    const bool pvalid = pk < H;
    const int pidx = pvalid ? pk : (fallback >= 0 ? fallback : 0);
    bool rvalid[R];
    int roff[R];  // word offset of row r within a slot (B H < 2^31)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rvalid[r] = row0 + r < B;
        roff[r] = (rvalid[r] ? row0 + r : row0) * H;
    }

    // the owner lane's word in the slot of each step parity, as 32-bit
    // unsigned offsets (2 B H < 2^32: the host keeps B H < 2^29); the
    // failure injection swaps the two
    const int pub_flip = (int)blockIdx.x == p.stall_block ? 1 : 0;
    const unsigned slot_words = (unsigned)B * (unsigned)H, my_word = (unsigned)orow * (unsigned)H + (unsigned)u;
    const unsigned pub_off[2] = {(unsigned)pub_flip * slot_words + my_word,
                                 (unsigned)(1 - pub_flip) * slot_words + my_word};
    // outputs of the previous step, stored after the next poll
    float o_h = 0.f, o_r = 0.f, o_z = 0.f, o_n = 0.f, o_a = 0.f;
    float* y_row = y + (size_t)orow * T * H + u;
    float* res_row = reserve ? reserve + (size_t)orow * T * 4 * H + 4 * u : nullptr;
    auto store_outputs = [&](int t) {
        y_row[(unsigned)t * (unsigned)H] = o_h;
        // the test on the kernel argument is wave-uniform (a per-lane pointer's
        // is not, and costs an exec-mask branch per step)
        if (reserve) *reinterpret_cast<float4*>(res_row + 4 * ((unsigned)t * (unsigned)H)) = make_float4(o_r, o_z, o_n, o_a);
    };
    // partial sums of the step in flight per row; the own slot's FMAs land
    // first.  Two accumulators per gate and row give each wave six
    // independent FMA chains; with four rows there are twelve chains with
    // one, which keeps that variant within 256 VGPRs (no scratch).
    constexpr int NACC = R == 4 ? 1 : 2;
    float ar[R][NACC], az[R][NACC], an[R][NACC];
    // slot j's FMAs of row r with its KH h values (wave-uniform)
    auto fma8 = [&](const float (&hv)[KH], int j, int r) {
#pragma unroll
        for (int i = 0; i < KH; ++i) {
            ar[r][i % NACC] = fmaf(hv[i], wr[KH * j + i], ar[r][i % NACC]);
            az[r][i % NACC] = fmaf(hv[i], wz[KH * j + i], az[r][i % NACC]);
            an[r][i % NACC] = fmaf(hv[i], wn[KH * j + i], an[r][i % NACC]);
        }
    };
    auto zero_acc = [&](int r) {
#pragma unroll
        for (int a = 0; a < NACC; ++a) ar[r][a] = az[r][a] = an[r][a] = 0.f;
    };
    auto acc_sum = [](const float (&a)[NACC]) {
        if constexpr (NACC == 2)
            return a[0] + a[1];
        else
            return a[0];
    };
    // KH consecutive floats of LDS as wave-uniform values
    auto lds8 = [](const float* src, float (&hv)[KH]) {
#pragma unroll
        for (int q = 0; q < KH; q += 4) {
            const float4 a = *reinterpret_cast<const float4*>(src + q);
            hv[q] = a.x; hv[q + 1] = a.y; hv[q + 2] = a.z; hv[q + 3] = a.w;
        }
    };
    auto local_fmas = [&](int par) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            zero_acc(r);
            float hl[KH];
            lds8(&hloc[par][r][KP * Q + KH * hf], hl);
            fma8(hl, 0, r);
        }
    };
    unsigned long long first_read[R];
#pragma unroll
    for (int r = 0; r < R; ++r) first_read[r] = 0;
    // step 0's own slot from h0
#pragma unroll
    for (int r = 0; r < R; ++r) {
        zero_acc(r);
        float hv[KH];
#pragma unroll
        for (int i = 0; i < KH; ++i) {
            const int k = kof(0, i);
            hv[i] = k < H && rvalid[r] ? h0[roff[r] + k] : 0.f;
        }
        fma8(hv, 0, r);
    }
    // kind: 1 = step 0 (its h values come from h0; it runs before the loop,
    // so no later step tests t), 3 = a step with at least one more after it
    // (its tests of t + 1 < T fold away), 0 = tested at run time (the last
    // steps).  Measured on MI355X (same box, three alternating pairs):
    // without the run-time tests in the bulk of the steps, c2 forward 401 ->
    // 393 us per launch, c5 7.70 -> 7.61 ms, H = 128 and 192 -5.5 and -3 us.
    auto step = [&](auto kind, int t, const float (&cur)[3], float (&nxt)[3]) -> bool {
        constexpr int KF = decltype(kind)::value;
        // @probe:step_begin
        if constexpr (NR > 0) {
            float hx[R];
            if constexpr (KF == 1) {
#pragma unroll
                for (int r = 0; r < R; ++r) hx[r] = pvalid && rvalid[r] ? h0[roff[r] + pidx] : 0.f;
            } else {
                const unsigned long long* src = exch + (size_t)((t - 1) & 1) * B * H + pidx;
                const unsigned long long* pp[R];
                bool pv[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    pp[r] = src + roff[r];
                    pv[r] = pvalid && rvalid[r];
                }
                bool ok = true;
                rec::wait_words<R, R == 1, R == 1>(pp, pv, first_read, p.tag_base + (unsigned)t, wc, ok);
#pragma unroll
                for (int r = 0; r < R; ++r) hx[r] = pv[r] ? __uint_as_float((unsigned)first_read[r]) : 0.f;
                if (__builtin_expect(!ok, 0)) s_abort = 1;
            }
            // lanes 0..NP-1 hold slot 1 + l / 8, entry l % 8 of half 0 (NP..
            // of half 1): through the wave's LDS rows to every lane (one wave
            // writes and reads the rows; LDS keeps a wave's accesses in order)
#pragma unroll
            for (int r = 0; r < R; ++r) hrem[wave][r][lane] = hx[r];
            __builtin_amdgcn_wave_barrier();
        }
        // with one row, its h values are read ahead of the owner's memory
        // operations
        float hv0[NR > 0 ? NR : 1][KH];
        if constexpr (R == 1) {
#pragma unroll
            for (int jj = 0; jj < NR; ++jj) lds8(&hrem[wave][0][NP * hf + KH * jj], hv0[jj]);
        }
        if (owner) {
            if (!IO && t > 0) store_outputs(t - 1);
            if (KF == 3 || t + 1 < T) load_gx(nxt, t + 1);
        }
        // @probe:polled
        if constexpr (NR > 0) {
            // four rows at four slices: every row one slot's h values at a
            // time (registers); otherwise row 0 all slots at once
            constexpr bool by_slot = R == 4 && S == 4;
            if constexpr (R > 1 && !by_slot) {
#pragma unroll
                for (int jj = 0; jj < NR; ++jj) lds8(&hrem[wave][0][NP * hf + KH * jj], hv0[jj]);
            }
            if constexpr (!by_slot) {
#pragma unroll
                for (int jj = 0; jj < NR; ++jj) fma8(hv0[jj], jj + 1, 0);
            }
#pragma unroll
            for (int r = by_slot ? 0 : 1; r < R; ++r) {
                if constexpr (by_slot) {
                    // one slot's h values at a time (registers)
#pragma unroll
                    for (int jj = 0; jj < NR; ++jj) {
                        __builtin_amdgcn_sched_barrier(0);
                        float hv[KH];
                        lds8(&hrem[wave][r][NP * hf + KH * jj], hv);
                        fma8(hv, jj + 1, r);
                    }
                } else {
                    // one row's h values at a time (registers)
                    __builtin_amdgcn_sched_barrier(0);
                    float hv[NR][KH];
#pragma unroll
                    for (int jj = 0; jj < NR; ++jj) lds8(&hrem[wave][r][NP * hf + KH * jj], hv[jj]);
#pragma unroll
                    for (int jj = 0; jj < NR; ++jj) fma8(hv[jj], jj + 1, r);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // halves: lanes 0-31 get the r sum and lanes 32-63 the z sum of
            // unit fu, every lane the n sum (lower half + upper half)
            const float r0 = acc_sum(ar[r]), z0 = acc_sum(az[r]), n0 = acc_sum(an[r]);
            const auto prz = __builtin_amdgcn_permlane32_swap(__float_as_uint(r0), __float_as_uint(z0), false, false);
            const auto pn = __builtin_amdgcn_permlane32_swap(__float_as_uint(n0), __float_as_uint(n0), false, false);
            part[t & 1][Q][hf][r][fu] = __uint_as_float(prz[0]) + __uint_as_float(prz[1]);
            part[t & 1][Q][2 + hf][r][fu] = __uint_as_float(pn[0]) + __uint_as_float(pn[1]);
        }
        // @probe:computed
        __syncthreads();
        // @probe:synced
        const bool abort_now = s_abort != 0;  // read with the partials
        if (owner) {
            const int pb = t & 1, wr_ = wave;
            // every partial requested before the first add
            float pq[3][NQ];
#pragma unroll
            for (int g = 0; g < 3; ++g)
#pragma unroll
                for (int q = 0; q < NQ; ++q) pq[g][q] = part[pb][q][g][wr_][lane];
            __builtin_amdgcn_sched_barrier(0);
            auto tree4 = [&](int g) {
                if constexpr (NQ == 8)
                    return rec::tree8([&](int q) { return pq[g][q]; });
                else
                    return (pq[g][0] + pq[g][1]) + (pq[g][2] + pq[g][3]);
            };
            const float sr = bias_r + tree4(0);
            const float sz = bias_z + tree4(1);
            const float sn = bias_n + tree4(2);
            const float r = rec::sigmoid_f(cur[0] + sr);
            const float z = rec::sigmoid_f(cur[1] + sz);
            const float n = rec::tanh_f(cur[2] + r * sn);
            const float h = n + z * (h_prev - n);
            if constexpr (NR > 0) {
                // the offset made opaque here, so the 64-bit address is
                // formed per step instead of one per step parity being kept
                // across the loop (at four rows and four slices that pair no
                // longer fits the 256 VGPRs)
                unsigned off = pub_off[t & 1];
                asm volatile("" : "+v"(off));
                rec::publish_word(exch + off, rec::pack_word(h, p.tag_base + (unsigned)(t + 1)), xlocal);
            }
            o_h = h;
            o_r = r;
            o_z = z;
            o_n = n;
            o_a = sn;
            h_prev = h;
            if constexpr (IO) {
                io_out[t & 1][0][lane] = h;
                io_out[t & 1][1][lane] = r;
                io_out[t & 1][2][lane] = z;
                io_out[t & 1][3][lane] = n;
                io_out[t & 1][4][lane] = sn;
            }
        }
        if (wave < R) hloc[t & 1][wave][lane] = owner ? h_prev : 0.f;  // zero past H and B
        __syncthreads();
        // @probe:released
        // the own slot of step t+1 while the other slices' words travel,
        // with the first poll reads of step t+1 already in flight
        if (KF == 3 || t + 1 < T) {
            if constexpr (NR > 0) {
                const unsigned long long* src = exch + (size_t)(t & 1) * B * H + pidx;
#pragma unroll
                for (int r = 0; r < R; ++r) first_read[r] = rec::load_word(src + roff[r]);
            }
            local_fmas(t & 1);
        }
        // @probe:step_end
        return !abort_now;
    };
    // step t stores the outputs of step t - 1: after a step that aborts,
    // rows t_stop .. T-1 were not stored
    int t_stop = T;
    using First = std::integral_constant<int, 1>;
    using Bulk = std::integral_constant<int, 3>;
    using Any = std::integral_constant<int, 0>;
    if (T > 0 && !step(First{}, 0, gxs[0], gxs[1])) {
        t_stop = 0;
    } else {
        int t = 1;
        for (; t + 2 < T; t += 2) {
            if (!step(Bulk{}, t, gxs[1], gxs[0])) {
                t_stop = t;
                break;
            }
            if (!step(Bulk{}, t + 1, gxs[0], gxs[1])) {
                t_stop = t + 1;
                break;
            }
        }
        if (t_stop == T) {
            for (; t < T; t += 2) {
                if (!step(Any{}, t, gxs[1], gxs[0])) {
                    t_stop = t;
                    break;
                }
                if (t + 1 < T && !step(Any{}, t + 1, gxs[0], gxs[1])) {
                    t_stop = t + 1;
                    break;
                }
            }
        }
    }
    // @probe:kernel_end
    const bool aborted = t_stop < T;
    if (owner) {
        if constexpr (!IO) {
            if (!aborted) {
                store_outputs(T - 1);
            } else {
                o_h = o_r = o_z = o_n = o_a = __builtin_nanf("");
                for (int t = t_stop; t < T; ++t) store_outputs(t);
            }
        }
        hn[(unsigned)(orow * H + u)] = aborted ? __builtin_nanf("") : h_prev;  // B H < 2^31
    }
}

// ------------------------------------------------- forward, four rows ---
// Forward recurrence with four batch rows per workgroup on the matrix cores
// (v_mfma_f32_4x4x1_16b_f32).  With four rows the W_hh product of a step is
// a [64 units x 3 gates] x k x [4 rows] block per workgroup, and the 4x4x1
// MFMA fills all of it: block b of the sixteen takes units 4 b .. 4 b + 3, its
// four columns the four rows, so one instruction is 64 units x 4 rows of one
// k and gate (256 multiply-adds).  Measured on MI355X it issues one per 4.1 ns
// per SIMD in this loop shape (two wavefronts per SIMD, three accumulators),
// against 1.4-1.8 ns per 64-lane v_fmac_f32, i.e. 1.4x the rate of the VALU
// FMAs, which bound the four-row step (a wavefront issuing MFMAs and one
// issuing VALU FMAs on the same SIMD do not overlap).
// Lane l of every wavefront is unit 64 s + l (MFMA A row l % 4 of block l / 4)
// and holds, for each slot j (slot 0 = the workgroup's own slice, then the
// others in rotation), the three gates' W_hh at the eight k =
// 64 ((s + j) mod S) + 8 w + c, c < 8 (24 S VGPRs).  The B operand of k is
// h_{t-1}[row l % 4][k] in lane l, read from LDS four k at a time.  A
// wavefront's D registers hold its k's share of the gate sums, D[g] reg r of
// lane l being unit 4 (l / 4) + r of row l % 4; the eight shares meet in LDS
// and the owner of row r (wavefront r) adds them in a fixed tree.  The
// exchange, its words and tags, the owners' gate math, outputs and failure
// handling are those of gru_fwd_local_kernel with four rows.
template <int S, bool FULL = false>
__global__ __launch_bounds__(NTH) void gru_fwd_mfma4_kernel(
    const float* __restrict__ gx, const float* __restrict__ h0, const float* __restrict__ w_hh,
    const float* __restrict__ b_hh, float* __restrict__ y, float* __restrict__ hn,
    float* __restrict__ reserve, unsigned long long* __restrict__ exch, int* __restrict__ abort_flag,
    RegParams p) {
    constexpr int R = 4;
    constexpr int NR = S - 1;        // remote slots
    constexpr int WE = 32 * NR;      // polled words per wavefront: (slot, c, row)
    constexpr int NPR = WE > 64 ? 2 : 1;  // poll registers per lane
    typedef float f4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) float part[2][NW][3][R][64];  // [parity][wave][gate][row][unit]
    __shared__ __attribute__((aligned(16))) float hloc[2][R][64];          // [parity][row][unit]
    __shared__ __attribute__((aligned(16))) float hrem[NW][NR > 0 ? NR : 1][R][8];  // per wave: [slot][row][c]
    __shared__ int s_abort;
    __shared__ int s_local;

    const int B = p.B, T = p.T, H = FULL ? 64 * S : p.H;  // FULL: whole slices, H a constant
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const rec::GroupCoords gc = rec::group_coords(p.S);
    if (gc.g >= p.G) return;  // padding workgroup of a grid rounded up to whole XCDs
    const int s = gc.s;
    const int row0 = gc.g * R;
    const int u = s * 64 + lane;  // this lane's unit (A row, owner unit)
    const bool uvalid = FULL || u < H;
    const int lrow = lane & 3;    // this lane's B column / D column: row lrow
    auto kof = [&](int j, int c) { return 64 * ((s + j) % S) + 8 * wave + c; };

    // A operands: wa[g][8 j + c] = W_hh[g H + u][kof(j, c)] (0 past H)
    float wa[3][8 * S];
#pragma unroll
    for (int j = 0; j < S; ++j)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int k = kof(j, c);
            const bool ok = uvalid && k < H;
#pragma unroll
            for (int g = 0; g < 3; ++g) wa[g][8 * j + c] = ok ? w_hh[((size_t)g * H + u) * H + k] : 0.f;
        }

    // wave r < R owns row row0 + r: its gate math, outputs and exchange words
    const int orow = row0 + (wave < R ? wave : 0);
    const bool owner = wave < R && uvalid && orow < B;
    float h_prev = 0.f, bias_r = 0.f, bias_z = 0.f, bias_n = 0.f;
    float gxs[2][3];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int c = 0; c < 3; ++c) gxs[e][c] = 0.f;
    const float* gx_row = gx + (size_t)orow * T * 3 * H + u;
    auto load_gx = [&](float (&d)[3], int t) {
        const float* gp = gx_row + (size_t)t * 3 * H;
        d[0] = gp[0];
        d[1] = gp[H];
        d[2] = gp[2 * H];
    };
    if (owner) {
        h_prev = h0[(size_t)orow * H + u];
        bias_r = b_hh[u];
        bias_z = b_hh[H + u];
        bias_n = b_hh[2 * H + u];
        load_gx(gxs[0], 0);
    }
    if (threadIdx.x == 0) s_abort = 0;
    const rec::WaitCtl wc{abort_flag, p.abort_count, p.spin_limit};
    const bool xlocal = rec::group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, wc, &s_local);

    // Polled word e of the wavefront: remote slot 1 + e / 32, c = (e / 4) % 8,
    // row e % 4; lane l polls e = l and (S = 4) e = 64 + l.  A word whose k is
    // past H re-reads the wavefront's first valid word (word 0 when none); a
    // row past B reads the group's first row.
    bool rvalid[R];
    unsigned roff[R];  // word offset of row r within a slot (B H < 2^29)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rvalid[r] = row0 + r < B;
        roff[r] = (unsigned)(rvalid[r] ? row0 + r : row0) * (unsigned)H;
    }
    int fallback = -1;
#pragma unroll
    for (int e = 0; e < WE; e += 4) {
        const int k = kof(1 + e / 32, (e / 4) % 8);
        if (fallback < 0 && k < H) fallback = k;
    }
    if (fallback < 0) fallback = 0;
    unsigned poff[NPR];
    bool pval[NPR];
#pragma unroll
    for (int v = 0; v < NPR; ++v) {
        const int e = 64 * v + lane;
        const bool in = e < WE;
        const int k = in ? kof(1 + e / 32, (e / 4) % 8) : H;
        const int r = e & 3;
        pval[v] = in && k < H && rvalid[r];
        poff[v] = (pval[v] ? roff[r] : roff[0]) + (unsigned)(k < H ? k : fallback);
    }

    const int pub_flip = (int)blockIdx.x == p.stall_block ? 1 : 0;
    const unsigned slot_words = (unsigned)B * (unsigned)H, my_word = (unsigned)orow * (unsigned)H + (unsigned)u;
    const unsigned pub_off[2] = {(unsigned)pub_flip * slot_words + my_word,
                                 (unsigned)(1 - pub_flip) * slot_words + my_word};
    float o_h = 0.f, o_r = 0.f, o_z = 0.f, o_n = 0.f, o_a = 0.f;
    float* y_row = y + (size_t)orow * T * H + u;
    float* res_row = reserve ? reserve + (size_t)orow * T * 4 * H + 4 * u : nullptr;
    auto store_outputs = [&](int t) {
        y_row[(size_t)t * H] = o_h;
        if (res_row) *reinterpret_cast<float4*>(res_row + (size_t)t * 4 * H) = make_float4(o_r, o_z, o_n, o_a);
    };

    f4 acc[3];
    auto zero_acc = [&]() {
#pragma unroll
        for (int g = 0; g < 3; ++g) acc[g] = f4{0.f, 0.f, 0.f, 0.f};
    };
    // slot j's eight k with the B operands hb[c] = h[row lrow][kof(j, c)]
    auto mfma8 = [&](const float (&hb)[8], int j) {
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int g = 0; g < 3; ++g)
                acc[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(wa[g][8 * j + c], hb[c], acc[g], 0, 0, 0);
    };
    auto lds8 = [](const float* src, float (&hv)[8]) {
        const float4 a = *reinterpret_cast<const float4*>(src);
        const float4 b = *reinterpret_cast<const float4*>(src + 4);
        hv[0] = a.x; hv[1] = a.y; hv[2] = a.z; hv[3] = a.w;
        hv[4] = b.x; hv[5] = b.y; hv[6] = b.z; hv[7] = b.w;
    };
    // own slot of the next step from the owners' h in LDS
    auto local_mfmas = [&](int par) {
        zero_acc();
        float hb[8];
        lds8(&hloc[par][lrow][8 * wave], hb);
        mfma8(hb, 0);
    };
    unsigned long long first_read[NPR];
#pragma unroll
    for (int v = 0; v < NPR; ++v) first_read[v] = 0;
    // step 0's own slot from h0
    {
        zero_acc();
        float hb[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int k = kof(0, c);
            hb[c] = k < H && rvalid[lrow] ? h0[roff[lrow] + k] : 0.f;
        }
        mfma8(hb, 0);
    }

    auto step = [&](int t, const float (&cur)[3], float (&nxt)[3]) -> bool {
        // @probe:step_begin
        if constexpr (NR > 0) {
            float hx[NPR];
            if (t == 0) {
#pragma unroll
                for (int v = 0; v < NPR; ++v) {
                    const int e = 64 * v + lane;
                    hx[v] = pval[v] ? h0[poff[v] - roff[e & 3] + (unsigned)(row0 + (e & 3)) * (unsigned)H] : 0.f;
                }
            } else {
                const unsigned long long* src = exch + (size_t)((t - 1) & 1) * B * H;
                const unsigned long long* pp[NPR];
#pragma unroll
                for (int v = 0; v < NPR; ++v) pp[v] = src + poff[v];
                bool ok = true;
                rec::wait_words<NPR, true>(pp, pval, first_read, p.tag_base + (unsigned)t, wc, ok);
#pragma unroll
                for (int v = 0; v < NPR; ++v) hx[v] = pval[v] ? __uint_as_float((unsigned)first_read[v]) : 0.f;
                if (!ok) s_abort = 1;
            }
            // word e to hrem[wave][slot e / 32][row e % 4][c (e / 4) % 8]
#pragma unroll
            for (int v = 0; v < NPR; ++v) {
                const int e = 64 * v + lane;
                if (e < WE) hrem[wave][e / 32][e & 3][(e / 4) & 7] = hx[v];
            }
            __builtin_amdgcn_wave_barrier();
        }
        if (owner) {
            if (t > 0) store_outputs(t - 1);
            if (t + 1 < T) load_gx(nxt, t + 1);
        }
        // @probe:polled
#pragma unroll
        for (int jj = 0; jj < NR; ++jj) {
            float hb[8];
            lds8(&hrem[wave][jj][lrow][0], hb);
            mfma8(hb, jj + 1);
        }
        // this wavefront's shares: D[g] reg r of lane l = unit 4 (l / 4) + r, row l % 4
#pragma unroll
        for (int g = 0; g < 3; ++g)
            *reinterpret_cast<float4*>(&part[t & 1][wave][g][lrow][4 * (lane >> 2)]) =
                make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
        // @probe:computed
        __syncthreads();
        // @probe:synced
        const bool abort_now = s_abort != 0;
        if (owner) {
            const int pb = t & 1, rr = wave;
            auto sum8 = [&](int g) { return rec::tree8([&](int w2) { return part[pb][w2][g][rr][lane]; }); };
            const float sr = bias_r + sum8(0);
            const float sz = bias_z + sum8(1);
            const float sn = bias_n + sum8(2);
            const float r = rec::sigmoid_f(cur[0] + sr);
            const float z = rec::sigmoid_f(cur[1] + sz);
            const float n = rec::tanh_f(cur[2] + r * sn);
            const float h = n + z * (h_prev - n);
            if constexpr (NR > 0) {
                unsigned off = pub_off[t & 1];
                asm volatile("" : "+v"(off));
                rec::publish_word(exch + off, rec::pack_word(h, p.tag_base + (unsigned)(t + 1)), xlocal);
            }
            o_h = h;
            o_r = r;
            o_z = z;
            o_n = n;
            o_a = sn;
            h_prev = h;
        }
        if (wave < R) hloc[t & 1][wave][lane] = owner ? h_prev : 0.f;  // zero past H and B
        __syncthreads();
        // @probe:released
        if (t + 1 < T) {
            if constexpr (NR > 0) {
                const unsigned long long* src = exch + (size_t)(t & 1) * B * H;
#pragma unroll
                for (int v = 0; v < NPR; ++v) first_read[v] = rec::load_word(src + poff[v]);
            }
            local_mfmas(t & 1);
        }
        // @probe:step_end
        return !abort_now;
    };
    int t_stop = T;
    for (int t = 0; t < T; t += 2) {
        if (!step(t, gxs[0], gxs[1])) {
            t_stop = t;
            break;
        }
        if (t + 1 < T && !step(t + 1, gxs[1], gxs[0])) {
            t_stop = t + 1;
            break;
        }
    }
    // @probe:kernel_end
    const bool aborted = t_stop < T;
    if (owner) {
        if (!aborted) {
            store_outputs(T - 1);
        } else {
            o_h = o_r = o_z = o_n = o_a = __builtin_nanf("");
            for (int t = t_stop; t < T; ++t) store_outputs(t);
        }
        hn[(unsigned)(orow * H + u)] = aborted ? __builtin_nanf("") : h_prev;
    }
}

// ------------------------------------------------------------ backward ---
// Transposed sum over the four 16-lane rows: given t[v] (v = 0..3) in every
// row, returns in row r the sum of t[r] over the rows, (R0 + R2) + (R1 + R3).
// v_permlane32_swap(x, y) -> (x.R0 x.R1 y.R0 y.R1), (x.R2 x.R3 y.R2 y.R3);
// v_permlane16_swap(x, y) -> (x.R0 y.R0 x.R2 y.R2), (x.R1 y.R1 x.R3 y.R3).
__device__ __forceinline__ float rows_transpose_sum(const float (&t)[4]) {
    auto sw32 = [](float x, float y) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
        return __uint_as_float(p[0]) + __uint_as_float(p[1]);
    };
    const float s02 = sw32(t[0], t[2]);  // rows 0,1: t0 pairs; rows 2,3: t2 pairs
    const float s13 = sw32(t[1], t[3]);
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(s02), __float_as_uint(s13), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Backward recurrence, S = ceil(H / 64) slices and R batch rows per
// workgroup (every wavefront runs the FMAs of all R rows; wavefront r < R
// owns row r), with the workgroup's own G_h words taken from LDS.  The
// description below is for one row.
// The 3H G_h words of a step are split into the workgroup's own 192 (gate
// c, unit m of its slice at index e = 64 c + m) and 192 (S - 1) remote ones
// (flat index r: slot 1 + r / 192 of the other slices in rotation, then e).
// The workgroup's 32 sixteen-lane rows are j-groups: row J = 4 w + rho of
// wave w takes own entries 6 J .. 6 J + 5 and remote entries RE J ..
// RE J + RE - 1 (RE = 6 (S - 1)), and
// lane q of the row takes units 64 s + 4 q .. 4 q + 3, so every G value
// feeds four FMAs of a lane.  The G values reach the FMAs as VGPRs uniform
// over a row (ds_read_b128 from LDS, one address per row): plain v_fmac_f32
// issues at ~1.2 ns per SIMD with two waves per SIMD on MI355X against
// ~2.0 ns for the row-broadcast DPP form, and with four FMAs per value the
// broadcast reads (1 KB per instruction) stay within LDS bandwidth.  The
// four rows' partials of a lane's four units are summed by a transposing
// reduction (three permlane swaps leave unit 4 q + r's total in row r;
// summing each unit in every row took eight and cost ~45 ns more per step),
// then across the 8 waves in LDS.  At the end of a step the owner reduces dh,
// runs the next step's pointwise math, publishes its G words and writes
// them to LDS; after a second barrier every wave runs the own entries' FMAs
// while the other slices' words travel.
//
// The owner keeps its per-step G stores: the ninth-wavefront form of the
// forward, with the own entries' weights in LDS to fit 168 VGPRs, measured
// 0.50-0.51 vs 0.48 ms per c2 launch.
//
// PH = 2 (four rows): each step runs as two phases of two rows, so that one
// half's exchange travels while the other half computes (c4 backward 2.32
// vs 2.37 us per step; the step is bound by the VALU work of four rows, not
// by the exchange).
//
// NWB wavefronts (8, or 16 for one row: 64 j-groups of 3 own and 3 (S - 1)
// remote entries, one poll register per lane, 122 VGPRs at S = 4).  The
// remote FMAs are bound by the SIMD's VALU issue rate (running them twice
// per step added 144 FMA instructions per SIMD and ~139 ns), so sixteen
// wavefronts issue the same instructions per SIMD; measured at c2 (same
// box, three pairs) the one-row backward took 444.2-447.0 vs 447.5-448.4
// us per launch and the step 1.355-1.358 vs 1.361-1.364 ms.
template <int S, int R, int NWB = NW, int PH = 1, bool FULL = false>
__global__ __launch_bounds__(64 * NWB) void gru_bwd_local_kernel(
    const float* __restrict__ dy, const float* __restrict__ dhn, const float* __restrict__ reserve,
    const float* __restrict__ h0, const float* __restrict__ y, const float* __restrict__ w_hh,
    float* __restrict__ gout, float* __restrict__ dh0, unsigned long long* __restrict__ exch,
    int* __restrict__ abort_flag, RegParams p) {
    static_assert(R == 1 || R == 2 || R == 4, "rows per workgroup");
    static_assert(NWB == 8 || NWB == 16, "wavefronts per workgroup");
    static_assert(PH == 1 || (PH == 2 && R % 2 == 0), "phases per step");
    constexpr int RP = R / PH;                       // rows per phase
    constexpr int NJ = 4 * NWB;                      // j-groups (sixteen-lane rows)
    constexpr int OWN = 192 / NJ;                    // own entries per j-group (6 or 3)
    constexpr int RE = OWN * (S - 1);                // remote entries per j-group
    constexpr int WE = 4 * RE;                       // remote entries polled per wave and row
    constexpr int GR = RE > 0 ? (RE + 3) / 4 * 4 : 4;  // LDS row of a j-group's polled words
    constexpr int NW2 = WE > 64 ? 2 : 1;             // poll registers per row
    __shared__ __attribute__((aligned(16))) float part[2][NWB][R][64];
    __shared__ __attribute__((aligned(16))) float gloc[R][NJ][OWN > 4 ? 8 : 4];  // own G words by j-group
    // per wave and row: polled words by j-group (j-group rho's GR at rho GR),
    // then 64 entries that lanes without a word write in the two-phase form
    // instead of branching (c4 backward 4.47 -> 4.36 ms per step; the
    // one-phase form keeps its branch, which measured no slower)
    __shared__ __attribute__((aligned(16))) float grem[NWB][R][4 * GR + 64];
    __shared__ int s_abort;
    __shared__ int s_abort2[2];  // two phases per step: by step parity
    __shared__ int s_local;

    // FULL: H = 64 S, a compile-time constant, and every lane's unit exists
    const int B = p.B, T = p.T, H = FULL ? 64 * S : p.H;
    const int H3 = 3 * H;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
    const rec::GroupCoords gc = rec::group_coords(p.S);
    if (gc.g >= p.G) return;  // padding workgroup of a grid rounded up to whole XCDs
    const int row0 = gc.g * R;  // the group's first batch row
    const int s = gc.s;
    const int u = s * 64 + lane;  // the owner lane's unit
    const bool uvalid = FULL || u < H;
    const int i0 = T - p.t_end, i1 = T - p.t_begin;  // steps i0 .. i1-1 (t = T-1-i)

    const int rho = lane >> 4, q = lane & 15;
    const int J = 4 * wave + rho;
    const int ub = s * 64 + 4 * q;  // the lane's first FMA unit
    // W_hh row of own entry e / remote entry r; valid = the unit exists
    auto own_row = [&](int e, bool& valid) {
        const int m = e & 63;
        valid = 64 * s + m < H;
        return (e >> 6) * H + 64 * s + m;
    };
    auto rem_row = [&](int r, bool& valid) {
        const int e = r % 192, m = e & 63, sl = (s + 1 + r / 192) % S;
        valid = 64 * sl + m < H;
        return (e >> 6) * H + 64 * sl + m;
    };

    // W_hh[j][ub .. ub + 3] for the j-group's own (wl) and remote (wm) entries
    float wl[OWN][4], wm[RE > 0 ? RE : 1][4];
    const bool vec = p.wvec != 0;
    auto load4 = [&](int jr, bool ok, float (&d)[4]) {
        const float* src = w_hh + (size_t)jr * H + ub;
        if (vec) {
            const float4 v = (ok && ub < H) ? *reinterpret_cast<const float4*>(src) : make_float4(0.f, 0.f, 0.f, 0.f);
            d[0] = v.x;
            d[1] = v.y;
            d[2] = v.z;
            d[3] = v.w;
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) d[v] = (ok && ub + v < H) ? src[v] : 0.f;
        }
    };
#pragma unroll
    for (int i = 0; i < OWN; ++i) {
        bool ok;
        const int jr = own_row(OWN * J + i, ok);
        load4(jr, ok, wl[i]);
    }
#pragma unroll
    for (int i = 0; i < RE; ++i) {
        bool ok;
        const int jr = rem_row(RE * J + i, ok);
        load4(jr, ok, wm[i]);
    }

    // wave r < R owns row row0 + r: its pointwise math, G stores and words
    const int orow = row0 + (wave < R ? wave : 0);
    // the owner lane's first word in the slot of each step parity (32-bit
    // unsigned offsets, 6 B H < 2^32: the host keeps B H < 2^29); the
    // failure injection swaps the two
    const int pub_flip = (int)blockIdx.x == p.stall_block ? 1 : 0;
    const unsigned slot_words = (unsigned)B * (unsigned)H3, my_word = (unsigned)orow * (unsigned)H3 + (unsigned)u;
    const unsigned pub_off[2] = {(unsigned)pub_flip * slot_words + my_word,
                                 (unsigned)(1 - pub_flip) * slot_words + my_word};
    const bool owner = wave < R && uvalid && orow < B;
    float dh = 0.f, ddirect = 0.f;
    float o_dan = 0.f, o_drh = 0.f, o_dzh = 0.f, o_dnh = 0.f;
    float ins[2][6];
    // The owner row's bases are wave-uniform (scalar) and fixed; a step adds
    // t H, a 32-bit product (B T H < 2^29, checked on the host), so the step
    // loop carries no 64-bit multiplies.
    const size_t row_el = (size_t)orow * T * H;
    const float* dy_r = dy ? dy + row_el : nullptr;
    const float* res_r = reserve + 4 * row_el;
    const float* y_r = y + row_el;
    const float* h0_r = h0 + (size_t)orow * H;
    float* g_r = gout + 4 * row_el;
    auto load_inputs = [&](float (&d)[6], int t) {
        const unsigned tH = (unsigned)t * (unsigned)H;
        d[0] = dy_r ? dy_r[tH + u] : 0.f;
        // the unit's (r, z, n, a_n) as one float4 (reserve [B, T, H, 4])
        const float4 c4 = *reinterpret_cast<const float4*>(res_r + 4 * (tH + u));
        d[1] = c4.x;
        d[2] = c4.y;
        d[3] = c4.z;
        d[4] = c4.w;
        d[5] = t > 0 ? y_r[tH - H + u] : h0_r[u];
    };
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int c = 0; c < 6; ++c) ins[e][c] = 0.f;
    if (owner) {
        if (dhn) dh = dhn[(size_t)orow * H + u];
        load_inputs(ins[0], T - 1 - i0);
        if (i0 + 1 < i1) load_inputs(ins[1], T - 2 - i0);
    }
    if (threadIdx.x == 0) {
        s_abort = 0;
        s_abort2[0] = s_abort2[1] = 0;
    }
    const rec::WaitCtl wc{abort_flag, p.abort_count, p.spin_limit};
    const bool xlocal = rec::group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, wc, &s_local);

    // Wave w polls remote entries WE w .. WE w + WE - 1 of every row:
    // register 0 lane l entry WE w + l (l < WE), register 1 (S = 4: WE = 72)
    // lane l entry WE w + 64 + l % 8.  Lanes without a word re-read the
    // register's first valid word (else the wave's first valid remote word,
    // else word 0); a row past B reads the group's first row.
    int first_any = -1, first1 = -1;
#pragma unroll
    for (int e = 0; e < WE; ++e) {
        bool ok;
        const int jr = rem_row(WE * wave + e, ok);
        if (ok && first_any < 0) first_any = jr;
        if (ok && e >= 64 && first1 < 0) first1 = jr;
    }
    if (first_any < 0) first_any = 0;
    if (first1 < 0) first1 = first_any;
    bool pv0 = false, pv1 = false;
    int pidx0 = lane < WE ? rem_row(WE * wave + lane, pv0) : 0;
    int pidx1 = WE > 64 ? rem_row(WE * wave + 64 + (lane & 7), pv1) : 0;
    if (!pv0) pidx0 = first_any;
    if (!pv1) pidx1 = first1;
    // where a lane writes its polled words in grem (entry e to j-group e / RE,
    // position e % RE)
    constexpr int RE1 = RE > 0 ? RE : 1;
    const int gslot0 = lane < WE ? (lane / RE1) * GR + lane % RE1 : 4 * GR + lane;
    const int gslot1 = lane < WE - 64 ? ((64 + lane) / RE1) * GR + (64 + lane) % RE1 : 4 * GR + lane;
    bool rvalid[R];
    int roff[R];  // word offset of row r within a slot (3 B H < 2^31)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rvalid[r] = row0 + r < B;
        roff[r] = (rvalid[r] ? row0 + r : row0) * H3;
    }

    // pointwise step i (t = T-1-i) from dh and its inputs: publishes G_h,t,
    // writes it to LDS by j-group, keeps the gate gradients for the store
    // after the next poll
    // tsum: this step's W_hh^T G_h sum (dh_t = ddirect + tsum).  The factors
    // that depend only on the saved activations are formed first, so the
    // chain from the sum to the published words is one add and two
    // multiplications.
    auto pointwise = [&](int i, const float (&cur)[6], bool act, float tsum) {
        if (act && owner) {
            const float cr = cur[1], cz = cur[2], cn = cur[3], ca = cur[4], hp = cur[5];
            const float f_n = (1.0f - cz) * (1.0f - cn * cn);      // dn^ / g
            const float f_r = ca * (cr * (1.0f - cr));             // dr^ / dn^
            const float f_z = (hp - cn) * (cz * (1.0f - cz));      // dz^ / g
            const float gsum = (ddirect + cur[0]) + tsum;          // g = dh_t + dy_t
            o_dnh = gsum * f_n;
            o_dan = o_dnh * cr;
            o_drh = o_dnh * f_r;
            o_dzh = gsum * f_z;
            ddirect = gsum * cz;
            if constexpr (RE > 0) {
                const unsigned tag = (unsigned)(i + 1);
                unsigned long long* wp = exch + pub_off[i & 1];
                unsigned long long* const pp3[3] = {wp, wp + H, wp + 2 * H};
                const unsigned long long w3[3] = {rec::pack_word(o_drh, tag), rec::pack_word(o_dzh, tag),
                                                  rec::pack_word(o_dan, tag)};
                rec::publish_words<3>(pp3, w3, xlocal);
            }
        }
        if (act && wave < R) {
            const float gv[3] = {owner ? o_drh : 0.f, owner ? o_dzh : 0.f, owner ? o_dan : 0.f};
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const int e = 64 * c + lane;
                gloc[wave][e / OWN][e % OWN] = gv[c];
            }
        }
    };
    float acc[R][2][4];
    // FMAs of row r's n values g[0 .. n-1] of the j-group with the weights wt
    auto fma_group = [&](int r, const float* g, int n, const float (*wt)[4]) {
#pragma unroll
        for (int i = 0; i < n; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[r][i & 1][v] = fmaf(g[i], wt[i][v], acc[r][i & 1][v]);
    };
    auto local_fmas_rows = [&](int ra, int nr) {
#pragma unroll
        for (int r = ra; r < ra + nr; ++r) {
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[r][0][v] = acc[r][1][v] = 0.f;
            const float4 a = *reinterpret_cast<const float4*>(&gloc[r][J][0]);
            if constexpr (OWN == 6) {
                const float4 b = *reinterpret_cast<const float4*>(&gloc[r][J][4]);
                const float g[6] = {a.x, a.y, a.z, a.w, b.x, b.y};
                fma_group(r, g, 6, wl);
            } else {
                const float g[3] = {a.x, a.y, a.z};
                fma_group(r, g, 3, wl);
            }
        }
    };
    // the first poll reads of step i, issued ahead of its own-entry FMAs
    unsigned long long first_read[NW2 * R];
#pragma unroll
    for (int v = 0; v < NW2 * R; ++v) first_read[v] = 0;
    auto first_poll_rows = [&](int i, int ra, int nr) {
        const unsigned long long* slotp = exch + (size_t)(i & 1) * B * H3;
#pragma unroll
        for (int r = ra; r < ra + nr; ++r) {
            if constexpr (WE > 0) first_read[NW2 * r] = rec::load_word(slotp + roff[r] + pidx0);
            if constexpr (WE > 64) first_read[NW2 * r + 1] = rec::load_word(slotp + roff[r] + pidx1);
        }
    };
    // a j-group's polled words of row r from LDS
    auto read_grem = [&](int r, float (&g)[GR]) {
#pragma unroll
        for (int k = 0; k < GR / 4; ++k) {
            const float4 v = *reinterpret_cast<const float4*>(&grem[wave][r][GR * rho + 4 * k]);
            g[4 * k] = v.x;
            g[4 * k + 1] = v.y;
            g[4 * k + 2] = v.z;
            g[4 * k + 3] = v.w;
        }
    };
    // one timestep (i-th from the end): its G words are published and its
    // own-entry FMAs done; false when the workgroup must stop
    // kind: 3 = at least two steps follow (the next step, and the input loads
    // two steps ahead, exist), 0 = tested at run time
    auto step = [&](auto kind, int i, float (&cur)[6], const float (&nxt)[6]) -> bool {
        constexpr int KIND = decltype(kind)::value;
        // @probe:step_begin
        const int t = T - 1 - i;
        const unsigned long long* slotp = exch + (size_t)(i & 1) * B * H3;
        float g0[GR];
        if constexpr (WE > 0) {
            const unsigned long long* pp[NW2 * R];
            bool pv[NW2 * R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                pp[NW2 * r] = slotp + roff[r] + pidx0;
                pv[NW2 * r] = pv0 && rvalid[r];
                if constexpr (NW2 == 2) {
                    pp[NW2 * r + 1] = slotp + roff[r] + pidx1;
                    pv[NW2 * r + 1] = pv1 && rvalid[r];
                }
            }
            bool ok = true;
            rec::wait_words<NW2 * R>(pp, pv, first_read, (unsigned)(i + 1), wc, ok);
            if (!ok) s_abort = 1;
            // polled entry e of the wave to row e / RE, position e % RE of its
            // LDS block (one wave writes and reads the blocks; LDS keeps a
            // wave's accesses in order)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float gr0 = pv[NW2 * r] ? __uint_as_float((unsigned)first_read[NW2 * r]) : 0.f;
                if (lane < WE) grem[wave][r][gslot0] = gr0;
                if constexpr (NW2 == 2) {
                    const float gr1 = pv[NW2 * r + 1] ? __uint_as_float((unsigned)first_read[NW2 * r + 1]) : 0.f;
                    if (lane < WE - 64) grem[wave][r][gslot1] = gr1;
                }
            }
            __builtin_amdgcn_wave_barrier();
            read_grem(0, g0);
        }
        if (owner) {
            // streaming stores: G is read once, by the gradient GEMMs after
            // this kernel, so it need not take MALL space from the reserve,
            // y and dy this kernel still has to read (backward 0.449 vs
            // 0.467 ms per c2 launch, same-box A/B)
            float* op = g_r + 4 * (unsigned)t * (unsigned)H;  // wave-uniform
            __builtin_nontemporal_store(o_dan, op + u);
            __builtin_nontemporal_store(o_drh, op + H + u);
            __builtin_nontemporal_store(o_dzh, op + 2 * H + u);
            __builtin_nontemporal_store(o_dnh, op + 3 * H + u);
            if (KIND == 3 || t - 2 >= p.t_begin) load_inputs(cur, t - 2);
        }
        // @probe:polled
        if constexpr (RE > 0) {
            fma_group(0, g0, RE, wm);
#pragma unroll
            for (int r = 1; r < R; ++r) {
                // one row's G values at a time (registers)
                __builtin_amdgcn_sched_barrier(0);
                float g[GR];
                read_grem(r, g);
                fma_group(r, g, RE, wm);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float tot[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) tot[v] = acc[r][0][v] + acc[r][1][v];
            // row rho holds the wave's total for unit 4 q + rho
            part[i & 1][wave][r][4 * q + rho] = rows_transpose_sum(tot);
        }
        // @probe:computed
        __syncthreads();
        // @probe:synced
        const bool abort_now = s_abort != 0;  // read with the partials
        float tsum = 0.f;
        if (owner) {
            // every partial requested before the first add (one LDS latency
            // instead of one per half)
            float pw[NWB];
#pragma unroll
            for (int w2 = 0; w2 < NWB; ++w2) pw[w2] = part[i & 1][w2][wave][lane];
            __builtin_amdgcn_sched_barrier(0);
            const float lo = rec::tree8([&](int w2) { return pw[w2]; });
            if constexpr (NWB == 16)
                tsum = lo + rec::tree8([&](int w2) { return pw[8 + w2]; });
            else
                tsum = lo;
            dh = ddirect + tsum;
        }
        const bool more = KIND == 3 || i + 1 < i1;
        if (more) pointwise(i + 1, nxt, true, tsum);
        // @probe:published
        __syncthreads();
        // @probe:released
        if (more) {
            first_poll_rows(i + 1, 0, R);
            local_fmas_rows(0, R);
        }
        // @probe:step_end
        return !abort_now;
    };
    // Two phases per step (PH = 2): the rows of phase 1 wait for their words,
    // run their FMAs and reach their barrier while the words of phase 0's
    // rows for the next step travel, and the other way round, so each
    // half's exchange is hidden behind the other half's work.  One barrier
    // per phase: it publishes the phase's partial sums to its owners and the
    // other phase's own G words (written by that phase's owners after the
    // previous barrier) to every wavefront.  Phase ra (rows ra .. ra + RP - 1)
    // of step i; the owners are wavefronts ra .. ra + RP - 1.
    auto phase = [&](int i, int ra, float (&cur)[6], const float (&nxt)[6]) -> bool {
        const int t = T - 1 - i;
        const bool mine = wave >= ra && wave < ra + RP;
        // @probe:phase_begin
        first_poll_rows(i, ra, RP);
        local_fmas_rows(ra, RP);
        float g0[GR];
        if constexpr (WE > 0) {
            const unsigned long long* slotp = exch + (size_t)(i & 1) * B * H3;
            const unsigned long long* pp[NW2 * RP];
            bool pv[NW2 * RP];
            unsigned long long fr[NW2 * RP];
#pragma unroll
            for (int k = 0; k < RP; ++k) {
                const int r = ra + k;
                pp[NW2 * k] = slotp + roff[r] + pidx0;
                pv[NW2 * k] = pv0 && rvalid[r];
                fr[NW2 * k] = first_read[NW2 * r];
                if constexpr (NW2 == 2) {
                    pp[NW2 * k + 1] = slotp + roff[r] + pidx1;
                    pv[NW2 * k + 1] = pv1 && rvalid[r];
                    fr[NW2 * k + 1] = first_read[NW2 * r + 1];
                }
            }
            bool ok = true;
            rec::wait_words<NW2 * RP>(pp, pv, fr, (unsigned)(i + 1), wc, ok);
            if (!ok) s_abort2[i & 1] = 1;
#pragma unroll
            for (int k = 0; k < RP; ++k) {
                const int r = ra + k;
                const float gr0 = pv[NW2 * k] ? __uint_as_float((unsigned)fr[NW2 * k]) : 0.f;
                grem[wave][r][gslot0] = gr0;
                if constexpr (NW2 == 2) {
                    const float gr1 = pv[NW2 * k + 1] ? __uint_as_float((unsigned)fr[NW2 * k + 1]) : 0.f;
                    grem[wave][r][gslot1] = gr1;
                }
            }
            __builtin_amdgcn_wave_barrier();
            read_grem(ra, g0);
        }
        // @probe:phase_polled
        if (owner && mine) {
            float* op = g_r + 4 * (unsigned)t * (unsigned)H;  // wave-uniform
            __builtin_nontemporal_store(o_dan, op + u);
            __builtin_nontemporal_store(o_drh, op + H + u);
            __builtin_nontemporal_store(o_dzh, op + 2 * H + u);
            __builtin_nontemporal_store(o_dnh, op + 3 * H + u);
            if (t - 2 >= p.t_begin) load_inputs(cur, t - 2);
        }
        if constexpr (RE > 0) {
            fma_group(ra, g0, RE, wm);
#pragma unroll
            for (int k = 1; k < RP; ++k) {
                __builtin_amdgcn_sched_barrier(0);
                float g[GR];
                read_grem(ra + k, g);
                fma_group(ra + k, g, RE, wm);
            }
        }
#pragma unroll
        for (int k = 0; k < RP; ++k) {
            const int r = ra + k;
            float tot[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) tot[v] = acc[r][0][v] + acc[r][1][v];
            part[i & 1][wave][r][4 * q + rho] = rows_transpose_sum(tot);
        }
        // @probe:phase_computed
        __syncthreads();
        // @probe:phase_synced
        // every wait of step i has set its flag before the barrier of the
        // step's last phase; the next step's waits set the other parity's
        const bool abort_now = ra + RP == R && s_abort2[i & 1] != 0;
        float tsum = 0.f;
        if (owner && mine) {
            tsum = rec::tree8([&](int w2) { return part[i & 1][w2][wave][lane]; });
            dh = ddirect + tsum;
        }
        if (i + 1 < i1) pointwise(i + 1, nxt, mine, tsum);
        // @probe:phase_end
        return !abort_now;
    };
    if (i0 < i1) pointwise(i0, ins[0], true, dh);  // dh_T = dhn (ddirect is 0)
    __syncthreads();
    // step i stores the G row of step i: after a step that aborts, rows
    // i_stop + 1 .. i1 - 1 were not stored
    int i_stop = i1;
    if constexpr (PH == 1) {
        first_poll_rows(i0, 0, R);
        local_fmas_rows(0, R);
        using Bulk = std::integral_constant<int, 3>;
        using Any = std::integral_constant<int, 0>;
        // Steps followed by at least two more run without the run-time tests
        // of the next step and of the loads two steps ahead (the last steps
        // keep them).  Measured on MI355X (same box, three alternating
        // pairs): c5 backward 3326-3330 -> 3252-3255 us per launch, H = 128
        // 346-347 -> 338-340 us; the whole-slice instances at three and four
        // slices (built with max-ilp) measured slower with it (c2 +5 us) and
        // keep the single loop.
        constexpr bool kBulk = !(FULL && S >= 3);
        int i = i0;
        if constexpr (kBulk) {
            // steps i and i + 1 both followed by two more
            for (; i + 3 < i1; i += 2) {
                if (!step(Bulk{}, i, ins[0], ins[1])) {
                    i_stop = i;
                    break;
                }
                if (!step(Bulk{}, i + 1, ins[1], ins[0])) {
                    i_stop = i + 1;
                    break;
                }
            }
        }
        if (i_stop == i1) {
            for (; i < i1; i += 2) {
                if (!step(Any{}, i, ins[0], ins[1])) {
                    i_stop = i;
                    break;
                }
                if (i + 1 < i1 && !step(Any{}, i + 1, ins[1], ins[0])) {
                    i_stop = i + 1;
                    break;
                }
            }
        }
    } else {
        static_assert(NWB == 8, "two phases with eight wavefronts");
        for (int i = i0; i < i1; i += 2) {
            phase(i, 0, ins[0], ins[1]);
            if (!phase(i, RP, ins[0], ins[1])) {
                i_stop = i;
                break;
            }
            if (i + 1 < i1) {
                phase(i + 1, 0, ins[1], ins[0]);
                if (!phase(i + 1, RP, ins[1], ins[0])) {
                    i_stop = i + 1;
                    break;
                }
            }
        }
    }
    // @probe:kernel_end
    const bool aborted = i_stop < i1;
    if (owner) {
        if (aborted) {
            const float nan = __builtin_nanf("");
            for (int i = i_stop + 1; i < i1; ++i) {
                float* op = gout + ((size_t)orow * T + (T - 1 - i)) * 4 * H;
                op[u] = nan;
                op[H + u] = nan;
                op[2 * H + u] = nan;
                op[3 * H + u] = nan;
            }
        }
        dh0[(size_t)orow * H + u] = aborted ? __builtin_nanf("") : dh;
    }
}
}  // namespace

// The one-row backward's whole-slice instances (gru_bwd_local_kernel<S, 1, 16,
// 1, true>, H = 64 S) for `slices` S = 3 or 4; they are compiled in a
// translation unit of their own (gru_rec_bwd1.hip), built with its own
// machine-scheduler strategy.
const void* rec_bwd1_kernel(int slices);
// The one-row forward at four whole slices (gru_fwd_local_kernel<4, 1, false,
// 16, true>, H = 256), likewise (gru_rec_fwd1.hip).
const void* rec_fwd1_kernel();

}  // namespace rka
