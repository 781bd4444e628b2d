// Register-resident persistent GRU recurrences (hidden size <= 256).
//
// Workgroup (g, s) owns hidden units [64 s, 64 s + 64) of batch rows
// [ROWS g, ROWS g + ROWS); lane l of every wavefront is unit 64 s + l.  The
// W_hh entries the workgroup needs live in VGPRs for the whole sequence:
//   forward : wavefront w holds, per lane, the k-chunk [w*chunk, (w+1)*chunk)
//             of the three rows (r, z, n) of its unit (3*chunk registers);
//   backward: wavefront w holds, per lane, the j-chunk of its unit's column
//             of W_hh over the 3H gate rows (chunk registers).
// Each step a wavefront polls only the exchanged words of its own chunk
// (h_{t-1} forward, G_h,t backward; one word per lane per 64), turns them
// into groups of 16 values replicated in the four 16-lane rows
// (v_permlane16/32_swap) and runs the chunk's FMAs with the broadcast folded
// into each FMA (DPP row_newbcast), without LDS or readlane; the 8 wavefront
// partials are reduced in LDS (one barrier per step) and wavefront r applies
// the gate math of row r.  With 64 units per workgroup a hidden size of 256
// needs 4 exchanging workgroups per batch row, which sit on one XCD.
//
// At one batch row per workgroup and four slices (193 <= H <= 256, the
// B = 64, H = 256 shape) the *_local kernels replace these: every wavefront
// holds an equal share of each slice's k (forward) or j (backward) values,
// the owner writes its own slice's new words to LDS as well as publishing
// them, and after a second barrier the wavefronts run the own slice's
// quarter of the FMAs while the other three slices' words are in flight.
// Measured at B=64, H=256, T=512: forward 0.570 -> 0.529 ms, backward
// 0.615 -> 0.567 ms.
//
// Measured on MI355X at B=64, H=256, T=512 (same box, alternating runs):
//   * readlane broadcasts into scalar FMA operands instead of DPP: forward
//     0.726 vs 0.706 ms, backward 1.182 vs 0.934 ms (a readlane costs ~11
//     cycles of issue per wave, a DPP FMA ~5-7, a plain FMA ~5-6);
//   * polling 16-word groups replicated in every row (6 loads per backward
//     wave) instead of one word per lane: backward 1.25 vs 0.95 ms;
//   * exec-masking lanes without a word instead of letting them re-read a
//     word of their own wave: backward 1.04 vs 0.93 ms;
//   * backward owner issuing its G stores and the loads of its next inputs
//     before the poll instead of after it (inputs loaded two steps ahead,
//     single-round polls so that no poll load is left in flight): 0.943 vs
//     0.848 ms; the same reordering in the forward: 0.825 vs 0.782 ms (its
//     stores and loads are few, and it keeps the two-round pipelined poll).
// Alternatives measured slower earlier (kept out):
//   * 128 units per workgroup (2 exchanging workgroups, but twice the FMAs on
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
//   n = tanh(gx_n + r a_n); h_t = n + z (h_{t-1} - n); reserve = (r, z, n, a_n)
// Backward maths (a100_gru_h256_kernels.cu:842-866,915-932), g = dh_t + dy_t:
//   dz = g (h_{t-1} - n), dn^ = g (1 - z)(1 - n^2), dr^ = dn^ a_n r (1 - r),
//   dz^ = dz z (1 - z), da_n = dn^ r; dh_{t-1} = g z + G_h W_hh;
//   g_out[b,t] = (da_n, dr^, dz^, dn^).
#include "rec_common.h"

#include <algorithm>

namespace rka {
namespace {

using rec::NTH;
using rec::NW;

struct RegParams {
    int B, T, H;
    int G, S;      // groups of ROWS rows, slices of 64 units
    int chunk;     // k (forward) or j (backward) values per wavefront
    int wvec;      // forward: W_hh rows may be read as aligned float4
    int t_begin, t_end;  // backward: time range processed
    unsigned long long* xcc_words;  // start-up XCD check (nullable)
    unsigned xcc_tag;
};

// Row-broadcast dot products over one group of 16 values.  A VGPR operand
// of a DPP instruction (the accumulator of v_fmac_f32 is one) written by a
// preceding VALU instruction needs wait states before it is read (the
// compiler pads with s_nop below a distance of about five), so consecutive
// FMAs go to independent partial sums: K parity for the three gates of the
// forward (distance 6), K mod 8 for the backward (distance 8).
//   a?[K & 1][r] += src[r](lane K of the row) * w?[K], K = 0..15
template <int ROWS, int K = 0>
__device__ __forceinline__ void dot16x3(float (&ar)[2][ROWS], float (&az)[2][ROWS], float (&an)[2][ROWS],
                                        const float (&src)[ROWS], const float* wr, const float* wz,
                                        const float* wn) {
    if constexpr (K < 16) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            rec::fma_row_bcast<K>(ar[K & 1][r], src[r], wr[K]);
            rec::fma_row_bcast<K>(az[K & 1][r], src[r], wz[K]);
            rec::fma_row_bcast<K>(an[K & 1][r], src[r], wn[K]);
        }
        dot16x3<ROWS, K + 1>(ar, az, an, src, wr, wz, wn);
    }
}

//   acc[K & 7][r] += src[r](lane K of the row) * w[K], K = 0..15
template <int ROWS, int K = 0>
__device__ __forceinline__ void dot16(float (&acc)[8][ROWS], const float (&src)[ROWS], const float* w) {
    if constexpr (K < 16) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) rec::fma_row_bcast<K>(acc[K & 7][r], src[r], w[K]);
        dot16<ROWS, K + 1>(acc, src, w);
    }
}

// ------------------------------------------------------------- forward ---
template <int NK, int ROWS>
__global__ __launch_bounds__(NTH) void gru_fwd_reg_kernel(
    const float* __restrict__ gx, const float* __restrict__ h0, const float* __restrict__ w_hh,
    const float* __restrict__ b_hh, float* __restrict__ y, float* __restrict__ hn,
    float* __restrict__ reserve, unsigned long long* __restrict__ exch, int* __restrict__ abort_flag,
    RegParams p) {
    __shared__ float part[2][NW][3][ROWS][64];
    __shared__ int s_abort;

    const int B = p.B, T = p.T, H = p.H;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const rec::GroupCoords gc = rec::group_coords(p.G, p.S);
    const int g = gc.g;
    const int s = gc.s;
    const int u = s * 64 + lane;
    const bool uvalid = u < H;
    const int row0 = g * ROWS;
    const int kbeg = wave * p.chunk;

    // k-chunk of the three W_hh rows of unit u
    float wr[NK], wz[NK], wn[NK];
    const bool vec = p.wvec != 0;
#pragma unroll
    for (int k = 0; k < NK; k += 4) {
        const int kk = kbeg + k;
        const float* pr = w_hh + (size_t)u * H + kk;
        const float* pz = pr + (size_t)H * H;
        const float* pn = pz + (size_t)H * H;
        if (vec) {
            const bool ok = uvalid && k < p.chunk && kk < H;
            const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 a = ok ? *reinterpret_cast<const float4*>(pr) : z4;
            const float4 b = ok ? *reinterpret_cast<const float4*>(pz) : z4;
            const float4 c = ok ? *reinterpret_cast<const float4*>(pn) : z4;
            wr[k] = a.x; wr[k + 1] = a.y; wr[k + 2] = a.z; wr[k + 3] = a.w;
            wz[k] = b.x; wz[k + 1] = b.y; wz[k + 2] = b.z; wz[k + 3] = b.w;
            wn[k] = c.x; wn[k + 1] = c.y; wn[k + 2] = c.z; wn[k + 3] = c.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const bool ok = uvalid && k + c < p.chunk && kk + c < H;
                wr[k + c] = ok ? pr[c] : 0.f;
                wz[k + c] = ok ? pz[c] : 0.f;
                wn[k + c] = ok ? pn[c] : 0.f;
            }
        }
    }

    // Owner wavefronts (gate math of row row0 + orow, unit u): the ROWS
    // wavefronts from the first one whose k-chunk lies in this workgroup's
    // own slice, so the owner's poll reads words it published itself.
    const int own0 = min(NW - 1, (64 * s) / p.chunk);
    const int orow = (wave - own0 + NW) % NW;
    const int prow = row0 + orow;
    const bool owner = orow < ROWS && prow < B && uvalid;
    float h_prev = 0.f, bias_r = 0.f, bias_z = 0.f, bias_n = 0.f;
    // gx of step t in set t & 1, loaded one step ahead right after a poll:
    // the vector-memory counter retires in order (stores included), so
    // memory operations issued ahead of a poll would hold up its completion.
    float gxs[2][3];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int c = 0; c < 3; ++c) gxs[e][c] = 0.f;
    const float* gx_row = gx + (size_t)prow * T * 3 * H + u;
    auto load_gx = [&](float (&d)[3], int t) {
        const float* gp = gx_row + (size_t)t * 3 * H;
        d[0] = gp[0];
        d[1] = gp[H];
        d[2] = gp[2 * H];
    };
    if (owner) {
        h_prev = h0[(size_t)prow * H + u];
        bias_r = b_hh[u];
        bias_z = b_hh[H + u];
        bias_n = b_hh[2 * H + u];
        load_gx(gxs[0], 0);
    }
    if (threadIdx.x == 0) s_abort = 0;
    __shared__ int s_local;
    // the group = the S workgroups of rec::group_coords; plain publishing stores when they share an XCD
    const bool xlocal = rec::group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, abort_flag, &s_local);

    // Lane l polls k = kbeg + 64 q + l (NP words per lane); the 16-value
    // groups the row-broadcast FMAs consume are then built in registers.
    constexpr int NV = NK / 16;
    constexpr int NP = (NK + 63) / 64;
    bool kvalid[NP];
    int kidx[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        const int kc = 64 * q + rec::poll_lane<NV>(q, lane);
        kvalid[q] = kc < p.chunk && kbeg + kc < H;
        // invalid lanes re-read the wave's last valid word (or word 0)
        kidx[q] = kvalid[q] ? kbeg + kc : rec::last_valid(kbeg, p.chunk, H);
    }
    // outputs of the previous step, stored after the next poll
    float o_h = 0.f, o_r = 0.f, o_z = 0.f, o_n = 0.f, o_a = 0.f;
    float* y_row = y + (size_t)prow * T * H + u;
    float* res_row = reserve ? reserve + (size_t)prow * T * 4 * H + u : nullptr;
    auto store_outputs = [&](int t) {
        y_row[(size_t)t * H] = o_h;
        if (res_row) {
            float* cp = res_row + (size_t)t * 4 * H;
            cp[0] = o_r;
            cp[H] = o_z;
            cp[2 * H] = o_n;
            cp[3 * H] = o_a;
        }
    };
    // one timestep; gate inputs in cur, next step's loaded into nxt; false
    // when the workgroup must stop
    auto step = [&](int t, const float (&cur)[3], float (&nxt)[3]) -> bool {
        // @probe:step_begin
        // h_{t-1}[row][kbeg + 64 p + lane]
        float hx[NP][ROWS];
        if (t == 0) {
#pragma unroll
            for (int q = 0; q < NP; ++q)
#pragma unroll
                for (int r = 0; r < ROWS; ++r)
                    hx[q][r] = (kvalid[q] && row0 + r < B) ? h0[(size_t)(row0 + r) * H + kidx[q]] : 0.f;
        } else {
            const unsigned long long* src = exch + (size_t)((t - 1) & 1) * B * H;
            constexpr int N = NP * ROWS;
            const unsigned long long* pp[N];
            bool pv[N];
            unsigned long long w[N];
#pragma unroll
            for (int q = 0; q < NP; ++q)
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const int e = q * ROWS + r;
                    pv[e] = kvalid[q] && row0 + r < B;
                    pp[e] = src + (size_t)(row0 + r < B ? row0 + r : row0) * H + kidx[q];
                    w[e] = rec::load_word(pp[e]);
                }
            bool ok = true;
            rec::wait_words<N>(pp, pv, w, (unsigned)t, abort_flag, ok);
#pragma unroll
            for (int q = 0; q < NP; ++q)
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const int e = q * ROWS + r;
                    hx[q][r] = pv[e] ? __uint_as_float((unsigned)w[e]) : 0.f;
                }
            if (!ok) s_abort = 1;
        }
        float hv[NV][ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) rec::replicate_rows<NV>(hx, r, hv);
        // the polled words are consumed before any store or load is issued
        // behind them (a later use would wait for those too)
        if (owner) {
            if (t > 0) store_outputs(t - 1);
            if (t + 1 < T) load_gx(nxt, t + 1);
        }
        // @probe:polled
        float ar[2][ROWS], az[2][ROWS], an[2][ROWS];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int r = 0; r < ROWS; ++r) ar[e][r] = az[e][r] = an[e][r] = 0.f;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
#pragma unroll
            for (int r = 0; r < ROWS; ++r) rec::dpp_src_guard(hv[v][r]);
            dot16x3<ROWS>(ar, az, an, hv[v], wr + 16 * v, wz + 16 * v, wn + 16 * v);
        }
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            part[t & 1][wave][0][r][lane] = ar[0][r] + ar[1][r];
            part[t & 1][wave][1][r][lane] = az[0][r] + az[1][r];
            part[t & 1][wave][2][r][lane] = an[0][r] + an[1][r];
        }
        // @probe:computed
        __syncthreads();
        // @probe:synced
        // read with the partials; the owner's step goes ahead regardless (an
        // aborted launch only ends with NaN final states)
        const bool abort_now = s_abort != 0;
        if (owner) {
            const int pb = t & 1;
            const float sr = bias_r + rec::tree8([&](int w2) { return part[pb][w2][0][orow][lane]; });
            const float sz = bias_z + rec::tree8([&](int w2) { return part[pb][w2][1][orow][lane]; });
            const float sn = bias_n + rec::tree8([&](int w2) { return part[pb][w2][2][orow][lane]; });
            const float r = rec::sigmoid_f(cur[0] + sr);
            const float z = rec::sigmoid_f(cur[1] + sz);
            const float n = rec::tanh_f(cur[2] + r * sn);
            const float h = n + z * (h_prev - n);
            rec::publish_word(exch + (size_t)(t & 1) * B * H + (size_t)prow * H + u,
                              rec::pack_word(h, (unsigned)(t + 1)), xlocal);
            o_h = h;
            o_r = r;
            o_z = z;
            o_n = n;
            o_a = sn;
            h_prev = h;
        }
        // @probe:step_end
        return !abort_now;
    };
    bool aborted = false;
    for (int t = 0; t < T; t += 2) {
        if (!step(t, gxs[0], gxs[1])) {
            aborted = true;
            break;
        }
        if (t + 1 < T && !step(t + 1, gxs[1], gxs[0])) {
            aborted = true;
            break;
        }
    }
    // @probe:kernel_end
    if (owner) {
        if (!aborted) store_outputs(T - 1);
        hn[(size_t)prow * H + u] = aborted ? __builtin_nanf("") : h_prev;
    }
}

// Forward recurrence for one batch row per workgroup, S = ceil(H / 64)
// slices of 64 units (one workgroup each), with the workgroup's own slice of
// h_{t-1} taken from LDS (S = 1: no exchange at all).
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
template <int S>
__global__ __launch_bounds__(NTH) void gru_fwd_local_kernel(
    const float* __restrict__ gx, const float* __restrict__ h0, const float* __restrict__ w_hh,
    const float* __restrict__ b_hh, float* __restrict__ y, float* __restrict__ hn,
    float* __restrict__ reserve, unsigned long long* __restrict__ exch, int* __restrict__ abort_flag,
    RegParams p) {
    constexpr int NR = S - 1;              // remote slots
    constexpr int NP = NR > 0 ? 8 * NR : 4;  // polled h values per wave half
    __shared__ float part[2][4][3][64];  // [step parity][k quarter][gate][unit]
    __shared__ __attribute__((aligned(16))) float hloc[2][64];
    __shared__ __attribute__((aligned(16))) float hrem[NW][2][NP];  // per wave and half: the polled h values
    __shared__ int s_abort;

    const int B = p.B, T = p.T, H = p.H;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const rec::GroupCoords gc = rec::group_coords(p.G, p.S);
    const int row = gc.g;
    const int s = gc.s;
    const int u = s * 64 + lane;  // the owner lane's unit
    const bool uvalid = u < H;
    // FMA layout: wave w takes units 32 (w / 4) + l % 32 of the slice and k
    // quarter Q = w % 4; half hf = l / 32 of the wave the eight k
    // 64 ((s + j) mod 4) + 16 Q + 8 hf + i of slot j
    const int hf = lane >> 5, uu = lane & 31, Q = wave & 3;
    const int fu = 32 * (wave >> 2) + uu;  // the lane's FMA unit within the slice
    const int uf = s * 64 + fu;
    const bool ufvalid = uf < H;
    auto kofh = [&](int half, int j, int i) { return 64 * ((s + j) % S) + 16 * Q + 8 * half + i; };
    auto kof = [&](int j, int i) { return kofh(hf, j, i); };

    // slot j's W_hh entries in w?[8 j .. 8 j + 7]
    float wr[8 * S], wz[8 * S], wn[8 * S];
    const bool vec = p.wvec != 0;
#pragma unroll
    for (int j = 0; j < S; ++j) {
#pragma unroll
        for (int i = 0; i < 8; i += 4) {
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
                const int e = 8 * j + i;
                wr[e] = a.x; wr[e + 1] = a.y; wr[e + 2] = a.z; wr[e + 3] = a.w;
                wz[e] = b.x; wz[e + 1] = b.y; wz[e + 2] = b.z; wz[e + 3] = b.w;
                wn[e] = c.x; wn[e + 1] = c.y; wn[e + 2] = c.z; wn[e + 3] = c.w;
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const bool ok = ufvalid && k + c < H;
                    wr[8 * j + i + c] = ok ? pr[c] : 0.f;
                    wz[8 * j + i + c] = ok ? pz[c] : 0.f;
                    wn[8 * j + i + c] = ok ? pn[c] : 0.f;
                }
            }
        }
    }

    const bool owner = wave == 0 && uvalid;
    float h_prev = 0.f, bias_r = 0.f, bias_z = 0.f, bias_n = 0.f;
    float gxs[2][3];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int c = 0; c < 3; ++c) gxs[e][c] = 0.f;
    const float* gx_row = gx + (size_t)row * T * 3 * H + u;
    auto load_gx = [&](float (&d)[3], int t) {
        const float* gp = gx_row + (size_t)t * 3 * H;
        d[0] = gp[0];
        d[1] = gp[H];
        d[2] = gp[2 * H];
    };
    if (owner) {
        h_prev = h0[(size_t)row * H + u];
        bias_r = b_hh[u];
        bias_z = b_hh[H + u];
        bias_n = b_hh[2 * H + u];
        load_gx(gxs[0], 0);
    }
    if (threadIdx.x == 0) s_abort = 0;
    __shared__ int s_local;
    const bool xlocal = rec::group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, abort_flag, &s_local);

    // Lane l < 2 NP polls half l / NP, slot 1 + (l % NP) / 8, entry l % 8;
    // other lanes, and lanes of a k past H, re-read the wave's first valid
    // remote word (word 0 when it has none).
    auto pkof = [&](int l) { return kofh(l / NP, 1 + (l % NP) / 8, l % 8); };
    int fallback = -1;
#pragma unroll
    for (int l = 0; l < 2 * NP * (NR > 0); ++l) {
        const int k = pkof(l);
        if (fallback < 0 && k < H) fallback = k;
    }
    const int pk = NR > 0 && lane < 2 * NP ? pkof(lane) : H;
    const bool pvalid = pk < H;
    const int pidx = pvalid ? pk : (fallback >= 0 ? fallback : 0);

    // outputs of the previous step, stored after the next poll
    float o_h = 0.f, o_r = 0.f, o_z = 0.f, o_n = 0.f, o_a = 0.f;
    float* y_row = y + (size_t)row * T * H + u;
    float* res_row = reserve ? reserve + (size_t)row * T * 4 * H + u : nullptr;
    auto store_outputs = [&](int t) {
        y_row[(size_t)t * H] = o_h;
        if (res_row) {
            float* cp = res_row + (size_t)t * 4 * H;
            cp[0] = o_r;
            cp[H] = o_z;
            cp[2 * H] = o_n;
            cp[3 * H] = o_a;
        }
    };
    // partial sums of the step in flight; the own slot's FMAs land first
    float ar[2], az[2], an[2];
    // slot j's FMAs with its eight h values (wave-uniform)
    auto fma8 = [&](const float (&hv)[8], int j) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ar[i & 1] = fmaf(hv[i], wr[8 * j + i], ar[i & 1]);
            az[i & 1] = fmaf(hv[i], wz[8 * j + i], az[i & 1]);
            an[i & 1] = fmaf(hv[i], wn[8 * j + i], an[i & 1]);
        }
    };
    auto local_fmas = [&](const float (&hv)[8]) {
        ar[0] = ar[1] = az[0] = az[1] = an[0] = an[1] = 0.f;
        fma8(hv, 0);
    };
    // eight consecutive floats of LDS as wave-uniform values
    auto lds8 = [](const float* src, float (&hv)[8]) {
        const float4 a = *reinterpret_cast<const float4*>(src);
        const float4 b = *reinterpret_cast<const float4*>(src + 4);
        hv[0] = a.x; hv[1] = a.y; hv[2] = a.z; hv[3] = a.w;
        hv[4] = b.x; hv[5] = b.y; hv[6] = b.z; hv[7] = b.w;
    };
    unsigned long long first_read = 0;
    // step 0's own slot from h0
    {
        float hv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int k = kof(0, i);
            hv[i] = k < H ? h0[(size_t)row * H + k] : 0.f;
        }
        local_fmas(hv);
    }
    auto step = [&](int t, const float (&cur)[3], float (&nxt)[3]) -> bool {
        // @probe:step_begin
        float hv[NR > 0 ? NR : 1][8];
        if constexpr (NR > 0) {
            float hx;
            if (t == 0) {
                hx = pvalid ? h0[(size_t)row * H + pidx] : 0.f;
            } else {
                const unsigned long long* src = exch + (size_t)((t - 1) & 1) * B * H + (size_t)row * H;
                const unsigned long long* pp[1] = {src + pidx};
                const bool pv[1] = {pvalid};
                unsigned long long w[1] = {first_read};
                bool ok = true;
                rec::wait_words<1>(pp, pv, w, (unsigned)t, abort_flag, ok);
                hx = pvalid ? __uint_as_float((unsigned)w[0]) : 0.f;
                if (!ok) s_abort = 1;
            }
            // lanes 0..NP-1 hold slot 1 + l / 8, entry l % 8 of half 0 (NP..
            // of half 1): through the wave's LDS row to every lane (one wave
            // writes and reads the row; LDS keeps a wave's accesses in order)
            if (lane < 2 * NP) hrem[wave][lane / NP][lane % NP] = hx;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int jj = 0; jj < NR; ++jj) lds8(&hrem[wave][hf][8 * jj], hv[jj]);
        }
        if (owner) {
            if (t > 0) store_outputs(t - 1);
            if (t + 1 < T) load_gx(nxt, t + 1);
        }
        // @probe:polled
#pragma unroll
        for (int jj = 0; jj < NR; ++jj) fma8(hv[jj], jj + 1);
        {
            // halves: lanes 0-31 get the r sum and lanes 32-63 the z sum of
            // unit fu, every lane the n sum (lower half + upper half)
            const float r0 = ar[0] + ar[1], z0 = az[0] + az[1], n0 = an[0] + an[1];
            const auto prz = __builtin_amdgcn_permlane32_swap(__float_as_uint(r0), __float_as_uint(z0), false, false);
            const auto pn = __builtin_amdgcn_permlane32_swap(__float_as_uint(n0), __float_as_uint(n0), false, false);
            part[t & 1][Q][hf][fu] = __uint_as_float(prz[0]) + __uint_as_float(prz[1]);
            if (hf == 0) part[t & 1][Q][2][fu] = __uint_as_float(pn[0]) + __uint_as_float(pn[1]);
        }
        // @probe:computed
        __syncthreads();
        // @probe:synced
        const bool abort_now = s_abort != 0;  // read with the partials
        if (owner) {
            const int pb = t & 1;
            auto tree4 = [&](int g) {
                return (part[pb][0][g][lane] + part[pb][1][g][lane]) + (part[pb][2][g][lane] + part[pb][3][g][lane]);
            };
            const float sr = bias_r + tree4(0);
            const float sz = bias_z + tree4(1);
            const float sn = bias_n + tree4(2);
            const float r = rec::sigmoid_f(cur[0] + sr);
            const float z = rec::sigmoid_f(cur[1] + sz);
            const float n = rec::tanh_f(cur[2] + r * sn);
            const float h = n + z * (h_prev - n);
            if constexpr (NR > 0)
                rec::publish_word(exch + (size_t)(t & 1) * B * H + (size_t)row * H + u,
                                  rec::pack_word(h, (unsigned)(t + 1)), xlocal);
            o_h = h;
            o_r = r;
            o_z = z;
            o_n = n;
            o_a = sn;
            h_prev = h;
        }
        if (wave == 0) hloc[t & 1][lane] = owner ? h_prev : 0.f;  // zero past H
        __syncthreads();
        // @probe:released
        // the own slot of step t+1 while the other slices' words travel,
        // with the first poll read of step t+1 already in flight
        if (t + 1 < T) {
            if constexpr (NR > 0) first_read = rec::load_word(exch + (size_t)(t & 1) * B * H + (size_t)row * H + pidx);
            float hl[8];
            lds8(&hloc[t & 1][16 * Q + 8 * hf], hl);
            local_fmas(hl);
        }
        // @probe:step_end
        return !abort_now;
    };
    bool aborted = false;
    for (int t = 0; t < T; t += 2) {
        if (!step(t, gxs[0], gxs[1])) {
            aborted = true;
            break;
        }
        if (t + 1 < T && !step(t + 1, gxs[1], gxs[0])) {
            aborted = true;
            break;
        }
    }
    // @probe:kernel_end
    if (owner) {
        if (!aborted) store_outputs(T - 1);
        hn[(size_t)row * H + u] = aborted ? __builtin_nanf("") : h_prev;
    }
}

// ------------------------------------------------------------ backward ---
template <int NJ, int ROWS>
__global__ __launch_bounds__(NTH) void gru_bwd_reg_kernel(
    const float* __restrict__ dy, const float* __restrict__ dhn, const float* __restrict__ reserve,
    const float* __restrict__ h0, const float* __restrict__ y, const float* __restrict__ w_hh,
    float* __restrict__ gout, float* __restrict__ dh0, unsigned long long* __restrict__ exch,
    int* __restrict__ abort_flag, RegParams p) {
    __shared__ float part[2][NW][ROWS][64];
    __shared__ int s_abort;

    const int B = p.B, T = p.T, H = p.H;
    const int H3 = 3 * H;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const rec::GroupCoords gc = rec::group_coords(p.G, p.S);
    const int g = gc.g;
    const int s = gc.s;
    const int u = s * 64 + lane;
    const bool uvalid = u < H;
    const int row0 = g * ROWS;
    const int jbeg = wave * p.chunk;

    // j-chunk of column u of W_hh (coalesced: lanes read consecutive units)
    float w[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
        const int j = jbeg + jj;
        w[jj] = (uvalid && jj < p.chunk && j < H3) ? w_hh[(size_t)j * H + u] : 0.f;
    }

    const int prow = row0 + wave;
    const bool owner = wave < ROWS && prow < B && uvalid;
    // Inputs of the pointwise step t (dy, r, z, n, a_n, h_{t-1}) live in set
    // (T - 1 - t) & 1 and are loaded two steps ahead, right after a poll: the
    // vector-memory counter retires in order (stores included), so loads and
    // stores issued ahead of a poll would delay its completion.
    float dh = 0.f;
    float ins[2][6];
    auto load_inputs = [&](float (&d)[6], int t) {
        const size_t bt = (size_t)prow * T + t;
        d[0] = dy ? dy[bt * H + u] : 0.f;
        const float* cp = reserve + bt * 4 * H;
        d[1] = cp[u];
        d[2] = cp[H + u];
        d[3] = cp[2 * H + u];
        d[4] = cp[3 * H + u];
        d[5] = t > 0 ? y[(bt - 1) * H + u] : h0[(size_t)prow * H + u];
    };
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int c = 0; c < 6; ++c) ins[e][c] = 0.f;
    // steps i0 .. i1-1 (i = T-1-t) of the time range
    const int i0 = T - p.t_end, i1 = T - p.t_begin;
    if (owner) {
        if (dhn) dh = dhn[(size_t)prow * H + u];
        load_inputs(ins[0], T - 1 - i0);
        if (i0 + 1 < i1) load_inputs(ins[1], T - 2 - i0);
    }
    if (threadIdx.x == 0) s_abort = 0;
    __shared__ int s_local;
    const bool xlocal = rec::group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, abort_flag, &s_local);

    // Lane l polls j = jbeg + 64 p + l (see the forward).
    constexpr int NV = NJ / 16;
    constexpr int NP = (NJ + 63) / 64;
    bool jvalid[NP];
    int jidx[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        const int jc = 64 * q + rec::poll_lane<NV>(q, lane);
        jvalid[q] = jc < p.chunk && jbeg + jc < H3;
        jidx[q] = jvalid[q] ? jbeg + jc : rec::last_valid(jbeg, p.chunk, H3);
    }
    float ddirect = 0.f;
    // one timestep (i-th from the end); false when the workgroup must stop
    auto step = [&](int i, float (&cur)[6]) -> bool {
        // @probe:step_begin
        const int t = T - 1 - i;
        unsigned long long* slotp = exch + (size_t)(i & 1) * B * H3;
        const unsigned tag = (unsigned)(i + 1);
        float dan = 0.f, drh = 0.f, dzh = 0.f, dnh = 0.f;
        if (owner) {
            const float gsum = dh + cur[0];
            const float cr = cur[1], cz = cur[2], cn = cur[3], ca = cur[4], hp = cur[5];
            const float dz = gsum * (hp - cn);
            dnh = gsum * (1.0f - cz) * (1.0f - cn * cn);
            dan = dnh * cr;
            drh = dnh * ca * cr * (1.0f - cr);
            dzh = dz * cz * (1.0f - cz);
            ddirect = gsum * cz;
            unsigned long long* wp = slotp + (size_t)prow * H3 + u;
            unsigned long long* const pp3[3] = {wp, wp + H, wp + 2 * H};
            const unsigned long long w3[3] = {rec::pack_word(drh, tag), rec::pack_word(dzh, tag),
                                              rec::pack_word(dan, tag)};
            rec::publish_words<3>(pp3, w3, xlocal);
        }
        // @probe:published
        // G_h,t[row][jbeg + 64 q + lane]
        float gx_[NP][ROWS];
        {
            constexpr int N = NP * ROWS;
            const unsigned long long* pp[N];
            bool pv[N];
            unsigned long long wd[N];
#pragma unroll
            for (int q = 0; q < NP; ++q)
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const int e = q * ROWS + r;
                    pv[e] = jvalid[q] && row0 + r < B;
                    pp[e] = slotp + (size_t)(row0 + r < B ? row0 + r : row0) * H3 + jidx[q];
                    wd[e] = rec::load_word(pp[e]);
                }
            bool ok = true;
            rec::wait_words<N>(pp, pv, wd, tag, abort_flag, ok);
#pragma unroll
            for (int q = 0; q < NP; ++q)
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const int e = q * ROWS + r;
                    gx_[q][r] = pv[e] ? __uint_as_float((unsigned)wd[e]) : 0.f;
                }
            if (!ok) s_abort = 1;
        }
        if (owner) {
            float* op = gout + ((size_t)prow * T + t) * 4 * H;
            op[u] = dan;
            op[H + u] = drh;
            op[2 * H + u] = dzh;
            op[3 * H + u] = dnh;
            if (t - 2 >= p.t_begin) load_inputs(cur, t - 2);
        }
        float gv[NV][ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) rec::replicate_rows<NV>(gx_, r, gv);
        // @probe:polled
        float acc[8][ROWS];
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[e][r] = 0.f;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
#pragma unroll
            for (int r = 0; r < ROWS; ++r) rec::dpp_src_guard(gv[v][r]);
            dot16<ROWS>(acc, gv[v], w + 16 * v);
        }
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
            part[i & 1][wave][r][lane] =
                ((acc[0][r] + acc[1][r]) + (acc[2][r] + acc[3][r])) + ((acc[4][r] + acc[5][r]) + (acc[6][r] + acc[7][r]));
        // @probe:computed
        __syncthreads();
        // @probe:synced
        const bool abort_now = s_abort != 0;  // read with the partials
        if (owner) {
            const int pb = i & 1;
            dh = ddirect + rec::tree8([&](int w2) { return part[pb][w2][wave][lane]; });
        }
        // @probe:step_end
        return !abort_now;
    };
    bool aborted = false;
    for (int i = i0; i < i1; i += 2) {
        if (!step(i, ins[0])) {
            aborted = true;
            break;
        }
        if (i + 1 < i1 && !step(i + 1, ins[1])) {
            aborted = true;
            break;
        }
    }
    // @probe:kernel_end
    if (owner) dh0[(size_t)prow * H + u] = aborted ? __builtin_nanf("") : dh;
}

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

// Backward recurrence for one batch row per workgroup, S = ceil(H / 64)
// slices, with the workgroup's own G_h words taken from LDS.
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
template <int S>
__global__ __launch_bounds__(NTH) void gru_bwd_local_kernel(
    const float* __restrict__ dy, const float* __restrict__ dhn, const float* __restrict__ reserve,
    const float* __restrict__ h0, const float* __restrict__ y, const float* __restrict__ w_hh,
    float* __restrict__ gout, float* __restrict__ dh0, unsigned long long* __restrict__ exch,
    int* __restrict__ abort_flag, RegParams p) {
    constexpr int RE = 6 * (S - 1);                  // remote entries per j-group
    constexpr int WE = 4 * RE;                       // remote entries polled per wave
    constexpr int GR = RE > 0 ? (RE + 3) / 4 * 4 : 4;  // LDS row of a j-group's polled words
    __shared__ __attribute__((aligned(16))) float part[2][NW][64];
    __shared__ __attribute__((aligned(16))) float gloc[32][8];      // own G words by j-group (6 used)
    __shared__ __attribute__((aligned(16))) float grem[NW][4][GR];  // per wave: polled words by row
    __shared__ int s_abort;

    const int B = p.B, T = p.T, H = p.H;
    const int H3 = 3 * H;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const rec::GroupCoords gc = rec::group_coords(p.G, p.S);
    const int row = gc.g;
    const int s = gc.s;
    const int u = s * 64 + lane;  // the owner lane's unit
    const bool uvalid = u < H;
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

    // W_hh[j][ub .. ub + 3] for the row's own (wl) and remote (wm) entries
    float wl[6][4], wm[RE > 0 ? RE : 1][4];
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
    for (int i = 0; i < 6; ++i) {
        bool ok;
        const int jr = own_row(6 * J + i, ok);
        load4(jr, ok, wl[i]);
    }
#pragma unroll
    for (int i = 0; i < RE; ++i) {
        bool ok;
        const int jr = rem_row(RE * J + i, ok);
        load4(jr, ok, wm[i]);
    }

    const bool owner = wave == 0 && uvalid;
    float dh = 0.f, ddirect = 0.f;
    float o_dan = 0.f, o_drh = 0.f, o_dzh = 0.f, o_dnh = 0.f;
    float ins[2][6];
    auto load_inputs = [&](float (&d)[6], int t) {
        const size_t bt = (size_t)row * T + t;
        d[0] = dy ? dy[bt * H + u] : 0.f;
        const float* cp = reserve + bt * 4 * H;
        d[1] = cp[u];
        d[2] = cp[H + u];
        d[3] = cp[2 * H + u];
        d[4] = cp[3 * H + u];
        d[5] = t > 0 ? y[(bt - 1) * H + u] : h0[(size_t)row * H + u];
    };
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int c = 0; c < 6; ++c) ins[e][c] = 0.f;
    const int i0 = T - p.t_end, i1 = T - p.t_begin;
    if (owner) {
        if (dhn) dh = dhn[(size_t)row * H + u];
        load_inputs(ins[0], T - 1 - i0);
        if (i0 + 1 < i1) load_inputs(ins[1], T - 2 - i0);
    }
    if (threadIdx.x == 0) s_abort = 0;
    __shared__ int s_local;
    const bool xlocal = rec::group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, abort_flag, &s_local);

    // Wave w polls remote entries WE w .. WE w + WE - 1: register 0 lane l
    // entry WE w + l (l < WE), register 1 (S = 4: WE = 72) lane l entry
    // WE w + 64 + l % 8.  Lanes without a word re-read the register's first
    // valid word (else the wave's first valid remote word, else word 0).
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

    // pointwise step i (t = T-1-i) from dh and its inputs: publishes G_h,t,
    // writes it to LDS by j-group, keeps the gate gradients for the store
    // after the next poll
    auto pointwise = [&](int i, const float (&cur)[6]) {
        if (owner) {
            const float gsum = dh + cur[0];
            const float cr = cur[1], cz = cur[2], cn = cur[3], ca = cur[4], hp = cur[5];
            const float dz = gsum * (hp - cn);
            o_dnh = gsum * (1.0f - cz) * (1.0f - cn * cn);
            o_dan = o_dnh * cr;
            o_drh = o_dnh * ca * cr * (1.0f - cr);
            o_dzh = dz * cz * (1.0f - cz);
            ddirect = gsum * cz;
            if constexpr (RE > 0) {
                const unsigned tag = (unsigned)(i + 1);
                unsigned long long* wp = exch + (size_t)(i & 1) * B * H3 + (size_t)row * H3 + u;
                unsigned long long* const pp3[3] = {wp, wp + H, wp + 2 * H};
                const unsigned long long w3[3] = {rec::pack_word(o_drh, tag), rec::pack_word(o_dzh, tag),
                                                  rec::pack_word(o_dan, tag)};
                rec::publish_words<3>(pp3, w3, xlocal);
            }
        }
        if (wave == 0) {
            const float gv[3] = {owner ? o_drh : 0.f, owner ? o_dzh : 0.f, owner ? o_dan : 0.f};
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const int e = 64 * c + lane;
                gloc[e / 6][e % 6] = gv[c];
            }
        }
    };
    float acc[2][4];
    // FMAs of the row's n values g[0 .. n-1] with the weights wt
    auto fma_group = [&](const float* g, int n, const float (*wt)[4]) {
#pragma unroll
        for (int i = 0; i < n; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[i & 1][v] = fmaf(g[i], wt[i][v], acc[i & 1][v]);
    };
    auto local_fmas = [&]() {
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[0][v] = acc[1][v] = 0.f;
        const float4 a = *reinterpret_cast<const float4*>(&gloc[J][0]);
        const float4 b = *reinterpret_cast<const float4*>(&gloc[J][4]);
        const float g[6] = {a.x, a.y, a.z, a.w, b.x, b.y};
        fma_group(g, 6, wl);
    };
    // the first poll reads of step i, issued ahead of its own-entry FMAs
    unsigned long long first_read[2] = {0, 0};
    auto first_poll = [&](int i) {
        const unsigned long long* slotp = exch + (size_t)(i & 1) * B * H3 + (size_t)row * H3;
        if constexpr (WE > 0) first_read[0] = rec::load_word(slotp + pidx0);
        if constexpr (WE > 64) first_read[1] = rec::load_word(slotp + pidx1);
    };
    // one timestep (i-th from the end): its G words are published and its
    // own-entry FMAs done; false when the workgroup must stop
    auto step = [&](int i, float (&cur)[6], const float (&nxt)[6]) -> bool {
        // @probe:step_begin
        const int t = T - 1 - i;
        const unsigned long long* slotp = exch + (size_t)(i & 1) * B * H3 + (size_t)row * H3;
        float g[GR];
        if constexpr (WE > 0) {
            float gr0, gr1 = 0.f;
            bool ok = true;
            if constexpr (WE > 64) {
                const unsigned long long* pp[2] = {slotp + pidx0, slotp + pidx1};
                const bool pv[2] = {pv0, pv1};
                unsigned long long wd[2] = {first_read[0], first_read[1]};
                rec::wait_words<2>(pp, pv, wd, (unsigned)(i + 1), abort_flag, ok);
                gr0 = pv0 ? __uint_as_float((unsigned)wd[0]) : 0.f;
                gr1 = pv1 ? __uint_as_float((unsigned)wd[1]) : 0.f;
            } else {
                const unsigned long long* pp[1] = {slotp + pidx0};
                const bool pv[1] = {pv0};
                unsigned long long wd[1] = {first_read[0]};
                rec::wait_words<1>(pp, pv, wd, (unsigned)(i + 1), abort_flag, ok);
                gr0 = pv0 ? __uint_as_float((unsigned)wd[0]) : 0.f;
            }
            if (!ok) s_abort = 1;
            // polled entry e of the wave to row e / RE, position e % RE of its
            // LDS block (one wave writes and reads the block; LDS keeps a
            // wave's accesses in order)
            if (lane < WE) grem[wave][lane / RE][lane % RE] = gr0;
            if (WE > 64 && lane < WE - 64) grem[wave][(64 + lane) / RE][(64 + lane) % RE] = gr1;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int k = 0; k < GR / 4; ++k) {
                const float4 v = *reinterpret_cast<const float4*>(&grem[wave][rho][4 * k]);
                g[4 * k] = v.x;
                g[4 * k + 1] = v.y;
                g[4 * k + 2] = v.z;
                g[4 * k + 3] = v.w;
            }
        }
        if (owner) {
            float* op = gout + ((size_t)row * T + t) * 4 * H;
            op[u] = o_dan;
            op[H + u] = o_drh;
            op[2 * H + u] = o_dzh;
            op[3 * H + u] = o_dnh;
            if (t - 2 >= p.t_begin) load_inputs(cur, t - 2);
        }
        // @probe:polled
        if constexpr (RE > 0) fma_group(g, RE, wm);
        float tot[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) tot[v] = acc[0][v] + acc[1][v];
        // row rho holds the wave's total for unit 4 q + rho
        part[i & 1][wave][4 * q + rho] = rows_transpose_sum(tot);
        // @probe:computed
        __syncthreads();
        // @probe:synced
        const bool abort_now = s_abort != 0;  // read with the partials
        if (owner) dh = ddirect + rec::tree8([&](int w2) { return part[i & 1][w2][lane]; });
        const bool more = i + 1 < i1;
        if (more) pointwise(i + 1, nxt);
        // @probe:published
        __syncthreads();
        // @probe:released
        if (more) {
            first_poll(i + 1);
            local_fmas();
        }
        // @probe:step_end
        return !abort_now;
    };
    if (i0 < i1) pointwise(i0, ins[0]);
    __syncthreads();
    first_poll(i0);
    local_fmas();
    bool aborted = false;
    for (int i = i0; i < i1; i += 2) {
        if (!step(i, ins[0], ins[1])) {
            aborted = true;
            break;
        }
        if (i + 1 < i1 && !step(i + 1, ins[1], ins[0])) {
            aborted = true;
            break;
        }
    }
    // @probe:kernel_end
    if (owner) dh0[(size_t)row * H + u] = aborted ? __builtin_nanf("") : dh;
}

// ------------------------------------------------------------- config ---
// Compiled per-wavefront capacities; the row-broadcast FMAs consume the
// chunk in groups of 16.
constexpr int kFwdNK[] = {16, 32};
constexpr int kBwdNJ[] = {32, 48, 64, 96};

template <int ROWS>
const void* fwd_ptr(int nk) {
    switch (nk) {
        case 16: return reinterpret_cast<const void*>(&gru_fwd_reg_kernel<16, ROWS>);
        default: return reinterpret_cast<const void*>(&gru_fwd_reg_kernel<32, ROWS>);
    }
}

template <int ROWS>
const void* bwd_ptr(int nj) {
    switch (nj) {
        case 32: return reinterpret_cast<const void*>(&gru_bwd_reg_kernel<32, ROWS>);
        case 48: return reinterpret_cast<const void*>(&gru_bwd_reg_kernel<48, ROWS>);
        case 64: return reinterpret_cast<const void*>(&gru_bwd_reg_kernel<64, ROWS>);
        default: return reinterpret_cast<const void*>(&gru_bwd_reg_kernel<96, ROWS>);
    }
}

template <int S>
const void* local_ptr(int dir) {
    return dir == 0 ? reinterpret_cast<const void*>(&gru_fwd_local_kernel<S>)
                    : reinterpret_cast<const void*>(&gru_bwd_local_kernel<S>);
}

// One batch row per workgroup: the local-slice kernels (S slices); more rows:
// the row-broadcast kernels.
const void* kernel_ptr(int dir, int cap, int rows, int slices) {
    if (rows == 1) {
        switch (slices) {
            case 1: return local_ptr<1>(dir);
            case 2: return local_ptr<2>(dir);
            case 3: return local_ptr<3>(dir);
            default: return local_ptr<4>(dir);
        }
    }
    if (dir == 0) {
        if (rows == 2) return fwd_ptr<2>(cap);
        return fwd_ptr<4>(cap);
    }
    if (rows == 2) return bwd_ptr<2>(cap);
    return bwd_ptr<4>(cap);
}

// Per-wavefront chunk and the smallest compiled capacity that holds it.
void chunk_of(int dir, int H, int* chunk, int* cap) {
    const int len = dir == 0 ? H : 3 * H;
    *chunk = ((len + NW - 1) / NW + 15) / 16 * 16;
    *cap = 0;
    if (dir == 0) {
        for (int c : kFwdNK)
            if (c >= *chunk) { *cap = c; break; }
    } else {
        for (int c : kBwdNJ)
            if (c >= *chunk) { *cap = c; break; }
    }
}

}  // namespace

int reg_choose(int dir, int batch, int hidden, const DeviceInfo& dev, int fixed_units, int fixed_rows,
               RecConfig* cfg) {
    int chunk = 0, cap = 0;
    chunk_of(dir, hidden, &chunk, &cap);
    if (cap == 0) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "register-resident recurrence needs hidden_size <= 256");
    if (fixed_units && fixed_units != 64)
        return fail(RKA_ERR_INVALID_ARGUMENT, "register-resident recurrence uses 64 units per workgroup");
    const int S = (hidden + 63) / 64;
    for (int rows : {1, 2, 4}) {
        if (fixed_rows && rows != fixed_rows) continue;
        const int G = (batch + rows - 1) / rows;
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel_ptr(dir, cap, rows, S), NTH, 0) != hipSuccess)
            continue;
        if ((long)G * S > (long)per_cu * dev.num_cus) continue;
        cfg->kind = REC_REGISTER;
        cfg->groups = G;
        cfg->slices = S;
        cfg->units = 64;
        cfg->rows = rows;
        cfg->pair_waves = 0;
        cfg->chunk = chunk;
        cfg->lds_bytes = 0;
        return 0;
    }
    return fail(RKA_ERR_TOO_LARGE_FOR_RESIDENT_LAUNCH,
                "register-resident recurrence does not fit resident: batch=" + std::to_string(batch) +
                    ", hidden=" + std::to_string(hidden));
}

int reg_launch(int dir, const RecConfig& c, const rec::Args& a, hipStream_t stream) {
    int chunk = 0, cap = 0;
    chunk_of(dir, a.H, &chunk, &cap);
    if (cap == 0 || chunk != c.chunk) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "register recurrence: bad config");
    const bool aligned = (reinterpret_cast<uintptr_t>(a.w_hh) & 15u) == 0;
    RegParams prm{a.B, a.T, a.H, c.groups, c.slices, c.chunk,
                  (aligned && (a.H & 3) == 0 && (c.chunk & 3) == 0) ? 1 : 0, a.t_begin, a.t_end,
                  a.xcc_words, a.xcc_tag};
    const void* k = kernel_ptr(dir, cap, c.rows, c.slices);
    if (dir == 0) {
        void* args[] = {(void*)&a.gx, (void*)&a.h0, (void*)&a.w_hh, (void*)&a.b_hh, (void*)&a.y, (void*)&a.hn,
                        (void*)&a.reserve, (void*)&a.exch, (void*)&a.abort_flag, (void*)&prm};
        RKA_RETURN_IF_HIP(hipLaunchKernel(k, dim3(c.groups * c.slices), dim3(NTH), args, 0, stream));
    } else {
        void* args[] = {(void*)&a.dy, (void*)&a.dhn, (void*)&a.reserve, (void*)&a.h0, (void*)&a.y,
                        (void*)&a.w_hh, (void*)&a.gout, (void*)&a.dh0, (void*)&a.exch, (void*)&a.abort_flag,
                        (void*)&prm};
        RKA_RETURN_IF_HIP(hipLaunchKernel(k, dim3(c.groups * c.slices), dim3(NTH), args, 0, stream));
    }
    return 0;
}

}  // namespace rka
