// Forward recurrence on the matrix cores, for batches of 16-row groups.
//
// The register-resident forward (gru_rec_reg.hip) gives every workgroup one
// batch row and 64 hidden units and runs W_hh h_{t-1} as per-lane VALU FMAs;
// a batch of more than 64 rows at H = 256 then needs 2 or 4 rows per
// workgroup, multiplying every wavefront's FMAs.  Here workgroup (g, s) owns
// batch rows [16 g, 16 g + 16) and hidden units [16 s, 16 s + 16), and the
// step's product is one 48 x 16 x H matrix product on v_mfma_f32_16x16x4_f32
// (A = the 48 W_hh rows of the slice's r, z, n gates, B = h_{t-1} of the 16
// rows): 3 H / 4 MFMAs per workgroup and step, spread over 8 wavefronts.
// Wavefront w takes the contiguous K range [H w / 8, H (w + 1) / 8) (NKW =
// H / 32 four-deep K steps) for all three gates, so the h values it needs
// come from only H / 128 producer workgroups and every lane polls exactly
// the NKW words its B operand takes: no LDS relay.
//
// MFMA operand layout (v_mfma_f32_16x16x4_f32, 64 lanes): lane l supplies
// A[l % 16][l / 16] and B[l / 16][l % 16]; register r of the result holds
// D[4 (l / 16) + r][l % 16].  With A rows = units and B columns = batch
// rows, lane l of wavefront w holds for K step n
//   a[m][n] = W_hh[m H + 16 s + l % 16][4 (NKW w + n) + l / 16]
//   b[n]    = h_{t-1}[16 g + l % 16][4 (NKW w + n) + l / 16]
// and its results are the partial sums of units 16 s + 4 (l / 16) + r,
// batch row 16 g + l % 16 over the wavefront's K range.
//
// Exchange: each step's h_t is published as 64-bit words {fp32 bits, step
// tag} in a slot of the step's parity, laid out [unit][batch] so that the
// 16 batch rows a poll instruction's 16 lanes read at one k form one
// 128-byte line.  Every lane re-polls its NKW words until all carry the
// step's tag (a first pass polling one word per producer, then the rest,
// measured slower: 2.45 vs 2.31 us per step at c4).
//
// One barrier per step: the wavefronts write their partial sums (double
// buffered by step parity) and meet; owner wavefronts 0..3 (lane l: batch
// row 16 g + l % 16, unit 16 s + 4 w + l / 16) sum the eight partials per
// gate in a fixed tree, apply the gates, publish h_t, store y and the
// reserve, and load the next step's input gates; the other wavefronts go
// straight to polling the next step's words.  A writer reaches step t + 2
// (the same slot) only after every member of its group has published step
// t + 1, i.e. finished reading step t, so two slots suffice.
//
// Failure handling and start-up are those of the register kernels (rec::
// WaitCtl, group placement on one XCD, NaN into every unwritten row).
//
// Measured on MI355X (c4 shape, B = 256, H = 256, T = 1024, forward only):
// 2.31 us per step against 2.11 us for the register kernel at four rows per
// workgroup, and 2.5-2.7 us against 0.87-0.92 us at B = 16 / 64 (one row
// per register workgroup).  The matrix cores take ~0.4 us of the step (a
// timing copy without the MFMAs: 2.06 us); the rest is the exchange, every
// step waiting for the slowest of the group's 16 producers, and the owners'
// per-step input-gate loads, which miss to HBM at c4 (805 MB of gx) and hold
// back the CU's polls (without them: 2.04 us).  So the automatic choice
// never takes this kernel; rka_set_recurrence_config(0, RKA_REC_MFMA, 0, 0)
// forces it (tests, tuning).
//
// Forward maths (src/rnn_kernel/a100/prod/kernels/a100_gru_h256_kernels.cu:756-776):
//   a = W_hh h_{t-1} + b_hh; r = sigmoid(gx_r + a_r); z = sigmoid(gx_z + a_z);
//   n = tanh(gx_n + r a_n); h_t = n + z (h_{t-1} - n); reserve[b, t, u] = (r, z, n, a_n)
#include "rec_common.h"

#include <algorithm>

namespace rka {
namespace {

using rec::NTH;
using rec::NW;

typedef float floatx4 __attribute__((ext_vector_type(4)));

struct MfmaParams {
    int B, T, H;
    int G, S;                        // 16-row groups, 16-unit slices
    unsigned long long* xcc_words;   // start-up XCD check (nullable)
    unsigned xcc_tag;
    int spin_limit;
    unsigned long long* abort_count;
    int stall_block;
};

constexpr int kRows = 16;   // batch rows per workgroup
constexpr int kUnits = 16;  // hidden units per workgroup
constexpr int kPartStride = 17;  // LDS row (batch row) stride of a partial tile, padded

template <int NKW>
__global__ __launch_bounds__(NTH) void gru_fwd_mfma_kernel(
    const float* __restrict__ gx, const float* __restrict__ h0, const float* __restrict__ w_hh,
    const float* __restrict__ b_hh, float* __restrict__ y, float* __restrict__ hn,
    float* __restrict__ reserve, unsigned long long* __restrict__ exch, int* __restrict__ abort_flag,
    MfmaParams p) {
    static_assert(NKW >= 1 && NKW <= 8, "K steps per wavefront");
    // partial sums [step parity][gate][wavefront][batch row][unit]
    __shared__ float part[2][3][NW][kRows * kPartStride];
    __shared__ int s_abort;
    __shared__ int s_local;

    const int B = p.B, T = p.T, H = p.H;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const rec::GroupCoords gc = rec::group_coords(p.S);
    if (gc.g >= p.G) return;  // padding workgroup of a grid rounded up to whole XCDs
    const int g = gc.g, s = gc.s;
    const int col = lane & 15, kk = lane >> 4;

    // A operands: W_hh rows of the slice's units (row l % 16), k of the
    // wavefront's K steps
    float a[3][NKW];
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
        for (int n = 0; n < NKW; ++n)
            a[m][n] = w_hh[(size_t)(m * H + kUnits * s + col) * H + 4 * (NKW * wave + n) + kk];

    // the B words of this lane: h_{t-1}[16 g + col][k_n], k_n = 4 (NKW w + n) + kk,
    // at word k_n * B + 16 g + col of a slot
    const int brow = kRows * g + col;
    int woff[NKW];
#pragma unroll
    for (int n = 0; n < NKW; ++n) woff[n] = (4 * (NKW * wave + n) + kk) * B + brow;

    // owner wavefronts 0..3: batch row 16 g + col, unit 16 s + 4 w + kk
    const bool owner = wave < 4;
    const int ob = brow;
    const int ou = kUnits * s + 4 * wave + kk;
    float h_prev = 0.f, bias_r = 0.f, bias_z = 0.f, bias_n = 0.f;
    float gxs[2][3] = {{0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}};
    const float* gx_row = gx + (size_t)ob * T * 3 * H + ou;
    auto load_gx = [&](float (&d)[3], int t) {
        const float* gp = gx_row + (size_t)t * 3 * H;
        d[0] = gp[0];
        d[1] = gp[H];
        d[2] = gp[2 * H];
    };
    if (owner) {
        h_prev = h0[(size_t)ob * H + ou];
        bias_r = b_hh[ou];
        bias_z = b_hh[H + ou];
        bias_n = b_hh[2 * H + ou];
        load_gx(gxs[0], 0);
    }
    if (threadIdx.x == 0) s_abort = 0;
    const rec::WaitCtl wc{abort_flag, p.abort_count, p.spin_limit};
    const bool xlocal = rec::group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, wc, &s_local);

    // the owner lane's word in the slot of each step parity (32-bit
    // offsets, 2 B H < 2^31); the failure injection swaps the two
    const int pub_flip = (int)blockIdx.x == p.stall_block ? 1 : 0;
    const unsigned pub_off[2] = {(unsigned)(pub_flip * B * H + ou * B + ob),
                                 (unsigned)((1 - pub_flip) * B * H + ou * B + ob)};
    float* y_row = y + (size_t)ob * T * H + ou;
    float* res_row = reserve ? reserve + (size_t)ob * T * 4 * H + 4 * ou : nullptr;

    unsigned long long bw[NKW];
    auto step = [&](int t, const float (&cur)[3], float (&nxt)[3]) -> bool {
        float bv[NKW];
        if (t == 0) {
#pragma unroll
            for (int n = 0; n < NKW; ++n) bv[n] = h0[(size_t)brow * H + 4 * (NKW * wave + n) + kk];
        } else {
            const unsigned long long* slot = exch + (size_t)((t - 1) & 1) * B * H;
            const unsigned tag = (unsigned)t;
            bool ok = true;
            // every word of the lane, re-polled until its tag is current
            const unsigned long long* pp[NKW];
            bool pv[NKW];
#pragma unroll
            for (int n = 0; n < NKW; ++n) {
                pp[n] = slot + woff[n];
                pv[n] = true;
                bw[n] = rec::load_word(pp[n]);
            }
            rec::wait_words<NKW>(pp, pv, bw, tag, wc, ok);
            if (!ok) s_abort = 1;
            // a word whose wait gave up (or was skipped after the probe's
            // did) enters the sums as NaN, never as a stale value
#pragma unroll
            for (int n = 0; n < NKW; ++n)
                bv[n] = (unsigned)(bw[n] >> 32) == tag ? __uint_as_float((unsigned)bw[n]) : __builtin_nanf("");
        }
        // the owner's next input gates after its poll (a load that misses
        // to HBM holds back the CU's later loads, polls included)
        if (owner && t + 1 < T) load_gx(nxt, t + 1);
        floatx4 acc[3];
#pragma unroll
        for (int m = 0; m < 3; ++m) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int n = 0; n < NKW; ++n)
#pragma unroll
            for (int m = 0; m < 3; ++m)
                acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[m][n], bv[n], acc[m], 0, 0, 0);
        // result register r: unit 4 kk + r (within the slice), batch row col
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) part[t & 1][m][wave][col * kPartStride + 4 * kk + r] = acc[m][r];
        __syncthreads();
        const bool abort_now = s_abort != 0;  // read with the partials
        if (owner && !abort_now) {
            const float* pb = &part[t & 1][0][0][col * kPartStride + 4 * wave + kk];
            auto tree = [&](int m) {
                return rec::tree8([&](int w2) { return pb[(m * NW + w2) * kRows * kPartStride]; });
            };
            const float sr = bias_r + tree(0);
            const float sz = bias_z + tree(1);
            const float sn = bias_n + tree(2);
            const float r = rec::sigmoid_f(cur[0] + sr);
            const float z = rec::sigmoid_f(cur[1] + sz);
            const float n = rec::tanh_f(cur[2] + r * sn);
            const float h = n + z * (h_prev - n);
            unsigned off = pub_off[t & 1];
            asm volatile("" : "+v"(off));
            rec::publish_word(exch + off, rec::pack_word(h, (unsigned)(t + 1)), xlocal);
            y_row[(size_t)t * H] = h;
            if (res_row) *reinterpret_cast<float4*>(res_row + (size_t)t * 4 * H) = make_float4(r, z, n, sn);
            h_prev = h;
        }
        return !abort_now;
    };
    // step t stores the outputs of step t: after a step that aborts, rows
    // t_stop .. T-1 were not stored
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
    const bool aborted = t_stop < T;
    if (owner) {
        if (aborted) {
            const float nan = __builtin_nanf("");
            for (int t = t_stop; t < T; ++t) {
                y_row[(size_t)t * H] = nan;
                if (res_row) *reinterpret_cast<float4*>(res_row + (size_t)t * 4 * H) = make_float4(nan, nan, nan, nan);
            }
        }
        hn[(size_t)ob * H + ou] = aborted ? __builtin_nanf("") : h_prev;
    }
}

const void* mfma_ptr(int nkw) {
    switch (nkw) {
        case 1: return reinterpret_cast<const void*>(&gru_fwd_mfma_kernel<1>);
        case 2: return reinterpret_cast<const void*>(&gru_fwd_mfma_kernel<2>);
        case 3: return reinterpret_cast<const void*>(&gru_fwd_mfma_kernel<3>);
        case 4: return reinterpret_cast<const void*>(&gru_fwd_mfma_kernel<4>);
        case 5: return reinterpret_cast<const void*>(&gru_fwd_mfma_kernel<5>);
        case 6: return reinterpret_cast<const void*>(&gru_fwd_mfma_kernel<6>);
        case 7: return reinterpret_cast<const void*>(&gru_fwd_mfma_kernel<7>);
        case 8: return reinterpret_cast<const void*>(&gru_fwd_mfma_kernel<8>);
        default: return nullptr;
    }
}

// Unused dynamic LDS that keeps a workgroup above half of the CU's 160 KB,
// so that the 256 workgroups of a c4 launch take one CU each rather than
// two of them sharing a CU's matrix cores while another CU idles.
constexpr unsigned kSpreadLds = 61440;

}  // namespace

bool mfma_applicable(int dir, int batch, int hidden) {
    return dir == 0 && batch >= kRows && batch % kRows == 0 && hidden >= 32 && hidden <= 256 &&
           (hidden / 32) * 32 == hidden && mfma_ptr(hidden / 32) != nullptr;
}

int mfma_choose(int dir, int batch, int hidden, const DeviceInfo& dev, RecConfig* cfg) {
    if (!mfma_applicable(dir, batch, hidden))
        return fail(RKA_ERR_UNSUPPORTED_SHAPE,
                    "mfma recurrence: forward only, batch a multiple of 16, hidden_size a multiple of 32 in [32, 256]");
    const void* k = mfma_ptr(hidden / 32);
    RKA_RETURN_IF_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kSpreadLds));
    int per_cu = 0;
    RKA_RETURN_IF_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, NTH, kSpreadLds));
    const long cap = (long)per_cu * (dev.num_cus > 0 ? dev.num_cus : 256);
    const int S = hidden / kUnits;
    if (cap < S) return fail(RKA_ERR_TOO_LARGE_FOR_RESIDENT_LAUNCH, "mfma recurrence: a group does not fit");
    const int per_launch = batch_per_resident_launch(batch, kRows, S, cap);
    RecConfig c{};
    c.kind = REC_MFMA;
    c.groups = per_launch / kRows;
    c.slices = S;
    c.units = kUnits;
    c.rows = kRows;
    c.pair_waves = 0;
    c.chunk = 4 * (hidden / 32);
    c.lds_bytes = 0;
    c.launches = (batch + per_launch - 1) / per_launch;
    c.batch_per_launch = per_launch;
    c.resident = cap;
    *cfg = c;
    return 0;
}

int mfma_launch(int dir, const RecConfig& c, const rec::Args& a, hipStream_t stream) {
    if (dir != 0) return fail(RKA_ERR_INVALID_ARGUMENT, "mfma recurrence: forward only");
    MfmaParams prm{};
    prm.B = a.B;
    prm.T = a.T;
    prm.H = a.H;
    prm.G = c.groups;
    prm.S = c.slices;
    prm.xcc_words = a.xcc_words;
    prm.xcc_tag = a.xcc_tag;
    prm.spin_limit = a.spin_limit;
    prm.abort_count = a.abort_count;
    prm.stall_block = a.stall_block;
    if (a.B % kRows != 0 || c.groups * kRows != a.B)
        return fail(RKA_ERR_INVALID_ARGUMENT, "mfma recurrence: batch slice must be whole 16-row groups");
    const void* k = mfma_ptr(a.H / 32);
    if (!k) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "mfma recurrence: hidden_size");
    RKA_RETURN_IF_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kSpreadLds));
    void* args[] = {(void*)&a.gx, (void*)&a.h0, (void*)&a.w_hh, (void*)&a.b_hh, (void*)&a.y, (void*)&a.hn,
                    (void*)&a.reserve, (void*)&a.exch, (void*)&a.abort_flag, (void*)&prm};
    const unsigned blocks = (unsigned)(grid_groups(c, c.groups) * c.slices);
    RKA_RETURN_IF_HIP(hipLaunchKernel(k, dim3(blocks), dim3(NTH), args, kSpreadLds, stream));
    return 0;
}

}  // namespace rka
