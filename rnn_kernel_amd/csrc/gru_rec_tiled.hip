// LDS-tiled persistent GRU recurrences (the general family).
//
// The batch is cut into G groups of `rows` sequences and the hidden units
// into S slices of `units` units (a divisor of 64); workgroup (g, s) owns the
// (row, unit) pairs of that tile for the whole sequence and keeps the W_hh
// entries its units need in LDS, loaded once.  Each step it gathers the
// group's exchanged rows (h_{t-1} forward, G_h,t backward) into LDS, splits
// the dot products over its 8 wavefronts by k-chunk, reduces the partials in
// LDS and applies the gate math on the owning lanes.  Any hidden size whose
// tile fits in LDS is accepted; the register-resident kernels
// (gru_rec_reg.hip) are faster and are preferred where they apply.
//
// Forward maths (src/rnn_kernel/a100/prod/kernels/a100_gru_h256_kernels.cu:756-776):
//   a = W_hh h_{t-1} + b_hh; r = sigmoid(gx_r + a_r); z = sigmoid(gx_z + a_z);
//   n = tanh(gx_n + r a_n); h_t = n + z (h_{t-1} - n); reserve[b, t, u] = (r, z, n, a_n)
// Backward maths (a100_gru_h256_kernels.cu:842-866,915-932), g = dh_t + dy_t:
//   dz = g (h_{t-1} - n), dn^ = g (1 - z)(1 - n^2), dr^ = dn^ a_n r (1 - r),
//   dz^ = dz z (1 - z), da_n = dn^ r; dh_{t-1} = g z + G_h W_hh.
//   g_out[b,t] = (da_n, dr^, dz^, dn^), so that G_i = columns [H,4H) and
//   G_h = the rotation of columns [0,3H) are contiguous ranges.
#include "rec_common.h"

#include <algorithm>
#include <cmath>

namespace rka {
namespace {

struct RecParams {
    int B, T, H;
    int G, S, U, Bg;   // groups, slices, units per slice, rows per group
    int RP;            // padded LDS row length (floats) of the exchanged rows
    int KCH;           // k-chunk per wavefront (multiple of 4)
    int KLEN;          // dot-product length rounded up to 4 (H fwd, 3H bwd)
    int t_begin, t_end;  // backward: time range processed
    unsigned long long* xcc_words;  // start-up XCD check (nullable)
    unsigned xcc_tag;
    unsigned tag_base;                    // forward: added to every step tag (rec::Args::tag_base)
    int spin_limit;                       // poll rounds before a wait gives up
    unsigned long long* abort_count;      // per-device count of aborted launches
    int stall_block;                      // test failure injection (rec::Args::stall_block)
};

// Gathers `nrows` rows of `len` published words with step tag `tag` from
// src (row stride `len`) into LDS rows of stride RP.  Returns false when the
// wait gave up (see rec::WaitCtl) or another workgroup raised the abort flag.
__device__ bool gather_rows(const unsigned long long* __restrict__ src, int nrows, int len, unsigned tag,
                            float* __restrict__ dst, int RP, const rec::WaitCtl& wc) {
    using namespace rec;
    const int total = nrows * len;
    bool ok = true;
    for (int base = 0; base < total; base += NTH * 4) {
        unsigned long long w[4];
        int idx[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            idx[j] = base + j * NTH + (int)threadIdx.x;
            w[j] = idx[j] < total ? load_word(src + idx[j]) : 0ull;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (idx[j] >= total) continue;
            int spins = 0;
            while ((unsigned)(w[j] >> 32) != tag) {
                if (!ok) break;
                if (++spins >= wc.spin_limit) {
                    raise_abort(wc);
                    ok = false;
                    break;
                }
                if ((spins & 1023) == 0 && abort_raised(wc)) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                w[j] = load_word(src + idx[j]);
            }
            const int r = idx[j] / len;
            const int k = idx[j] - r * len;
            dst[r * RP + k] = __uint_as_float((unsigned)w[j]);
        }
    }
    return ok;
}

// ------------------------------------------------------------- forward ---
template <int PW>
__global__ __launch_bounds__(rec::NTH) void gru_rec_forward_kernel(
    const float* __restrict__ gx, const float* __restrict__ h0, const float* __restrict__ w_hh,
    const float* __restrict__ b_hh, float* __restrict__ y, float* __restrict__ hn,
    float* __restrict__ reserve, unsigned long long* __restrict__ exch, int* __restrict__ abort_flag,
    RecParams p) {
    using namespace rec;
    constexpr int KC = NW / PW;
    constexpr int NP = 64 * PW;  // pair slots per workgroup
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ int s_abort;

    const int B = p.B, T = p.T, H = p.H, RP = p.RP;
    float* Wl = lds;                         // [U][3][RP]  W_hh rows of the slice's units
    float* hl = Wl + p.U * 3 * RP;           // [Bg][RP]    h_{t-1} of the group's rows
    float* part = hl + p.Bg * RP;            // [2][KC][3][NP]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int pw = wave % PW;
    const int kc = wave / PW;
    const GroupCoords gc = group_coords(p.S);
    if (gc.g >= p.G) return;  // padding workgroup of a grid rounded up to whole XCDs
    const int g = gc.g;
    const int s = gc.s;
    const int pair = pw * 64 + lane;
    const int bl = pair / p.U;
    const int ul = pair - bl * p.U;
    const int b = g * p.Bg + bl;
    const int u = s * p.U + ul;
    const bool slot = bl < p.Bg;
    const bool valid = slot && b < B && u < H;
    const bool owner = valid && kc == 0;
    const int row0 = g * p.Bg;
    const int nrows = max(0, min(p.Bg, B - row0));

    for (int idx = tid; idx < p.U * 3 * RP; idx += NTH) {
        const int k = idx % RP;
        const int rest = idx / RP;
        const int gate = rest % 3;
        const int unit = s * p.U + rest / 3;
        Wl[idx] = (k < H && unit < H) ? w_hh[(size_t)(gate * H + unit) * H + k] : 0.f;
    }
    for (int idx = tid; idx < p.Bg * RP; idx += NTH) {
        const int r = idx / RP;
        const int k = idx - r * RP;
        hl[idx] = (r < nrows && k < H) ? h0[(size_t)(row0 + r) * H + k] : 0.f;
    }
    if (tid == 0) s_abort = 0;

    float h_prev = 0.f, bias_r = 0.f, bias_z = 0.f, bias_n = 0.f;
    float gxr = 0.f, gxz = 0.f, gxn = 0.f;
    if (owner) {
        h_prev = h0[(size_t)b * H + u];
        bias_r = b_hh[u];
        bias_z = b_hh[H + u];
        bias_n = b_hh[2 * H + u];
        const float* gp = gx + (size_t)b * T * 3 * H;
        gxr = gp[u];
        gxz = gp[H + u];
        gxn = gp[2 * H + u];
    }
    const int kbeg = kc * p.KCH;
    const int kend = min(p.KLEN, kbeg + p.KCH);
    const float* wr = Wl + (ul * 3) * RP;
    const float* hrow = hl + bl * RP;
    // iteration t stores the outputs of step t: after an iteration that
    // aborts, rows t_stop .. T-1 were not stored
    int t_stop = T;
    const int pub_flip = (int)blockIdx.x == p.stall_block ? 1 : 0;  // test failure injection
    const WaitCtl wc{abort_flag, p.abort_count, p.spin_limit};
    __shared__ int s_local;
    // the group = the S workgroups of rec::group_coords; plain publishing stores when they share an XCD
    const bool xlocal = group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, wc, &s_local);
    __syncthreads();

    for (int t = 0; t < T; ++t) {
        if (t > 0) {
            const unsigned long long* src = exch + (size_t)((t - 1) & 1) * B * H + (size_t)row0 * H;
            if (!gather_rows(src, nrows, H, p.tag_base + (unsigned)t, hl, RP, wc)) s_abort = 1;
            __syncthreads();
        }
        float ar = 0.f, az = 0.f, an = 0.f;
        if (slot) {
            for (int k = kbeg; k < kend; k += 4) {
                const float4 hv = *reinterpret_cast<const float4*>(hrow + k);
                const float4 w0 = *reinterpret_cast<const float4*>(wr + k);
                const float4 w1 = *reinterpret_cast<const float4*>(wr + RP + k);
                const float4 w2 = *reinterpret_cast<const float4*>(wr + 2 * RP + k);
                ar = fmaf(hv.x, w0.x, ar); ar = fmaf(hv.y, w0.y, ar);
                ar = fmaf(hv.z, w0.z, ar); ar = fmaf(hv.w, w0.w, ar);
                az = fmaf(hv.x, w1.x, az); az = fmaf(hv.y, w1.y, az);
                az = fmaf(hv.z, w1.z, az); az = fmaf(hv.w, w1.w, az);
                an = fmaf(hv.x, w2.x, an); an = fmaf(hv.y, w2.y, an);
                an = fmaf(hv.z, w2.z, an); an = fmaf(hv.w, w2.w, an);
            }
        }
        float* pp = part + ((t & 1) * KC + kc) * 3 * NP;
        pp[pair] = ar;
        pp[NP + pair] = az;
        pp[2 * NP + pair] = an;
        __syncthreads();
        if (s_abort) {
            t_stop = t;
            break;
        }
        if (owner) {
            float sr = bias_r, sz = bias_z, sn = bias_n;
            const float* pb = part + (t & 1) * KC * 3 * NP;
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                sr += pb[c * 3 * NP + pair];
                sz += pb[c * 3 * NP + NP + pair];
                sn += pb[c * 3 * NP + 2 * NP + pair];
            }
            const float r = sigmoid_f(gxr + sr);
            const float z = sigmoid_f(gxz + sz);
            const float n = tanh_f(gxn + r * sn);
            const float h = n + z * (h_prev - n);
            publish_word(exch + (size_t)((t & 1) ^ pub_flip) * B * H + (size_t)b * H + u,
                         pack_word(h, p.tag_base + (unsigned)(t + 1)), xlocal);
            const size_t bt = (size_t)b * T + t;
            y[bt * H + u] = h;
            if (reserve) *reinterpret_cast<float4*>(reserve + bt * 4 * H + 4 * u) = make_float4(r, z, n, sn);
            h_prev = h;
            if (t + 1 < T) {
                const float* gp = gx + (bt + 1) * 3 * H;
                gxr = gp[u];
                gxz = gp[H + u];
                gxn = gp[2 * H + u];
            }
        }
    }
    const bool aborted = t_stop < T;
    if (owner) {
        const float nan = __builtin_nanf("");
        for (int t = t_stop; t < T; ++t) {
            const size_t bt = (size_t)b * T + t;
            y[bt * H + u] = nan;
            if (reserve) *reinterpret_cast<float4*>(reserve + bt * 4 * H + 4 * u) = make_float4(nan, nan, nan, nan);
        }
        hn[(size_t)b * H + u] = aborted ? nan : h_prev;
    }
}

// ------------------------------------------------------------ backward ---
template <int PW>
__global__ __launch_bounds__(rec::NTH) void gru_rec_backward_kernel(
    const float* __restrict__ dy, const float* __restrict__ dhn, const float* __restrict__ reserve,
    const float* __restrict__ h0, const float* __restrict__ y, const float* __restrict__ w_hh,
    float* __restrict__ gout, float* __restrict__ dh0, unsigned long long* __restrict__ exch,
    int* __restrict__ abort_flag, RecParams p) {
    using namespace rec;
    constexpr int KC = NW / PW;
    constexpr int NP = 64 * PW;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ int s_abort;

    const int B = p.B, T = p.T, H = p.H, RP = p.RP;
    const int H3 = 3 * H;
    float* Wt = lds;                    // [U][RP]   column u of W_hh, all 3H gate rows
    float* gl = Wt + p.U * RP;          // [Bg][RP]  G_h,t rows of the group (r, z, n order)
    float* part = gl + p.Bg * RP;       // [2][KC][NP]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int pw = wave % PW;
    const int kc = wave / PW;
    const GroupCoords gc = group_coords(p.S);
    if (gc.g >= p.G) return;  // padding workgroup of a grid rounded up to whole XCDs
    const int g = gc.g;
    const int s = gc.s;
    const int pair = pw * 64 + lane;
    const int bl = pair / p.U;
    const int ul = pair - bl * p.U;
    const int b = g * p.Bg + bl;
    const int u = s * p.U + ul;
    const bool slot = bl < p.Bg;
    const bool valid = slot && b < B && u < H;
    const bool owner = valid && kc == 0;
    const int row0 = g * p.Bg;
    const int nrows = max(0, min(p.Bg, B - row0));

    for (int idx = tid; idx < p.U * RP; idx += NTH) {
        const int j = idx % RP;
        const int unit = s * p.U + idx / RP;
        Wt[idx] = (j < H3 && unit < H) ? w_hh[(size_t)j * H + unit] : 0.f;
    }
    for (int idx = tid; idx < p.Bg * RP; idx += NTH) gl[idx] = 0.f;
    if (tid == 0) s_abort = 0;

    float dh = 0.f;
    float dyv = 0.f, cr = 0.f, cz = 0.f, cn = 0.f, ca = 0.f, hp = 0.f;
    if (owner) {
        if (dhn) dh = dhn[(size_t)b * H + u];
        const int tl = p.t_end - 1;
        const size_t bt = (size_t)b * T + tl;
        if (dy) dyv = dy[bt * H + u];
        const float4 c4 = *reinterpret_cast<const float4*>(reserve + bt * 4 * H + 4 * u);
        cr = c4.x; cz = c4.y; cn = c4.z; ca = c4.w;
        hp = (tl > 0) ? y[(bt - 1) * H + u] : h0[(size_t)b * H + u];
    }
    const int kbeg = kc * p.KCH;
    const int kend = min(p.KLEN, kbeg + p.KCH);
    const float* wrow = Wt + ul * RP;
    const float* grow = gl + bl * RP;
    // iteration i stores the G row of step i: after an iteration that
    // aborts, rows i_stop + 1 .. T - 1 - t_begin were not stored
    const int i1 = T - p.t_begin;
    int i_stop = i1;
    const int pub_flip = (int)blockIdx.x == p.stall_block ? 1 : 0;  // test failure injection
    float ddirect = 0.f;
    const WaitCtl wc{abort_flag, p.abort_count, p.spin_limit};
    __shared__ int s_local;
    const bool xlocal = group_on_one_xcd(p.xcc_words, gc.first, gc.stride, p.S, p.xcc_tag, wc, &s_local);
    __syncthreads();

    // global step i = T-1-t over the time range (tags and slots continue
    // across consecutive range launches)
    for (int i = T - p.t_end; i < i1; ++i) {
        const int t = T - 1 - i;
        unsigned long long* slotp = exch + (size_t)(i & 1) * B * H3;
        if (owner) {
            const float gsum = dh + dyv;
            const float dz = gsum * (hp - cn);
            const float dnh = gsum * (1.0f - cz) * (1.0f - cn * cn);
            const float dan = dnh * cr;
            const float drh = dnh * ca * cr * (1.0f - cr);
            const float dzh = dz * cz * (1.0f - cz);
            ddirect = gsum * cz;
            const unsigned tag = (unsigned)(i + 1);
            unsigned long long* wp = exch + (size_t)((i & 1) ^ pub_flip) * B * H3 + (size_t)b * H3 + u;
            publish_word(wp, pack_word(drh, tag), xlocal);
            publish_word(wp + H, pack_word(dzh, tag), xlocal);
            publish_word(wp + 2 * H, pack_word(dan, tag), xlocal);
            const size_t bt = (size_t)b * T + t;
            float* op = gout + bt * 4 * H;  // streaming stores, as in the register family
            __builtin_nontemporal_store(dan, op + u);
            __builtin_nontemporal_store(drh, op + H + u);
            __builtin_nontemporal_store(dzh, op + 2 * H + u);
            __builtin_nontemporal_store(dnh, op + 3 * H + u);
            if (t > p.t_begin) {
                const size_t pbt = bt - 1;
                dyv = dy ? dy[pbt * H + u] : 0.f;
                const float4 c4 = *reinterpret_cast<const float4*>(reserve + pbt * 4 * H + 4 * u);
                cr = c4.x; cz = c4.y; cn = c4.z; ca = c4.w;
                hp = (t > 1) ? y[(pbt - 1) * H + u] : h0[(size_t)b * H + u];
            }
        }
        if (!gather_rows(slotp + (size_t)row0 * H3, nrows, H3, (unsigned)(i + 1), gl, RP, wc)) s_abort = 1;
        __syncthreads();
        float acc = 0.f;
        if (slot) {
            for (int k = kbeg; k < kend; k += 4) {
                const float4 gv = *reinterpret_cast<const float4*>(grow + k);
                const float4 wv = *reinterpret_cast<const float4*>(wrow + k);
                acc = fmaf(gv.x, wv.x, acc); acc = fmaf(gv.y, wv.y, acc);
                acc = fmaf(gv.z, wv.z, acc); acc = fmaf(gv.w, wv.w, acc);
            }
        }
        part[((i & 1) * KC + kc) * NP + pair] = acc;
        __syncthreads();
        if (s_abort) {
            i_stop = i;
            break;
        }
        if (owner) {
            float sum = ddirect;
            const float* pb = part + (i & 1) * KC * NP;
#pragma unroll
            for (int c = 0; c < KC; ++c) sum += pb[c * NP + pair];
            dh = sum;
        }
    }
    const bool aborted = i_stop < i1;
    if (owner) {
        const float nan = __builtin_nanf("");
        for (int i = i_stop + 1; i < i1; ++i) {
            float* op = gout + ((size_t)b * T + (T - 1 - i)) * 4 * H;
            op[u] = nan;
            op[H + u] = nan;
            op[2 * H + u] = nan;
            op[3 * H + u] = nan;
        }
        dh0[(size_t)b * H + u] = aborted ? nan : dh;
    }
}

int rows_padded(int len) {
    // Row stride = len rounded up to 64 floats plus 4: consecutive rows start
    // 4 banks apart, so the b128 reads of distinct rows do not conflict.
    return (len + 63) / 64 * 64 + 4;
}

int lds_bytes_for(int dir, int H, int U, int Bg, int PW) {
    const int KC = rec::NW / PW;
    const int NP = 64 * PW;
    if (dir == 0) {
        const int RP = rows_padded(H);
        return (U * 3 * RP + Bg * RP + 2 * KC * 3 * NP) * 4;
    }
    const int RP = rows_padded(3 * H);
    return (U * RP + Bg * RP + 2 * KC * NP) * 4;
}

const void* kernel_ptr(int dir, int PW) {
    if (dir == 0) {
        if (PW == 1) return reinterpret_cast<const void*>(&gru_rec_forward_kernel<1>);
        if (PW == 2) return reinterpret_cast<const void*>(&gru_rec_forward_kernel<2>);
        return reinterpret_cast<const void*>(&gru_rec_forward_kernel<4>);
    }
    if (PW == 1) return reinterpret_cast<const void*>(&gru_rec_backward_kernel<1>);
    if (PW == 2) return reinterpret_cast<const void*>(&gru_rec_backward_kernel<2>);
    return reinterpret_cast<const void*>(&gru_rec_backward_kernel<4>);
}

int max_resident(const DeviceInfo& dev, int dir, int PW, int lds) {
    const void* k = kernel_ptr(dir, PW);
    if (lds > 65536) {
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) return 0;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, rec::NTH, lds) != hipSuccess) return 0;
    return per_cu * dev.num_cus;
}

RecParams make_params(int dir, int B, int T, int H, const RecConfig& c) {
    RecParams p{};
    p.B = B;
    p.T = T;
    p.H = H;
    p.G = c.groups;
    p.S = c.slices;
    p.U = c.units;
    p.Bg = c.rows;
    const int len = dir == 0 ? H : 3 * H;
    p.RP = rows_padded(len);
    p.KLEN = (len + 3) / 4 * 4;
    const int KC = rec::NW / c.pair_waves;
    p.KCH = ((p.KLEN + KC - 1) / KC + 3) / 4 * 4;
    p.t_begin = 0;
    p.t_end = T;
    return p;
}

}  // namespace

// The decomposition with the lowest modelled cost among those whose tile
// fits LDS.  A grid that is not resident for the whole batch runs as
// launches over batch slices of the most groups that are (the cost of a
// step then counts once per launch).
int tiled_choose(int dir, int batch, int hidden, const DeviceInfo& dev, int fixed_u, int fixed_pw, RecConfig* cfg) {
    const int ncu = dev.num_cus > 0 ? dev.num_cus : 256;
    const int lds_cap = dev.max_lds_per_block > 0 ? dev.max_lds_per_block : 65536;
    bool found = false;
    double best = 0;
    RecConfig best_cfg{};
    for (int PW : {1, 2, 4}) {
        if (fixed_pw && PW != fixed_pw) continue;
        for (int U : {32, 16, 8, 4, 2, 1, 64}) {
            if (fixed_u && U != fixed_u) continue;
            const int Bg = std::min(PW * (64 / U), batch);
            if (Bg < 1) continue;
            // Only use PW > 1 when its extra rows are needed.
            if (PW > 1 && (PW / 2) * (64 / U) >= batch && !fixed_pw) continue;
            const int S = (hidden + U - 1) / U;
            const int lds = lds_bytes_for(dir, hidden, U, Bg, PW);
            if (lds > lds_cap) continue;
            const int cap = max_resident(dev, dir, PW, lds);
            if (cap < S) continue;
            const int per_launch = batch_per_resident_launch(batch, Bg, S, cap);
            const int launches = (batch + per_launch - 1) / per_launch;
            const int G = (per_launch + Bg - 1) / Bg;
            const int nwg = G * S;
            // Per-step cost model fitted to measured sweeps: the number of
            // slices exchanging per group dominates, then per-workgroup work
            // (times the workgroups sharing a CU) and the gathered volume.
            const double work = (double)Bg * U * hidden * 3.0 / (64.0 * PW);
            const double share = std::ceil((double)nwg / ncu);
            const double xfer = (double)Bg * hidden * (dir == 0 ? 1 : 3) / rec::NTH;
            double score = (work * share + 4.0 * xfer + 60.0 * S) * launches;
            if (!found || score < best) {
                found = true;
                best = score;
                best_cfg.kind = REC_TILED;
                best_cfg.groups = G;
                best_cfg.slices = S;
                best_cfg.units = U;
                best_cfg.rows = Bg;
                best_cfg.pair_waves = PW;
                best_cfg.chunk = 0;
                best_cfg.lds_bytes = lds;
                best_cfg.launches = launches;
                best_cfg.batch_per_launch = per_launch;
                best_cfg.resident = cap;
            }
        }
    }
    if (!found) {
        return fail(RKA_ERR_TOO_LARGE_FOR_RESIDENT_LAUNCH,
                    "no decomposition of the " + std::string(dir == 0 ? "forward" : "backward") +
                        " recurrence fits LDS: hidden=" + std::to_string(hidden));
    }
    *cfg = best_cfg;
    return 0;
}

int tiled_launch(int dir, const RecConfig& c, const rec::Args& a, hipStream_t stream) {
    RecParams prm = make_params(dir, a.B, a.T, a.H, c);
    prm.t_begin = a.t_begin;
    prm.t_end = a.t_end;
    prm.xcc_words = a.xcc_words;
    prm.xcc_tag = a.xcc_tag;
    prm.tag_base = a.tag_base;
    prm.spin_limit = a.spin_limit;
    prm.abort_count = a.abort_count;
    prm.stall_block = a.stall_block;
    const void* k = kernel_ptr(dir, c.pair_waves);
    const unsigned blocks = (unsigned)(grid_groups(c, c.groups) * c.slices);
    if (c.lds_bytes > 65536) {
        RKA_RETURN_IF_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, c.lds_bytes));
    }
    if (dir == 0) {
        void* args[] = {(void*)&a.gx, (void*)&a.h0, (void*)&a.w_hh, (void*)&a.b_hh, (void*)&a.y, (void*)&a.hn,
                        (void*)&a.reserve, (void*)&a.exch, (void*)&a.abort_flag, (void*)&prm};
        RKA_RETURN_IF_HIP(hipLaunchKernel(k, dim3(blocks), dim3(rec::NTH), args, (unsigned)c.lds_bytes, stream));
    } else {
        void* args[] = {(void*)&a.dy, (void*)&a.dhn, (void*)&a.reserve, (void*)&a.h0, (void*)&a.y,
                        (void*)&a.w_hh, (void*)&a.gout, (void*)&a.dh0, (void*)&a.exch, (void*)&a.abort_flag,
                        (void*)&prm};
        RKA_RETURN_IF_HIP(hipLaunchKernel(k, dim3(blocks), dim3(rec::NTH), args, (unsigned)c.lds_bytes, stream));
    }
    return 0;
}

}  // namespace rka
