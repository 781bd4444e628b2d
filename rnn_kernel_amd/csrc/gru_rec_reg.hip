// Host side of the register-resident persistent GRU recurrences: kernel
// choice per direction, rows and slices, and the launches (the kernels are
// in rec_reg_kernels.h).
#include "rec_reg_kernels.h"

namespace rka {
namespace {

// ------------------------------------------------------------- config ---
// Compute wavefronts of the one-row forward: sixteen at four slices (every
// wave has half the FMAs of eight, and the owner stores its own outputs: a
// workgroup holds at most 1024 threads), else eight plus the I/O wavefront.
// Measured on MI355X (same box, alternating runs, forward per launch): c2
// 434-437 vs 443 us; at one to three slices the I/O wavefront wins (H = 64,
// 128, 192: 359 / 365 / 403 vs 370 / 389 / 427 us).
constexpr int fwd_waves1(int S) { return S == 4 ? 16 : 8; }

template <int S>
const void* local_ptr(int dir, int rows, bool io, bool full) {
    if (dir == 1) {
        if (rows == 1) {
            // whole slices at three and four slices: the instances built with
            // max-ilp
            if constexpr (S >= 3) {
                if (full) return rec_bwd1_kernel(S);
                return reinterpret_cast<const void*>(&gru_bwd_local_kernel<S, 1, 16>);
            } else {
                return full ? reinterpret_cast<const void*>(&gru_bwd_local_kernel<S, 1, 16, 1, true>)
                            : reinterpret_cast<const void*>(&gru_bwd_local_kernel<S, 1, 16>);
            }
        }
        if (full && rows == 4) return reinterpret_cast<const void*>(&gru_bwd_local_kernel<S, 4, NW, 2, true>);
        switch (rows) {
            case 2: return reinterpret_cast<const void*>(&gru_bwd_local_kernel<S, 2>);
            default: return reinterpret_cast<const void*>(&gru_bwd_local_kernel<S, 4, NW, 2>);
        }
    }
    switch (rows) {
        case 1:
            if (full) {
                if constexpr (S == 4) return rec_fwd1_kernel();
                return io ? reinterpret_cast<const void*>(&gru_fwd_local_kernel<S, 1, true, NW, true>)
                          : reinterpret_cast<const void*>(&gru_fwd_local_kernel<S, 1, false, fwd_waves1(S), true>);
            }
            return io ? reinterpret_cast<const void*>(&gru_fwd_local_kernel<S, 1, true>)
                      : reinterpret_cast<const void*>(&gru_fwd_local_kernel<S, 1, false, fwd_waves1(S)>);
        case 2: return reinterpret_cast<const void*>(&gru_fwd_local_kernel<S, 2, false>);
        default:
            return full ? reinterpret_cast<const void*>(&gru_fwd_mfma4_kernel<S, true>)
                        : reinterpret_cast<const void*>(&gru_fwd_mfma4_kernel<S>);
    }
}

// Whether the kernel for (dir, rows, slices) has the I/O wavefront: the
// forward with one row per workgroup and eight compute wavefronts.
bool uses_io(int dir, int rows, int slices) { return dir == 0 && rows == 1 && fwd_waves1(slices) == 8; }

int block_threads(int dir, int rows, int slices) {
    if (dir == 1 && rows == 1) return 16 * 64;  // the one-row backward: sixteen wavefronts
    if (dir == 0 && rows == 1) return fwd_waves1(slices) * 64 + (uses_io(dir, rows, slices) ? 64 : 0);
    return NTH;
}

// The local-slice kernels: S slices, 1, 2 or 4 batch rows per workgroup.
// full: H = 64 * slices (the one-row forward has instances for it).
const void* kernel_ptr(int dir, int cap, int rows, int slices, bool full = false) {
    (void)cap;
    const bool io = uses_io(dir, rows, slices);
    switch (slices) {
        case 1: return local_ptr<1>(dir, rows, io, full);
        case 2: return local_ptr<2>(dir, rows, io, full);
        case 3: return local_ptr<3>(dir, rows, io, full);
        default: return local_ptr<4>(dir, rows, io, full);
    }
}

// Units per workgroup and whether the register-resident kernels hold H.
void chunk_of(int dir, int H, int* chunk, int* cap) {
    (void)dir;
    *chunk = 64;  // units per workgroup
    *cap = H <= 256 ? 1 : 0;
}

}  // namespace

// Batch rows per workgroup the local-slice kernels are built for.
int max_rows(int dir, int slices) {
    (void)dir;
    (void)slices;
    return 4;
}

// The fewest rows per workgroup whose B·S workgroups are resident; when
// none is, the most rows, and the batch runs as several launches over
// slices whose grids are resident.
int reg_choose(int dir, int batch, int hidden, const DeviceInfo& dev, int fixed_units, int fixed_rows,
               RecConfig* cfg) {
    int chunk = 0, cap = 0;
    chunk_of(dir, hidden, &chunk, &cap);
    if (cap == 0) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "register-resident recurrence needs hidden_size <= 256");
    if (fixed_units && fixed_units != 64)
        return fail(RKA_ERR_INVALID_ARGUMENT, "register-resident recurrence uses 64 units per workgroup");
    const int S = (hidden + 63) / 64;
    if (fixed_rows > max_rows(dir, S))
        return fail(RKA_ERR_UNSUPPORTED_SHAPE, "register-resident forward holds at most " +
                                                   std::to_string(max_rows(dir, S)) + " rows at hidden_size " +
                                                   std::to_string(hidden));
    int chosen = 0;
    long chosen_cap = 0;
    for (int rows : {1, 2, 4}) {
        if (rows > max_rows(dir, S) || (fixed_rows && rows != fixed_rows)) continue;
        const int G = (batch + rows - 1) / rows;
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel_ptr(dir, cap, rows, S), block_threads(dir, rows, S),
                                                         0) != hipSuccess)
            continue;
        const long resident = (long)per_cu * dev.num_cus;
        chosen = rows;  // the last candidate (the most rows) unless one fits
        chosen_cap = resident;
        if ((long)G * S <= resident) break;
    }
    if (chosen == 0 || chosen_cap < S)
        return fail(RKA_ERR_TOO_LARGE_FOR_RESIDENT_LAUNCH, "register-resident recurrence: no resident grid at hidden_size " +
                                                               std::to_string(hidden));
    cfg->kind = REC_REGISTER;
    cfg->batch_per_launch = batch_per_resident_launch(batch, chosen, S, chosen_cap);
    cfg->launches = (batch + cfg->batch_per_launch - 1) / cfg->batch_per_launch;
    cfg->groups = (cfg->batch_per_launch + chosen - 1) / chosen;
    cfg->slices = S;
    cfg->units = 64;
    cfg->rows = chosen;
    cfg->pair_waves = 0;
    cfg->chunk = chunk;
    cfg->lds_bytes = 0;
    cfg->resident = chosen_cap;
    return 0;
}

int reg_launch(int dir, const RecConfig& c, const rec::Args& a, hipStream_t stream) {
    int chunk = 0, cap = 0;
    chunk_of(dir, a.H, &chunk, &cap);
    if (cap == 0 || chunk != c.chunk) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "register recurrence: bad config");
    const bool aligned = (reinterpret_cast<uintptr_t>(a.w_hh) & 15u) == 0;
    RegParams prm{a.B, a.T, a.H, c.groups, c.slices, c.chunk,
                  (aligned && (a.H & 3) == 0 && (c.chunk & 3) == 0) ? 1 : 0, a.t_begin, a.t_end,
                  a.xcc_words, a.xcc_tag, a.tag_base, a.spin_limit, a.abort_count, a.stall_block};
    // whole slices: the forward always takes the compile-time-H instances;
    // the one-row backward only on grids of 128 or more workgroups (c2: 434
    // -> 427 us per launch; at 64 workgroups, c5, 3.44 -> 3.54 ms per step)
    bool full = a.H == 64 * c.slices;
    if (dir == 1 && c.rows == 1 && (long)c.groups * c.slices < 128) full = false;
    const void* k = kernel_ptr(dir, cap, c.rows, c.slices, full);
    if (k == nullptr) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "register recurrence: no kernel for this row count");
    const unsigned blocks = (unsigned)(grid_groups(c, c.groups) * c.slices);
    if (dir == 0) {
        void* args[] = {(void*)&a.gx, (void*)&a.h0, (void*)&a.w_hh, (void*)&a.b_hh, (void*)&a.y, (void*)&a.hn,
                        (void*)&a.reserve, (void*)&a.exch, (void*)&a.abort_flag, (void*)&prm};
        RKA_RETURN_IF_HIP(hipLaunchKernel(k, dim3(blocks), dim3(block_threads(dir, c.rows, c.slices)), args, 0, stream));
    } else {
        void* args[] = {(void*)&a.dy, (void*)&a.dhn, (void*)&a.reserve, (void*)&a.h0, (void*)&a.y,
                        (void*)&a.w_hh, (void*)&a.gout, (void*)&a.dh0, (void*)&a.exch, (void*)&a.abort_flag,
                        (void*)&prm};
        RKA_RETURN_IF_HIP(hipLaunchKernel(k, dim3(blocks), dim3(block_threads(dir, c.rows, c.slices)), args, 0, stream));
    }
    return 0;
}

}  // namespace rka
