// Internal declarations shared by the rnn_kernel_amd translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/rnn_kernel_amd.h"

namespace rka {

// ---------------------------------------------------------------- errors ---
void set_error(const std::string& msg);
void clear_error();

#define RKA_RETURN_IF_HIP(expr)                                                  \
    do {                                                                         \
        hipError_t rka_e_ = (expr);                                              \
        if (rka_e_ != hipSuccess) {                                              \
            ::rka::set_error(std::string(#expr) + ": " + hipGetErrorString(rka_e_)); \
            return static_cast<int>(rka_e_);                                     \
        }                                                                        \
    } while (0)

#define RKA_RETURN_IF_ERR(expr)      \
    do {                             \
        int rka_rc_ = (expr);        \
        if (rka_rc_ != 0) return rka_rc_; \
    } while (0)

int fail(int code, const std::string& msg);

// ------------------------------------------------------- device queries ---
struct DeviceInfo {
    int device = -1;
    int num_cus = 0;
    int max_lds_per_block = 0;
    bool gfx950 = false;
    std::string arch;
};
// Cached per device; returns 0 or an error code.
int current_device_info(const DeviceInfo** out);

// --------------------------------------------------------------- layout ---
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ----------------------------------------------------------------- GEMM ---
// Segment map of a row index i of the underlying 2-D array:
// len == 0: i; else (i / len) * stride + off + i % len.  With len = L,
// stride = T, off = t0 it selects rows (b, t0 .. t0+L-1) of a [B, T, .]
// tensor, i.e. one time chunk of every sequence.
struct SegMap {
    int len = 0, stride = 0, off = 0;
};

struct GemmOperand {
    const float* ptr = nullptr;
    int ld = 0;
    int kmajor = 0;            // 0: element (r,k) at ptr[r*ld+k]; 1: at ptr[k*ld+r]
    // Row remap for k-major operands used by the dW_hh product: when
    // shift_T > 0, k = b*shift_T + t reads row k-1 of ptr for t > 0 and row b
    // of shift_first (ld shift_ld) for t == 0, i.e. the rows of
    // [h0 ; y[:, :-1]] without materialising them.
    int shift_T = 0;
    const float* shift_first = nullptr;
    // applied first to the underlying row (k if kmajor, else r)
    SegMap seg{};
};

// C[m,n] = sum_k A(m,k) B(n,k) + bias[n]; direct store (row m of C at
// c_seg(m)).
// zero / zero_words: a buffer of 64-bit words the launch also clears (the
// next kernel's exchange state, so that it needs no fill launch of its own).
int gemm_direct(int m, int n, int k, const GemmOperand& a, const GemmOperand& b,
                const float* bias, float* c, int ldc, hipStream_t stream, SegMap c_seg = SegMap{},
                unsigned long long* zero = nullptr, size_t zero_words = 0);

// Split-K partial products only: slices [z_off, z_off + ksplit) of a
// partial buffer holding ksplit_total slices (layout as gemm_splitk).
int gemm_splitk_partials(int m, int n, int k, const GemmOperand& a, const GemmOperand& b, bool want_colsum,
                         float* partial, int ksplit, int z_off, int ksplit_total, hipStream_t stream);
// out[o] = sum of the ksplit_total slices at row (o + rot) % m; colsum likewise.
int splitk_reduce(int m, int n, const float* partial, int ksplit_total, int rot, float* c, int ldc,
                  float* colsum, hipStream_t stream);

// Split-K products reduce deterministically.  Output rows are rotated:
// out[o] = C[(o + rot) % m] (rot = 0: no rotation).  colsum (nullable)
// receives sum_k A(m,k) with the same rotation.  A partial buffer of
// ksplit slices holds splitk_partial_floats(m, n, ksplit) floats.
size_t splitk_partial_floats(int m, int n, int ksplit);
// One product of gemm_splitk_pair_partials.
struct SplitProduct {
    int m, n, k;
    GemmOperand a, b;
    float* c;
    int ldc;
    float* colsum;
    int rot;
    float* partial;
    int ksplit;
};
// The partial products of two split-K products in one launch (all slices
// of each; reduce each with splitk_reduce); only p0's B operand may carry
// the row remap.  With the reductions, the same results as two gemm_splitk
// calls with the same slices.
int gemm_splitk_pair_partials(const SplitProduct& p0, const SplitProduct& p1, hipStream_t stream);
int splitk_reduce(const SplitProduct& p, hipStream_t stream);
// Both products' reductions in one launch (the same results as two
// splitk_reduce calls).
int splitk_reduce_pair(const SplitProduct& p0, const SplitProduct& p1, hipStream_t stream);
// gemm_direct (no bias) and splitk_reduce_pair(p0, p1) in one launch: the
// same results as the two calls.
int gemm_direct_reduce_pair(int m, int n, int k, const GemmOperand& a, const GemmOperand& b, float* c, int ldc,
                            const SplitProduct& p0, const SplitProduct& p1, hipStream_t stream);
// rka_set_gemm_tiles (RKA_GEMM_TILES_AUTO or RKA_GEMM_TILES_128).
int set_gemm_tiles(int mode);
// Slices for a split-K product of about wgs_per_cu workgroups per CU
// (0: half a workgroup per CU, for products that share the GPU with a
// concurrently running recurrence); a multiple of 8 from 8 up.
int choose_ksplit(int m, int n, int k, int num_cus, int wgs_per_cu);

// ----------------------------------------------------------- recurrence ---
enum RecKind { REC_AUTO = 0, REC_TILED = 1, REC_REGISTER = 2 };

// A recurrence runs as `launches` kernel launches over consecutive batch
// slices of `batch_per_launch` rows (the last one possibly shorter), each a
// grid that is resident on an idle GPU: every workgroup of a launch can run
// at once, so no exchange group waits for another group to finish.
struct RecConfig {
    int kind = 0;          // REC_TILED or REC_REGISTER
    int groups = 0;        // batch-row groups per launch (of a full slice)
    int slices = 0;        // hidden-unit slices
    int units = 0;         // hidden units per slice
    int rows = 0;          // batch rows per group
    int pair_waves = 0;    // tiled: wavefronts holding (row, unit) pairs
    int chunk = 0;         // register: k (forward) / j (backward) values per wavefront
    int lds_bytes = 0;     // dynamic LDS (tiled) or 0
    int launches = 1;      // batch slices, one launch each
    int batch_per_launch = 0;
    long resident = 0;     // workgroups of the chosen kernel resident on the device
};
// Exchange groups in the grid of a launch of `groups` groups: rounded up to
// a multiple of 8 when that padded grid is still resident, so that each
// group's workgroups share one XCD (rec::group_coords); the padding
// workgroups exit at once.  Otherwise `groups`.
int grid_groups(const RecConfig& c, int groups);
// Batch rows per launch for a family whose grid of G groups of `rows` rows
// and S slices holds at most `cap` resident workgroups (cap >= S): the whole
// batch when it fits, else the most groups that fit, rounded down to a
// multiple of 8 when that leaves at least 8 (groups then share an XCD).
int batch_per_resident_launch(int batch, int rows, int S, long cap);
int choose_rec_config(int dir, int batch, int hidden, const DeviceInfo& dev, RecConfig* cfg);
// Per-direction override used by rka_set_recurrence_config: kind, units, param.
void set_rec_override(int dir, int kind, int units, int param);
// Poll rounds a recurrence wait makes before it gives up (the default, and
// the largest value rka_set_spin_limit accepts).
constexpr int kDefaultSpinPolls = 1 << 24;
constexpr int kMaxSpinPolls = 1 << 30;
void set_rec_spin_limit(int polls);
void set_rec_stall_block(int block);
// rka_set_exchange_stores: true forces agent-scope exchange stores.
void set_rec_agent_stores(bool on);
// Number of recurrence launches on the current device that aborted since
// the library was loaded (synchronises the device).
int rec_abort_count(unsigned long long* count);

size_t rec_workspace_bytes(int batch, int hidden);
int eval_gate_functions(const float* x, float* sig, float* th, int n, hipStream_t stream);

// zero_ws false: the workspace's recurrence state was cleared by an earlier
// kernel on the stream (rka_gru_forward's input GEMM).
int launch_rec_forward(const float* gx, const float* h0, const float* w_hh, const float* b_hh,
                       float* y, float* hn, float* reserve, void* ws, size_t ws_bytes,
                       int B, int T, int H, hipStream_t stream, bool zero_ws = true);
// The same with the exchange state in a static per-device array (no
// workspace); 2 B H words at most rec_noalloc_max_slot_bytes() / 8.
int launch_rec_forward_noalloc(const float* gx, const float* h0, const float* w_hh, const float* b_hh, float* y,
                               float* hn, float* reserve, int B, int T, int H, hipStream_t stream);
size_t rec_noalloc_max_slot_bytes();
int launch_rec_backward(const float* dy, const float* dhn, const float* reserve,
                        const float* h0, const float* y, const float* w_hh,
                        float* g, float* dh0, void* ws, size_t ws_bytes,
                        int B, int T, int H, hipStream_t stream);
// Steps t_end-1 .. t_begin only: dh_in seeds dh_{t_end-1} (NULL = 0), dh_out
// receives dh_{t_begin-1}.  Consecutive ranges (descending) on the same
// workspace continue one another; zero_ws must be set on the first.
int launch_rec_backward_range(const float* dy, const float* dh_in, const float* reserve,
                              const float* h0, const float* y, const float* w_hh,
                              float* g, float* dh_out, void* ws, size_t ws_bytes,
                              int B, int T, int H, int t_begin, int t_end, bool zero_ws, hipStream_t stream);

}  // namespace rka
