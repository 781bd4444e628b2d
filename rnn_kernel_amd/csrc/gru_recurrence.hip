// Recurrence dispatcher: picks the kernel family and decomposition for a
// shape, zeroes the exchange slots and launches the persistent kernel once
// per batch slice.
//
// Families (both persistent, the time loop inside the kernel, a plain
// launch of a grid that is resident on an idle GPU; a batch whose grid is
// not resident runs as several launches over batch slices):
//   register-resident (gru_rec_reg.hip)  hidden <= 256, W_hh slice in VGPRs;
//   LDS-tiled         (gru_rec_tiled.hip) any hidden whose tile fits LDS.
#include "rec_common.h"

#include <atomic>
#include <mutex>
#include <vector>

// Count of recurrence calls that aborted (a wait gave up), one per device;
// raised by the kernels through the pointer passed in their arguments, read
// by rka_recurrence_abort_count.  The abort flag is zeroed once per call
// (with the exchange words), so a call counts once.
__device__ unsigned long long rka_rec_abort_count;

namespace rka {

namespace {
std::mutex g_override_mutex;
struct Override {
    int kind = 0, units = 0, param = 0;
};
Override g_override[2];
std::atomic<int> g_spin_limit{kDefaultSpinPolls};
std::atomic<int> g_stall_block{-1};
std::atomic<bool> g_agent_stores{false};  // no start-up XCD check: agent-scope stores

std::mutex g_count_mutex;
std::vector<unsigned long long*> g_count_ptr;  // per device: address of rka_rec_abort_count

// Device address of this device's abort counter (the variable's host-side
// name is not a device address).
int abort_counter(int dev, unsigned long long** out) {
    std::lock_guard<std::mutex> lock(g_count_mutex);
    if ((int)g_count_ptr.size() <= dev) g_count_ptr.resize(dev + 1, nullptr);
    if (!g_count_ptr[dev]) {
        void* p = nullptr;
        RKA_RETURN_IF_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(rka_rec_abort_count)));
        g_count_ptr[dev] = reinterpret_cast<unsigned long long*>(p);
    }
    *out = g_count_ptr[dev];
    return 0;
}
}  // namespace

void set_rec_spin_limit(int polls) { g_spin_limit.store(polls > 0 ? polls : kDefaultSpinPolls); }
void set_rec_stall_block(int block) { g_stall_block.store(block); }
void set_rec_agent_stores(bool on) { g_agent_stores.store(on); }

int rec_abort_count(unsigned long long* count) {
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    unsigned long long* p = nullptr;
    RKA_RETURN_IF_ERR(abort_counter(dev->device, &p));
    RKA_RETURN_IF_HIP(hipDeviceSynchronize());
    RKA_RETURN_IF_HIP(hipMemcpy(count, p, sizeof(unsigned long long), hipMemcpyDeviceToHost));
    return 0;
}

int batch_per_resident_launch(int batch, int rows, int S, long cap) {
    const long G = (batch + rows - 1) / rows;
    if (G * S <= cap) return batch;
    long groups = cap / S;
    if (groups >= 8) groups -= groups % 8;
    return (int)std::min<long>(batch, groups * rows);
}

int grid_groups(const RecConfig& c, int groups) {
    if (groups % 8 == 0) return groups;
    const int padded = (groups + 7) / 8 * 8;
    return (long)padded * c.slices <= c.resident ? padded : groups;
}

void set_rec_override(int dir, int kind, int units, int param) {
    std::lock_guard<std::mutex> lock(g_override_mutex);
    g_override[dir] = Override{kind, units, param};
}

int choose_rec_config(int dir, int batch, int hidden, const DeviceInfo& dev, RecConfig* cfg) {
    Override o;
    {
        std::lock_guard<std::mutex> lock(g_override_mutex);
        o = g_override[dir];
    }
    if (o.kind == REC_TILED) return tiled_choose(dir, batch, hidden, dev, o.units, o.param, cfg);
    if (o.kind == REC_REGISTER) return reg_choose(dir, batch, hidden, dev, o.units, o.param, cfg);
    if (hidden <= 256 && reg_choose(dir, batch, hidden, dev, 0, 0, cfg) == 0) {
        clear_error();
        return 0;
    }
    return tiled_choose(dir, batch, hidden, dev, 0, 0, cfg);
}

namespace {
// Two exchange slots of [B, 4H] words (the largest user is the backward's
// [B, 3H] gate gradients), one start-up XCD word per workgroup, then a
// 256-byte trailer holding the abort flag.
size_t slots_bytes(int batch, int hidden) {
    return align_up((size_t)2 * batch * 4 * hidden * sizeof(unsigned long long), 256);
}
constexpr size_t kXccBytes = (size_t)rec::MAX_XCC_BLOCKS * sizeof(unsigned long long);
}  // namespace

size_t rec_workspace_bytes(int batch, int hidden) { return slots_bytes(batch, hidden) + kXccBytes + 256; }

namespace {

// Zeroes what a launch reads before it is written: the exchange words of
// the slots its direction uses, the start-up XCD words of its workgroups and
// the abort flag.
__global__ void fill_u64_kernel(unsigned long long* __restrict__ slots, size_t n_slots,
                                unsigned long long* __restrict__ xcc, size_t n_xcc, int* __restrict__ abort_flag) {
    const size_t total = n_slots + n_xcc;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        if (i < n_slots)
            slots[i] = 0ull;
        else
            xcc[i - n_slots] = 0ull;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *abort_flag = 0;
}

// Launches the recurrence of direction `dir` over the whole batch: one
// launch per batch slice of c.batch_per_launch rows (pointers offset to the
// slice's rows).  Slice k uses its own part of the exchange slots (words
// [2 r0 W, 2 (r0 + rows) W) for its first row r0, W = H forward, 3H
// backward) and start-up XCD words tagged with k, so consecutive time ranges
// of a chunked backward continue each slice on the same, once-zeroed
// workspace: tags are (steps done before this range) * launches + k + 1.
int launch_slices(int dir, const RecConfig& c, rec::Args a, unsigned long long* xcc_base, hipStream_t stream) {
    const int B = a.B, T = a.T, H = a.H;
    const size_t W = (size_t)(dir == 0 ? 1 : 3) * H;
    const unsigned long long* exch0 = a.exch;
    for (int k = 0; k < c.launches; ++k) {
        const int r0 = k * c.batch_per_launch;
        const int Bs = std::min(c.batch_per_launch, B - r0);
        RecConfig cs = c;
        cs.groups = (Bs + c.rows - 1) / c.rows;
        rec::Args s = a;
        s.B = Bs;
        auto off = [&](auto* p, size_t per_row) { return p ? p + (size_t)r0 * per_row : p; };
        s.gx = off(a.gx, (size_t)T * 3 * H);
        s.dy = off(a.dy, (size_t)T * H);
        s.dhn = off(a.dhn, (size_t)H);
        s.hn = off(a.hn, (size_t)H);
        s.gout = off(a.gout, (size_t)T * 4 * H);
        s.dh0 = off(a.dh0, (size_t)H);
        s.h0 = off(a.h0, (size_t)H);
        s.y = off(a.y, (size_t)T * H);
        s.reserve = off(a.reserve, (size_t)T * 4 * H);
        s.exch = const_cast<unsigned long long*>(exch0) + 2 * (size_t)r0 * W;
        const size_t blocks = (size_t)grid_groups(cs, cs.groups) * cs.slices;
        s.xcc_words = blocks <= (size_t)rec::MAX_XCC_BLOCKS && !g_agent_stores.load() ? xcc_base : nullptr;
        s.xcc_tag = (unsigned)((size_t)(T - a.t_end) * c.launches + k + 1);
        if (cs.kind == REC_REGISTER) {
            RKA_RETURN_IF_ERR(reg_launch(dir, cs, s, stream));
        } else {
            RKA_RETURN_IF_ERR(tiled_launch(dir, cs, s, stream));
        }
    }
    return 0;
}

// Where a launch's exchange state lives: the two slots of words, the
// start-up XCD words and the abort flag.
struct RecState {
    unsigned long long* exch;
    unsigned long long* xcc;
    int* flag;
};

// Launches direction `dir` with its exchange state at `st` (zeroed first
// when zero_ws; a backward range that continues the previous one keeps it).
int launch_at(int dir, rec::Args& a, const RecState& st, bool zero_ws, hipStream_t stream) {
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    RecConfig c{};
    RKA_RETURN_IF_ERR(choose_rec_config(dir, a.B, a.H, *dev, &c));
    if ((size_t)a.T * c.launches + c.launches >= 0xffffffffull)
        return fail(RKA_ERR_UNSUPPORTED_SHAPE, "recurrence: seq_len times batch slices exceeds the 32-bit step tags");
    a.exch = st.exch;
    a.abort_flag = st.flag;
    RKA_RETURN_IF_ERR(abort_counter(dev->device, &a.abort_count));
    unsigned long long* xcc = st.xcc;
    // Tags start at 1, so zeroed words never match; a fill kernel (not a
    // memset node) keeps the sequence capturable in a HIP graph.  Each slot
    // holds [B, H] words in the forward and [B, 3H] in the backward.  A range
    // launch that continues the previous one keeps its slots (tags grow).
    if (zero_ws) {
        const size_t n_slots = (size_t)2 * a.B * (dir == 0 ? 1 : 3) * a.H;
        const size_t blocks = (size_t)grid_groups(c, c.groups) * c.slices;
        const size_t n_xcc = blocks <= (size_t)rec::MAX_XCC_BLOCKS ? blocks : 0;
        const size_t n = n_slots + n_xcc;
        hipLaunchKernelGGL(fill_u64_kernel, dim3((unsigned)std::min<size_t>((n + 255) / 256, 1024)), dim3(256), 0,
                           stream, a.exch, n_slots, xcc, n_xcc, a.abort_flag);
        RKA_RETURN_IF_HIP(hipGetLastError());
    }
    a.spin_limit = g_spin_limit.load();
    a.stall_block = g_stall_block.load();
    return launch_slices(dir, c, a, xcc, stream);
}

int launch(int dir, rec::Args& a, void* ws, size_t ws_bytes, bool zero_ws, hipStream_t stream) {
    const size_t need = rec_workspace_bytes(a.B, a.H);
    if (ws == nullptr || ws_bytes < need)
        return fail(RKA_ERR_WORKSPACE_TOO_SMALL, "recurrence workspace too small: need " + std::to_string(need) +
                                                     " bytes, got " + std::to_string(ws_bytes));
    char* base = reinterpret_cast<char*>(ws);
    const RecState st{reinterpret_cast<unsigned long long*>(base),
                      reinterpret_cast<unsigned long long*>(base + slots_bytes(a.B, a.H)),
                      reinterpret_cast<int*>(base + need - 256)};
    return launch_at(dir, a, st, zero_ws, stream);
}

// ------------------------------------------- allocation-free forward ---
// Exchange state of rka_gru_recurrence_forward_noalloc: a file-scope device
// array, one per GPU, held until the process ends.  Layout: the forward's
// two slots of [B, H] words (at most kNoAllocSlotBytes), then the start-up
// XCD words, then the abort flag.  The array's name is a host-side
// stand-in, not a device address: host code uses only the address that
// hipGetSymbolAddress returns for the current device.
constexpr size_t kNoAllocSlotBytes = size_t(4) << 20;
constexpr size_t kNoAllocXccBytes = (size_t)rec::MAX_XCC_BLOCKS * sizeof(unsigned long long);
constexpr size_t kNoAllocScratchBytes = kNoAllocSlotBytes + kNoAllocXccBytes + 256;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
std::vector<char*> g_scratch_ptr;  // per device: device address of `scratch`
std::vector<unsigned> g_scratch_calls;  // per device: calls so far (step-tag base)

// Step-tag base of the next call on a device: the call count (1..255,
// wrapping) in the top 8 bits, so the steps (below 2^24) of two calls
// whose launches overlap on the shared array never share a tag.  Such calls
// race (documented); with distinct tags the waits of each give up on words
// the other overwrote, the calls abort (NaN outputs, the abort counter) and
// neither returns finite values taken from the other.
unsigned next_tag_base(int dev) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if ((int)g_scratch_calls.size() <= dev) g_scratch_calls.resize(dev + 1, 0u);
    const unsigned c = g_scratch_calls[dev] % 255u + 1u;
    g_scratch_calls[dev] = c;
    return c << 24;
}

int scratch_address(int dev, char** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        RKA_RETURN_IF_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch_ptr[dev] = reinterpret_cast<char*>(p);
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

namespace {
__global__ void eval_gate_kernel(const float* __restrict__ x, float* __restrict__ sig, float* __restrict__ th, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        sig[i] = rec::sigmoid_f(x[i]);
        th[i] = rec::tanh_f(x[i]);
    }
}
}  // namespace

int eval_gate_functions(const float* x, float* sig, float* th, int n, hipStream_t stream) {
    if (n < 0 || (n > 0 && (!x || !sig || !th))) return fail(RKA_ERR_INVALID_ARGUMENT, "eval_gate_functions: bad args");
    if (n == 0) return 0;
    hipLaunchKernelGGL(eval_gate_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, x, sig, th, n);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

size_t rec_noalloc_max_slot_bytes() { return kNoAllocSlotBytes; }

int launch_rec_forward_noalloc(const float* gx, const float* h0, const float* w_hh, const float* b_hh, float* y,
                               float* hn, float* reserve, int B, int T, int H, hipStream_t stream) {
    const size_t slot_bytes = align_up((size_t)2 * B * H * sizeof(unsigned long long), 256);
    if (slot_bytes > kNoAllocSlotBytes)
        return fail(RKA_ERR_UNSUPPORTED_SHAPE,
                    "rka_gru_recurrence_forward_noalloc: batch * hidden_size = " + std::to_string((size_t)B * H) +
                        " exceeds the static scratch limit of " + std::to_string(kNoAllocSlotBytes / 16) +
                        " (use rka_gru_recurrence_forward with a workspace)");
    if (T >= (1 << 24))
        return fail(RKA_ERR_UNSUPPORTED_SHAPE, "rka_gru_recurrence_forward_noalloc: seq_len " + std::to_string(T) +
                                                   " must stay below 2^24 (its step tags carry a call number)");
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    char* ptr = nullptr;
    RKA_RETURN_IF_ERR(scratch_address(dev->device, &ptr));
    const RecState st{reinterpret_cast<unsigned long long*>(ptr),
                      reinterpret_cast<unsigned long long*>(ptr + kNoAllocSlotBytes),
                      reinterpret_cast<int*>(ptr + kNoAllocSlotBytes + kNoAllocXccBytes)};
    rec::Args a;
    a.gx = gx;
    a.h0 = h0;
    a.w_hh = w_hh;
    a.b_hh = b_hh;
    a.y = y;
    a.hn = hn;
    a.reserve = reserve;
    a.B = B;
    a.T = T;
    a.H = H;
    a.t_begin = 0;
    a.t_end = T;
    a.tag_base = next_tag_base(dev->device);
    return launch_at(0, a, st, true, stream);
}

int launch_rec_forward(const float* gx, const float* h0, const float* w_hh, const float* b_hh,
                       float* y, float* hn, float* reserve, void* ws, size_t ws_bytes,
                       int B, int T, int H, hipStream_t stream, bool zero_ws) {
    rec::Args a;
    a.gx = gx;
    a.h0 = h0;
    a.w_hh = w_hh;
    a.b_hh = b_hh;
    a.y = y;
    a.hn = hn;
    a.reserve = reserve;
    a.B = B;
    a.T = T;
    a.H = H;
    a.t_begin = 0;
    a.t_end = T;
    return launch(0, a, ws, ws_bytes, zero_ws, stream);
}

int launch_rec_backward(const float* dy, const float* dhn, const float* reserve,
                        const float* h0, const float* y, const float* w_hh,
                        float* g, float* dh0, void* ws, size_t ws_bytes,
                        int B, int T, int H, hipStream_t stream) {
    return launch_rec_backward_range(dy, dhn, reserve, h0, y, w_hh, g, dh0, ws, ws_bytes, B, T, H, 0, T, true,
                                     stream);
}

int launch_rec_backward_range(const float* dy, const float* dh_in, const float* reserve,
                              const float* h0, const float* y, const float* w_hh,
                              float* g, float* dh_out, void* ws, size_t ws_bytes,
                              int B, int T, int H, int t_begin, int t_end, bool zero_ws, hipStream_t stream) {
    if (t_begin < 0 || t_end > T || t_begin >= t_end)
        return fail(RKA_ERR_INVALID_ARGUMENT, "backward recurrence: bad time range");
    const float* dhn = dh_in;
    float* dh0 = dh_out;
    rec::Args a;
    a.dy = dy;
    a.dhn = dhn;
    a.reserve = const_cast<float*>(reserve);
    a.h0 = h0;
    a.y = const_cast<float*>(y);
    a.w_hh = w_hh;
    a.gout = g;
    a.dh0 = dh0;
    a.B = B;
    a.T = T;
    a.H = H;
    a.t_begin = t_begin;
    a.t_end = t_end;
    return launch(1, a, ws, ws_bytes, zero_ws, stream);
}

}  // namespace rka
