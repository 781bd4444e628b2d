// extern "C" entry points of librnn_kernel_amd.so (declared in
// include/rnn_kernel_amd.h).  Argument validation, workspace carving and the
// order of the stage launches of one GRU layer live here; the kernels are in
// gemm_f32.hip and gru_recurrence.hip.
#include "rka_internal.h"

#include <cstring>
#include <mutex>
#include <vector>

namespace rka {

namespace {
thread_local std::string t_last_error;
std::mutex g_dev_mutex;
std::vector<DeviceInfo*> g_devs;
}  // namespace

void set_error(const std::string& msg) { t_last_error = msg; }
void clear_error() { t_last_error.clear(); }

int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

int current_device_info(const DeviceInfo** out) {
    int dev = 0;
    RKA_RETURN_IF_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_dev_mutex);
    if ((int)g_devs.size() <= dev) g_devs.resize(dev + 1, nullptr);
    if (!g_devs[dev]) {
        hipDeviceProp_t prop;
        RKA_RETURN_IF_HIP(hipGetDeviceProperties(&prop, dev));
        auto* info = new DeviceInfo();
        info->device = dev;
        info->num_cus = prop.multiProcessorCount;
        info->max_lds_per_block = (int)prop.sharedMemPerBlock;
        info->arch = prop.gcnArchName;
        info->gfx950 = info->arch.rfind("gfx950", 0) == 0;
        g_devs[dev] = info;
    }
    *out = g_devs[dev];
    if (!(*out)->gfx950)
        return fail(RKA_ERR_UNSUPPORTED_DEVICE,
                    "rnn_kernel_amd is built for gfx950 (MI355X); device " + std::to_string(dev) + " is " +
                        (*out)->arch);
    return 0;
}

namespace {

int check_dims(int B, int T, int I, int H) {
    if (B < 1 || T < 1 || H < 1 || I < 1)
        return fail(RKA_ERR_INVALID_ARGUMENT, "batch, seq_len, input_size and hidden_size must be >= 1");
    if ((size_t)B * T > (size_t)0x7fffffff / 4 / (size_t)std::max(H, I))
        return fail(RKA_ERR_UNSUPPORTED_SHAPE, "batch*seq_len*features exceeds 32-bit indexing");
    return 0;
}

struct FwdLayout {
    size_t gx, rec, total;
};
FwdLayout fwd_layout(int B, int T, int I, int H) {
    (void)I;
    FwdLayout l{};
    l.gx = 0;
    l.rec = align_up((size_t)B * T * 3 * H * sizeof(float), 256);
    l.total = l.rec + rec_workspace_bytes(B, H);
    return l;
}

struct BwdLayout {
    size_t g, rec, part_hh, part_ih, total;
    int ks_hh, ks_ih;  // split-K slices
};
BwdLayout bwd_layout(int B, int T, int I, int H) {
    BwdLayout l{};
    const int K = B * T;
    // the two products share one launch (gemm_splitk_pair), so each is sized
    // for half the CUs at three resident workgroups per CU
    l.ks_hh = choose_ksplit(3 * H, H, K, 128, 3);
    l.ks_ih = choose_ksplit(3 * H, I, K, 128, 3);
    l.g = 0;
    l.rec = align_up((size_t)B * T * 4 * H * sizeof(float), 256);
    l.part_hh = l.rec + align_up(rec_workspace_bytes(B, H), 256);
    l.part_ih = l.part_hh + align_up(splitk_partial_floats(3 * H, H, l.ks_hh) * sizeof(float), 256);
    l.total = l.part_ih + align_up(splitk_partial_floats(3 * H, I, l.ks_ih) * sizeof(float), 256);
    return l;
}

// ------------------------------------------------------ stage profiler ---
const char* const kStageNames[RKA_NUM_STAGES] = {"input_gemm", "forward_recurrence", "backward_recurrence",
                                                 "dw_gemm", "dw_reduce", "dx_gemm"};
struct ProfRecord {
    int stage;
    hipEvent_t start, stop;
};
std::mutex g_prof_mutex;
bool g_prof_on = false;
std::vector<ProfRecord> g_prof_records;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t take_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Brackets one stage's launches with events while profiling is enabled.
class StageScope {
  public:
    StageScope(int stage, hipStream_t s) : stage_(stage), s_(s) {
        std::lock_guard<std::mutex> lock(g_prof_mutex);
        if (!g_prof_on) return;
        start_ = take_event();
        stop_ = take_event();
        if (start_ && stop_ && hipEventRecord(start_, s_) == hipSuccess) return;
        start_ = stop_ = nullptr;
    }
    ~StageScope() {
        if (!start_) return;
        std::lock_guard<std::mutex> lock(g_prof_mutex);
        if (hipEventRecord(stop_, s_) == hipSuccess) g_prof_records.push_back({stage_, start_, stop_});
    }

  private:
    int stage_;
    hipStream_t s_;
    hipEvent_t start_ = nullptr, stop_ = nullptr;
};

}  // namespace
}  // namespace rka

using namespace rka;

extern "C" {

int rka_version(void) { return 2; }

const char* rka_last_error(void) { return t_last_error.c_str(); }

int rka_device_supported(int device) {
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return 0;
    if (hipSetDevice(device) != hipSuccess) {
        set_error("invalid device " + std::to_string(device));
        return 0;
    }
    const DeviceInfo* info = nullptr;
    const int rc = current_device_info(&info);
    (void)hipSetDevice(prev);
    return rc == 0 ? 1 : 0;
}

size_t rka_gru_reserve_bytes(int batch, int seq_len, int hidden_size) {
    if (batch < 1 || seq_len < 1 || hidden_size < 1) return 0;
    return (size_t)batch * seq_len * 4 * hidden_size * sizeof(float);
}

size_t rka_gru_forward_workspace_bytes(int batch, int seq_len, int input_size, int hidden_size) {
    if (batch < 1 || seq_len < 1 || hidden_size < 1 || input_size < 1) return 0;
    return fwd_layout(batch, seq_len, input_size, hidden_size).total;
}

size_t rka_gru_backward_workspace_bytes(int batch, int seq_len, int input_size, int hidden_size) {
    if (batch < 1 || seq_len < 1 || hidden_size < 1 || input_size < 1) return 0;
    return bwd_layout(batch, seq_len, input_size, hidden_size).total;
}

size_t rka_gru_recurrence_workspace_bytes(int batch, int hidden_size) {
    if (batch < 1 || hidden_size < 1) return 0;
    return rec_workspace_bytes(batch, hidden_size);
}

int rka_gru_forward(const float* x, const float* h0, const float* w_ih, const float* w_hh,
                    const float* b_ih, const float* b_hh, float* y, float* hn, float* reserve,
                    void* workspace, size_t workspace_bytes, int batch, int seq_len, int input_size,
                    int hidden_size, void* stream) {
    clear_error();
    const int B = batch, T = seq_len, I = input_size, H = hidden_size;
    RKA_RETURN_IF_ERR(check_dims(B, T, I, H));
    if (!x || !h0 || !w_ih || !w_hh || !b_ih || !b_hh || !y || !hn)
        return fail(RKA_ERR_INVALID_ARGUMENT, "rka_gru_forward: null tensor pointer");
    const FwdLayout l = fwd_layout(B, T, I, H);
    if (!workspace || workspace_bytes < l.total)
        return fail(RKA_ERR_WORKSPACE_TOO_SMALL, "rka_gru_forward: workspace needs " + std::to_string(l.total) +
                                                     " bytes, got " + std::to_string(workspace_bytes));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    char* ws = reinterpret_cast<char*>(workspace);
    float* gx = reinterpret_cast<float*>(ws + l.gx);
    // Gx = X W_ih^T + b_ih  (both operands row-major, k = input feature)
    GemmOperand a{x, I, 0, 0, nullptr};
    GemmOperand b{w_ih, I, 0, 0, nullptr};
    // the GEMM also clears the recurrence's exchange state (slots, start-up
    // XCD words, abort flag), which saves the recurrence its fill launch
    unsigned long long* rec_state = reinterpret_cast<unsigned long long*>(ws + l.rec);
    const size_t rec_words = rec_workspace_bytes(B, H) / sizeof(unsigned long long);
    {
        StageScope scope(0, s);
        RKA_RETURN_IF_ERR(gemm_direct(B * T, 3 * H, I, a, b, b_ih, gx, 3 * H, s, SegMap{}, rec_state, rec_words));
    }
    StageScope scope(1, s);
    return launch_rec_forward(gx, h0, w_hh, b_hh, y, hn, reserve, ws + l.rec, l.total - l.rec, B, T, H, s,
                              false);
}

int rka_gru_backward(const float* x, const float* h0, const float* w_ih, const float* w_hh,
                     const float* y, const float* reserve, const float* dy, const float* dhn,
                     float* dx, float* dh0, float* dw_ih, float* dw_hh, float* db_ih, float* db_hh,
                     void* workspace, size_t workspace_bytes, int batch, int seq_len, int input_size,
                     int hidden_size, void* stream) {
    clear_error();
    const int B = batch, T = seq_len, I = input_size, H = hidden_size;
    RKA_RETURN_IF_ERR(check_dims(B, T, I, H));
    if (!x || !h0 || !w_ih || !w_hh || !y || !reserve || !dh0 || !dw_ih || !dw_hh || !db_ih || !db_hh)
        return fail(RKA_ERR_INVALID_ARGUMENT, "rka_gru_backward: null tensor pointer");
    const BwdLayout l = bwd_layout(B, T, I, H);
    if (!workspace || workspace_bytes < l.total)
        return fail(RKA_ERR_WORKSPACE_TOO_SMALL, "rka_gru_backward: workspace needs " + std::to_string(l.total) +
                                                     " bytes, got " + std::to_string(workspace_bytes));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    char* ws = reinterpret_cast<char*>(workspace);
    float* g = reinterpret_cast<float*>(ws + l.g);
    {
        StageScope scope(2, s);
        RKA_RETURN_IF_ERR(launch_rec_backward(dy, dhn, reserve, h0, y, w_hh, g, dh0, ws + l.rec,
                                              l.part_hh - l.rec, B, T, H, s));
    }
    const int K = B * T;
    // dW_hh = G_h^T Hprev, G_h = g[:, 0:3H] in (n, r, z) order -> rotate rows by H;
    // dW_ih = G_i^T X, G_i = g[:, H:4H] in (r, z, n) order.  One launch.
    {
        const SplitProduct hh{3 * H, H, K, GemmOperand{g, 4 * H, 1, 0, nullptr}, GemmOperand{y, H, 1, T, h0},
                              dw_hh, H, db_hh, H, reinterpret_cast<float*>(ws + l.part_hh), l.ks_hh};
        const SplitProduct ih{3 * H, I, K, GemmOperand{g + H, 4 * H, 1, 0, nullptr}, GemmOperand{x, I, 1, 0, nullptr},
                              dw_ih, I, db_ih, 0, reinterpret_cast<float*>(ws + l.part_ih), l.ks_ih};
        {
            StageScope scope(3, s);
            RKA_RETURN_IF_ERR(gemm_splitk_pair_partials(hh, ih, s));
        }
        if (!dx) {
            StageScope scope(4, s);
            return splitk_reduce_pair(hh, ih, s);
        }
        // dX = G_i W_ih: A(m=bt, k=j) = g[bt, H+j]; B(n=i, k=j) = W_ih[j, i].
        // One launch with the reductions, which run beside its tiles (stage
        // dx_gemm; dw_reduce stays empty).
        GemmOperand ga{g + H, 4 * H, 0, 0, nullptr};
        GemmOperand wk{w_ih, I, 1, 0, nullptr};
        StageScope scope(5, s);
        return gemm_direct_reduce_pair(K, I, 3 * H, ga, wk, dx, I, hh, ih, s);
    }
    return 0;
}

int rka_gemm_f32(int m, int n, int k, const float* a, int lda, int a_kmajor, const float* b, int ldb,
                 int b_kmajor, const float* bias, float* c, int ldc, void* stream) {
    clear_error();
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    GemmOperand ao{a, lda, a_kmajor ? 1 : 0, 0, nullptr};
    GemmOperand bo{b, ldb, b_kmajor ? 1 : 0, 0, nullptr};
    return gemm_direct(m, n, k, ao, bo, bias, c, ldc, reinterpret_cast<hipStream_t>(stream));
}

int rka_gru_recurrence_forward(const float* gx, const float* h0, const float* w_hh, const float* b_hh,
                               float* y, float* hn, float* reserve, void* workspace, size_t workspace_bytes,
                               int batch, int seq_len, int hidden_size, void* stream) {
    clear_error();
    RKA_RETURN_IF_ERR(check_dims(batch, seq_len, 1, hidden_size));
    if (!gx || !h0 || !w_hh || !b_hh || !y || !hn)
        return fail(RKA_ERR_INVALID_ARGUMENT, "rka_gru_recurrence_forward: null tensor pointer");
    return launch_rec_forward(gx, h0, w_hh, b_hh, y, hn, reserve, workspace, workspace_bytes, batch, seq_len,
                              hidden_size, reinterpret_cast<hipStream_t>(stream));
}

int rka_gru_recurrence_forward_noalloc(const float* gx, const float* h0, const float* w_hh, const float* b_hh,
                                       float* y, float* hn, float* reserve, int batch, int seq_len, int hidden_size,
                                       void* stream) {
    clear_error();
    RKA_RETURN_IF_ERR(check_dims(batch, seq_len, 1, hidden_size));
    if (!gx || !h0 || !w_hh || !b_hh || !y || !hn)
        return fail(RKA_ERR_INVALID_ARGUMENT, "rka_gru_recurrence_forward_noalloc: null tensor pointer");
    return launch_rec_forward_noalloc(gx, h0, w_hh, b_hh, y, hn, reserve, batch, seq_len, hidden_size,
                                      reinterpret_cast<hipStream_t>(stream));
}

int rka_gru_recurrence_backward(const float* dy, const float* dhn, const float* reserve, const float* h0,
                                const float* y, const float* w_hh, float* g, float* dh0, void* workspace,
                                size_t workspace_bytes, int batch, int seq_len, int hidden_size, void* stream) {
    clear_error();
    RKA_RETURN_IF_ERR(check_dims(batch, seq_len, 1, hidden_size));
    if (!reserve || !h0 || !y || !w_hh || !g || !dh0)
        return fail(RKA_ERR_INVALID_ARGUMENT, "rka_gru_recurrence_backward: null tensor pointer");
    return launch_rec_backward(dy, dhn, reserve, h0, y, w_hh, g, dh0, workspace, workspace_bytes, batch,
                               seq_len, hidden_size, reinterpret_cast<hipStream_t>(stream));
}

int rka_set_recurrence_config(int dir, int kind, int units, int param) {
    clear_error();
    if (dir != 0 && dir != 1) return fail(RKA_ERR_INVALID_ARGUMENT, "dir must be 0 or 1");
    if (kind == REC_AUTO) {
        set_rec_override(dir, 0, 0, 0);
        return 0;
    }
    const bool ok_p = param == 0 || param == 1 || param == 2 || param == 4;
    if (kind == REC_TILED) {
        if (!(units == 0 || (units > 0 && units <= 64 && (64 % units) == 0)) || !ok_p)
            return fail(RKA_ERR_INVALID_ARGUMENT, "tiled: units must divide 64, pair_waves be 1, 2 or 4 (0 = auto)");
    } else if (kind == REC_REGISTER) {
        if (!ok_p || !(units == 0 || units == 64))
            return fail(RKA_ERR_INVALID_ARGUMENT, "register: units 64 (or 0), rows 1, 2 or 4 (0 = auto)");
    } else {
        return fail(RKA_ERR_INVALID_ARGUMENT, "kind must be 0 (auto), 1 (tiled) or 2 (register)");
    }
    set_rec_override(dir, kind, units, param);
    return 0;
}

int rka_set_exchange_stores(int mode) {
    clear_error();
    if (mode != RKA_EXCHANGE_AUTO && mode != RKA_EXCHANGE_AGENT)
        return fail(RKA_ERR_INVALID_ARGUMENT, "mode must be RKA_EXCHANGE_AUTO (0) or RKA_EXCHANGE_AGENT (1)");
    set_rec_agent_stores(mode == RKA_EXCHANGE_AGENT);
    return 0;
}

int rka_set_gemm_tiles(int mode) {
    clear_error();
    return set_gemm_tiles(mode);
}

int rka_set_spin_limit(int polls) {
    clear_error();
    if (polls < 0 || polls > kMaxSpinPolls)
        return fail(RKA_ERR_INVALID_ARGUMENT, "polls must be 0 (default, 2^24) .. " + std::to_string(kMaxSpinPolls));
    set_rec_spin_limit(polls);
    return 0;
}

int rka_set_stall_block(int block) {
    clear_error();
    if (block < -1) return fail(RKA_ERR_INVALID_ARGUMENT, "block must be -1 (off) or a workgroup index");
    set_rec_stall_block(block);
    return 0;
}

int rka_recurrence_abort_count(unsigned long long* count) {
    clear_error();
    if (!count) return fail(RKA_ERR_INVALID_ARGUMENT, "rka_recurrence_abort_count: null output pointer");
    return rec_abort_count(count);
}

int rka_describe_recurrence(int dir, int batch, int hidden_size, int* out, int n_out) {
    clear_error();
    if ((dir != 0 && dir != 1) || !out || n_out < 1)
        return fail(RKA_ERR_INVALID_ARGUMENT, "dir must be 0 or 1, out non-NULL and n_out >= 1");
    RKA_RETURN_IF_ERR(check_dims(batch, 1, 1, hidden_size));
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    RecConfig c{};
    RKA_RETURN_IF_ERR(choose_rec_config(dir, batch, hidden_size, *dev, &c));
    const int v[10] = {c.kind,      c.groups, c.slices,    c.units,    c.rows,
                       c.pair_waves, c.chunk, c.lds_bytes, c.launches, c.batch_per_launch};
    for (int i = 0; i < 10 && i < n_out; ++i) out[i] = v[i];
    return 0;
}

int rka_eval_gate_functions(const float* x, float* sigmoid_out, float* tanh_out, int n, void* stream) {
    clear_error();
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    return eval_gate_functions(x, sigmoid_out, tanh_out, n, reinterpret_cast<hipStream_t>(stream));
}

int rka_profile_enable(int on) {
    clear_error();
    std::lock_guard<std::mutex> lock(g_prof_mutex);
    g_prof_on = on != 0;
    return 0;
}

int rka_profile_read(double ms_out[RKA_NUM_STAGES], int count_out[RKA_NUM_STAGES]) {
    clear_error();
    std::vector<ProfRecord> recs;
    {
        std::lock_guard<std::mutex> lock(g_prof_mutex);
        recs.swap(g_prof_records);
    }
    for (int i = 0; i < RKA_NUM_STAGES; ++i) {
        if (ms_out) ms_out[i] = 0.0;
        if (count_out) count_out[i] = 0;
    }
    int rc = 0;
    for (const ProfRecord& r : recs) {
        float ms = 0.f;
        hipError_t e = hipEventSynchronize(r.stop);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.start, r.stop);
        if (e != hipSuccess && rc == 0) rc = fail((int)e, std::string("rka_profile_read: ") + hipGetErrorString(e));
        if (e == hipSuccess && r.stage >= 0 && r.stage < RKA_NUM_STAGES) {
            if (ms_out) ms_out[r.stage] += ms;
            if (count_out) count_out[r.stage] += 1;
        }
    }
    std::lock_guard<std::mutex> lock(g_prof_mutex);
    for (const ProfRecord& r : recs) {
        g_event_pool.push_back(r.start);
        g_event_pool.push_back(r.stop);
    }
    return rc;
}

const char* rka_profile_stage_name(int stage) {
    if (stage < 0 || stage >= RKA_NUM_STAGES) return "";
    return kStageNames[stage];
}

}  // extern "C"
