/*
 * rnn_kernel_amd — C ABI of the MI355X (gfx950) fp32 GRU training path.
 *
 * Conventions for every entry point:
 *   - all pointers are device pointers owned by the caller (PyTorch's caching
 *     allocator in the Python front end); the library never allocates device
 *     memory in these calls;
 *   - work is enqueued on `stream` (a hipStream_t, NULL = default stream) and
 *     is asynchronous: no host synchronisation happens inside;
 *   - the device is the calling thread's current HIP device;
 *   - the return value is 0 on success, otherwise a nonzero code; the message
 *     of the last failure on the calling thread is rka_last_error();
 *   - tensors are dense row-major fp32: x [B,T,I], y/dy [B,T,H] (batch
 *     first), h0/hn/dh0 [B,H], W_ih [3H,I], W_hh [3H,H], biases [3H], with
 *     nn.GRU's gate order r, z, n in row blocks [0,H), [H,2H), [2H,3H).
 *
 * The reference binds its kernels from Python with cuda-python
 * (cuLaunchCooperativeKernel on raw pointers, torch's current stream);
 * each entry point below names the reference launcher it replaces.
 */
#ifndef RNN_KERNEL_AMD_H
#define RNN_KERNEL_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes (besides hipError_t values passed through). */
#define RKA_OK 0
#define RKA_ERR_INVALID_ARGUMENT 1001
#define RKA_ERR_WORKSPACE_TOO_SMALL 1002
#define RKA_ERR_UNSUPPORTED_DEVICE 1003
#define RKA_ERR_UNSUPPORTED_SHAPE 1004
#define RKA_ERR_TOO_LARGE_FOR_RESIDENT_LAUNCH 1005

/* Library ABI version. */
int rka_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* rka_last_error(void);

/* 1 if `device` is a gfx950 (MI355X-class) GPU this library was built for,
 * 0 otherwise (message in rka_last_error()).  Replaces the reference's
 * _validate_a100_device / is_a100_available capability checks
 * (src/rnn_kernel/a100/prod/gru.py:109-117,139-148). */
int rka_device_supported(int device);

/* Bytes of the per-layer gate cache ("reserve") that rka_gru_forward writes
 * in training mode and rka_gru_backward reads: [B,T,H,4] fp32, the unit's
 * (r, z, n, a_n) contiguous (one 16-byte access per unit and step).
 * Replaces the reference's gate_cache [B,T,4H] allocation
 * (src/rnn_kernel/a100/prod/gru.py:238), which keeps the four gates in
 * blocks of H; the size is the same. */
size_t rka_gru_reserve_bytes(int batch, int seq_len, int hidden_size);

/* Workspace bytes rka_gru_forward needs (input-gate buffer, exchange
 * buffers, flags). */
size_t rka_gru_forward_workspace_bytes(int batch, int seq_len, int input_size, int hidden_size);

/*
 * Forward of one GRU layer: input projection (fp32 MFMA GEMM) followed by the
 * persistent recurrence.  Writes y [B,T,H] and hn [B,H].  When `reserve` is
 * non-NULL (training) it also writes the gate cache there; when NULL
 * (inference) no cache is written.
 * Replaces F.linear + _launch_forward / _launch_forward_no_cache + the h_n
 * copy (src/rnn_kernel/a100/prod/gru.py:519-525,226-376,610-616).
 */
int rka_gru_forward(const float* x, const float* h0,
                    const float* w_ih, const float* w_hh,
                    const float* b_ih, const float* b_hh,
                    float* y, float* hn, float* reserve,
                    void* workspace, size_t workspace_bytes,
                    int batch, int seq_len, int input_size, int hidden_size,
                    void* stream);

/* Workspace bytes rka_gru_backward needs (gate-gradient buffer, exchange
 * buffers, split-K partials, flags). */
size_t rka_gru_backward_workspace_bytes(int batch, int seq_len, int input_size, int hidden_size);

/*
 * Backward of one GRU layer from the forward's y and reserve.
 * dy [B,T,H] may be NULL (zeros, gru.py:534-535); dhn [B,H] may be NULL (no
 * gradient on h_n, gru.py:552-554); dx may be NULL (input gradient not
 * needed).  Writes (does not accumulate) dx, dh0, dw_ih, dw_hh, db_ih, db_hh.
 * Replaces _launch_pack_hidden_prev + _launch_backward_sequence + the cuBLAS
 * gradient GEMMs (src/rnn_kernel/a100/prod/gru.py:531-580,379-487).
 */
int rka_gru_backward(const float* x, const float* h0,
                     const float* w_ih, const float* w_hh,
                     const float* y, const float* reserve,
                     const float* dy, const float* dhn,
                     float* dx, float* dh0,
                     float* dw_ih, float* dw_hh, float* db_ih, float* db_hh,
                     void* workspace, size_t workspace_bytes,
                     int batch, int seq_len, int input_size, int hidden_size,
                     void* stream);

/*
 * Building blocks (each is a stage of the two calls above, exported for
 * kernel-level parity tests and profiling).
 */

/* C[m,n] = sum_k A(m,k) B(n,k) (+ bias[n] if bias != NULL), fp32 MFMA.
 * A(m,k) = a[m*lda+k] if a_kmajor == 0 else a[k*lda+m];
 * B(n,k) = b[n*ldb+k] if b_kmajor == 0 else b[k*ldb+n].
 * Any alignment and leading dimension below 2^22 (else
 * RKA_ERR_UNSUPPORTED_SHAPE, nothing launched); operands whose contiguous
 * extent, leading dimension and base are multiples of 16 bytes take the
 * faster float4 paths, the others give the same results bit for bit.
 * Replaces the torch F.linear / matmul calls of gru.py:519-523,571-578. */
int rka_gemm_f32(int m, int n, int k,
                 const float* a, int lda, int a_kmajor,
                 const float* b, int ldb, int b_kmajor,
                 const float* bias, float* c, int ldc, void* stream);

/* Workspace bytes of the recurrence-only calls below. */
size_t rka_gru_recurrence_workspace_bytes(int batch, int hidden_size);

/* Persistent forward recurrence from precomputed input gates gx [B,T,3H]
 * (x W_ih^T + b_ih).  Writes y, hn and (if non-NULL) the reserve.
 * Replaces _launch_forward / _launch_forward_no_cache
 * (src/rnn_kernel/a100/prod/gru.py:226-376). */
int rka_gru_recurrence_forward(const float* gx, const float* h0,
                               const float* w_hh, const float* b_hh,
                               float* y, float* hn, float* reserve,
                               void* workspace, size_t workspace_bytes,
                               int batch, int seq_len, int hidden_size,
                               void* stream);

/* The same as rka_gru_recurrence_forward without a workspace, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  No counterpart in the
 * reference.  The exchange state lives in a static device array of the
 * library (4 MiB + 32 KiB + 256 B): it is part of the library's code
 * object, so every process that loads the library holds it on each device
 * the code object is loaded on, until the process ends, whether or not it
 * calls this entry point; the first call on a device only looks up its
 * address there.  The call allocates no device memory.  Limit: batch * hidden_size <= 262144 (2 B H 8-byte
 * words in 4 MiB); larger shapes return RKA_ERR_UNSUPPORTED_SHAPE without
 * launching; so is seq_len >= 2^24.  Every call on a GPU shares that GPU's
 * array: calls ordered on one stream are safe (each zeroes the state it uses
 * first); calls that overlap on one GPU (different streams or threads
 * without ordering) race.  Each call's exchange words carry its own call
 * number, so overlapping calls never take each other's values: they abort
 * (NaN outputs, counted by rka_recurrence_abort_count) instead. */
int rka_gru_recurrence_forward_noalloc(const float* gx, const float* h0,
                                       const float* w_hh, const float* b_hh,
                                       float* y, float* hn, float* reserve,
                                       int batch, int seq_len, int hidden_size,
                                       void* stream);

/* Persistent reverse-time recurrence.  Writes the gate gradients
 * g [B,T,4H] as blocks (da_n, dr^, dz^, dn^) and dh0.  dy / dhn may be NULL.
 * Replaces _launch_backward_sequence (src/rnn_kernel/a100/prod/gru.py:415-487),
 * whose G_i / G_h outputs are the column ranges [H,4H) and the rotation of
 * [0,3H) of g. */
int rka_gru_recurrence_backward(const float* dy, const float* dhn,
                                const float* reserve, const float* h0,
                                const float* y, const float* w_hh,
                                float* g, float* dh0,
                                void* workspace, size_t workspace_bytes,
                                int batch, int seq_len, int hidden_size,
                                void* stream);

/* GEMM tile families (for tuning and A/B tests; affects later calls on all
 * threads).  RKA_GEMM_TILES_AUTO: the weight-gradient pair of
 * rka_gru_backward runs in 192x256 tiles, one twelve-wavefront workgroup
 * per CU, when its tiles and k-slices divide evenly over the CUs (c2, c4);
 * every other product in 128x128 tiles.  RKA_GEMM_TILES_128: 128x128 tiles
 * everywhere.  The results are the same bit for bit (each output element
 * sums its k in the same order, over the same k-slices).  No counterpart in
 * the reference (its products are cuBLAS calls,
 * src/rnn_kernel/a100/prod/gru.py:569-578). */
#define RKA_GEMM_TILES_AUTO 0
#define RKA_GEMM_TILES_128 1
int rka_set_gemm_tiles(int mode);

/* Poll rounds a recurrence kernel's wait for another workgroup's words
 * makes before it gives up (0 = the default, 2^24 rounds, about 2 s at the
 * fastest poll rate; at most 2^30).  Every recurrence grid is resident, so
 * a wait lasts about one timestep unless other kernels hold the CUs it
 * needs.  A wait that gives up aborts the launch: every workgroup leaves its time loop and
 * writes NaN into every output row it did not store (y and the reserve in
 * the forward, the gate-gradient rows in the backward) and into its final
 * states (hn, dh0), so the gradients computed from them (dW, db, dx) are
 * NaN as well; every value an aborted launch leaves is either NaN or the
 * value a complete run computes.  The call itself returns 0 (the kernels
 * are asynchronous); rka_recurrence_abort_count reports the abort.
 * Affects later launches on all threads.  No counterpart in the reference
 * (its recurrence kernels step with cooperative grid barriers, which wait
 * without a bound, and it refuses a grid that cannot be resident before
 * launching, src/rnn_kernel/a100/prod/gru.py:257-263); exported so tests
 * can drive the abort path from the host. */
int rka_set_spin_limit(int polls);

/* Failure injection for tests (-1 = off, the default): in every later
 * recurrence launch, the workgroup with block index `block` publishes its
 * exchange words where its partners never look for them, so their waits
 * give up (after the rka_set_spin_limit bound) and the launch aborts, every
 * kernel still exiting normally.  Affects later launches on all threads.
 * No counterpart in the reference; exported so tests can force the abort
 * path deterministically. */
int rka_set_stall_block(int block);

/* How recurrence workgroups publish their exchange words.
 * RKA_EXCHANGE_AUTO (the default): with plain stores, which stay in the
 * XCD's L2, when a start-up check finds every workgroup of the exchange
 * group on one XCD (the grid is laid out so that they are whenever it is
 * still resident with the group count rounded up to a multiple of 8), else
 * with agent-scope stores.  RKA_EXCHANGE_AGENT: always agent-scope stores
 * (slower; the same results bit for bit).  Affects later launches on all
 * threads.  No counterpart in the reference; exported so tests cover both
 * store paths at every shape. */
#define RKA_EXCHANGE_AUTO 0
#define RKA_EXCHANGE_AGENT 1
int rka_set_exchange_stores(int mode);

/* Number of recurrence calls on the current device that aborted (a wait
 * gave up, see rka_set_spin_limit) since the library was loaded.  A call is
 * one direction of one layer (rka_gru_forward, rka_gru_backward or a
 * recurrence-only entry point), counted once however many of its launches
 * (batch slices, time ranges) aborted.  Synchronises the device first, so
 * it covers every call enqueued before.  Host code checks it at its synchronisation points; the
 * Python front end raises RuntimeError when it has grown.  No counterpart
 * in the reference (whose launches cannot abort). */
int rka_recurrence_abort_count(unsigned long long* count);

/* Override the recurrence kernel choice for direction `dir` (0 forward,
 * 1 backward); affects later calls on all threads.  For tuning and tests.
 * kind 0: automatic (register-resident kernel when hidden_size <= 256, with
 *         the fewest batch rows per workgroup whose grid is resident, else
 *         four rows and one resident launch per batch slice; LDS-tiled
 *         above 256);
 * kind 1: LDS-tiled; units = hidden units per workgroup (a divisor of 64,
 *         0 = auto), param = wavefronts holding (row, unit) pairs (1, 2, 4,
 *         0 = auto);
 * kind 2: register-resident; units = 64 (or 0), param = batch rows per
 *         workgroup (1, 2, 4, 0 = auto). */
#define RKA_REC_AUTO 0
#define RKA_REC_TILED 1
#define RKA_REC_REGISTER 2
int rka_set_recurrence_config(int dir, int kind, int units, int param);

/* Describe the decomposition the next recurrence call would use for this
 * shape: writes the first min(n_out, 10) of {kind, groups (per launch),
 * slices, units, rows_per_group, pair_waves, chunk, lds_bytes, launches,
 * batch_per_launch} to out and returns 0 (n_out < 1 is an error).  A batch
 * whose grid would not be resident on an idle GPU runs as `launches`
 * launches over consecutive slices of batch_per_launch rows, each grid
 * resident (the reference refuses such a batch instead,
 * src/rnn_kernel/a100/prod/gru.py:257-263). */
int rka_describe_recurrence(int dir, int batch, int hidden_size, int* out, int n_out);

/* Evaluates the recurrence kernels' gate nonlinearities (the same device
 * functions) elementwise: sigmoid_out = sigmoid(x), tanh_out = tanh(x).
 * For accuracy tests of those functions; no reference counterpart. */
int rka_eval_gate_functions(const float* x, float* sigmoid_out, float* tanh_out, int n, void* stream);

/*
 * Measurement of the exchange the persistent recurrences step with (for
 * bench.py's roofline; no counterpart in the reference, whose recurrences
 * step with cooperative grid barriers, a100_gru_h256_kernels.cu:698-778).
 * `pairs` pairs of workgroups (eight wavefronts each, all polling; the two
 * sides of a pair eight block ids apart, so on one XCD) ping-pong a 64-bit
 * word `iters` times: plain store to publish, agent-scope loads to poll, as
 * the recurrences do.  Writes the mean round trip in ns and whether every
 * pair ran on one XCD.  Synchronous (it waits for the device and copies the
 * timings back); every wait is bounded and one that gives up is an error.
 * The workspace is device memory of rka_exchange_probe_workspace_bytes(pairs).
 */
size_t rka_exchange_probe_workspace_bytes(int pairs);
int rka_measure_exchange_latency(int pairs, int iters, void* workspace, size_t workspace_bytes,
                                 double* round_trip_ns, int* same_xcd);

/*
 * Measurement of the issue rate of non-packed fp32 FMAs (v_fmac_f32 with
 * VGPR operands, the form of the recurrences' W_hh products; for bench.py's
 * roofline, no counterpart in the reference).  Every CU runs one or two
 * 512-thread workgroups whose lanes advance 12 or 24 independent FMA chains;
 * writes the best of the four configurations as ns per wave64 instruction
 * per SIMD and as TFLOP/s over the device.  Synchronous.  The workspace is
 * device memory of rka_fma_probe_workspace_bytes() (0 if no device).
 */
size_t rka_fma_probe_workspace_bytes(void);
int rka_measure_fma_rate(void* workspace, size_t workspace_bytes, double* ns_per_instruction, double* tflops);

/*
 * Stage profiler (the native counterpart of the reference's per-phase CUDA
 * events, rnn_benchmark.py:642-694).  While enabled, every stage launch of
 * rka_gru_forward / rka_gru_backward is bracketed by a pair of hipEvents on
 * its stream; rka_profile_read() waits for the recorded events, returns the
 * summed milliseconds and launch counts per stage and clears the records.
 * Stage ids: 0 input GEMM, 1 forward recurrence, 2 backward recurrence,
 * 3 dW_hh and dW_ih split-K products (one launch), 4 their split-K
 * reductions into dW and db, 5 dx GEMM.  When dx is requested, the
 * reductions run in the dx GEMM's launch and are reported under stage 5
 * (stage 4 then has no launches).
 */
#define RKA_NUM_STAGES 6
int rka_profile_enable(int on);
int rka_profile_read(double ms_out[RKA_NUM_STAGES], int count_out[RKA_NUM_STAGES]);
const char* rka_profile_stage_name(int stage);

/*
 * Training-step operations on either side of the GRU in the reference's
 * benchmark harness (rnn_benchmark.py:510,525,636,722): the Linear(H, 1)
 * head, the mean-squared-error loss and the AdamW update, which the
 * reference runs as PyTorch ops (nn.Linear, F.mse_loss, torch.optim.AdamW).
 * Every reduction runs in a fixed order (bitwise reproducible).
 */

/* Workspace bytes of rka_mse_forward for n elements. */
size_t rka_mse_workspace_bytes(size_t n);

/* loss[0] = sum_i (pred_i - target_i)^2 / n  (F.mse_loss, reduction 'mean',
 * rnn_benchmark.py:636). */
int rka_mse_forward(const float* pred, const float* target, float* loss, void* workspace, size_t workspace_bytes,
                    size_t n, void* stream);

/* grad_pred_i = grad_loss[0] * 2 (pred_i - target_i) / n  (its backward). */
int rka_mse_backward(const float* pred, const float* target, const float* grad_loss, float* grad_pred, size_t n,
                     void* stream);

/* pred[r] = sum_h out[r, h] w[h] + b[0] for rows r < rows of out [rows, hidden]
 * (self.head = nn.Linear(hidden_size, 1); head(out).squeeze(-1),
 * rnn_benchmark.py:510,525). */
int rka_head_forward(const float* out, const float* w, const float* b, float* pred, int rows, int hidden,
                     void* stream);

/* Workspace bytes of rka_head_backward. */
size_t rka_head_backward_workspace_bytes(int rows, int hidden);

/* dout[r, h] = dpred[r] w[h] (skipped when dout is NULL),
 * dw[h] = sum_r dpred[r] out[r, h], db[0] = sum_r dpred[r]. */
int rka_head_backward(const float* out, const float* w, const float* dpred, float* dout, float* dw, float* db,
                      void* workspace, size_t workspace_bytes, int rows, int hidden, void* stream);

/* One AdamW step (torch.optim.AdamW: decoupled weight decay, bias-corrected
 * moments; rnn_benchmark.py:722) over `count` tensors: params[i], grads[i],
 * exp_avgs[i], exp_avg_sqs[i] are device pointers of numels[i] floats; the
 * pointer arrays themselves are host memory.  `step` counts from 1.  The
 * hyper-parameters are doubles: scalars such as 1 - beta2 are formed in
 * double and rounded to fp32 once, as torch forms them from Python floats. */
int rka_adamw_step(float* const* params, const float* const* grads, float* const* exp_avgs,
                   float* const* exp_avg_sqs, const size_t* numels, int count, double lr, double beta1,
                   double beta2, double eps, double weight_decay, int step, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RNN_KERNEL_AMD_H */
