// fp32 GEMMs of the GRU path on gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// One kernel template serves the four products of a layer:
//   input projection  Gx  = X W_ih^T + b_ih        (A row-major, B row-major)
//   input gradient    dX  = G_i W_ih               (A row-major, B k-major)
//   weight gradients  dW  = G^T [X | Hprev]        (A k-major,  B k-major)
// C[m,n] = sum_k A(m,k) B(n,k).  A workgroup of 4 wavefronts computes a
// 128x128 tile; each wavefront owns a 64x64 quadrant as 2x2 MFMA 32x32
// blocks.  Operand tiles of 16 (direct) or 32 (split-K) k-steps are staged
// through LDS in k-major form
// ([k][row], padded) so that the MFMA operand reads of a half-wave are 32
// consecutive floats (conflict free); the next tile (two tiles for the input
// projection) is prefetched into registers while the current one is consumed
// (double-buffered LDS, one barrier per tile).  Each operand layout is a
// template instance, so no product carries another's address arithmetic
// (c2: 4-5 % faster than one kernel with runtime layout flags).  The weight
// gradients (K = B*T rows) use split-K with a fixed-order reduction, so
// results are deterministic run to run.
#include "rka_internal.h"

namespace rka {
namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int LDSP = BM + 4;  // padded LDS row (floats); multiple of 4 for b128 stores
constexpr int NT = 256;

typedef float floatx16 __attribute__((ext_vector_type(16)));

// Address of element (row r, k) of an operand whose layout is fixed at
// compile time: KMAJOR 0 = element (r,k) at ptr[r*ld+k], 1 = at ptr[k*ld+r].
// SHIFT: the [h0 ; y[:, :-1]] row remap of the dW_hh B operand (k = b*T + t
// reads row k-1 for t > 0 and row b of shift_first for t == 0).  SEG: the
// products of one backward time chunk (SegMap rows).  Compiled per layout so
// that no product carries the others' address arithmetic or branches.
template <bool SEG>
__device__ __forceinline__ int seg_map(const SegMap& s, int i) {
    if constexpr (!SEG) return i;
    return s.len ? (i / s.len) * s.stride + s.off + i % s.len : i;
}

template <int KMAJOR, bool SHIFT, bool SEG>
__device__ __forceinline__ const float* elem_ptr(const GemmOperand& op, int r, int k) {
    if constexpr (KMAJOR == 0) {
        return op.ptr + (size_t)seg_map<SEG>(op.seg, r) * op.ld + k;
    } else {
        k = seg_map<SEG>(op.seg, k);
        if constexpr (SHIFT) {
            const int t = k % op.shift_T;
            if (t == 0) return op.shift_first + (size_t)(k / op.shift_T) * op.ld + r;
            return op.ptr + (size_t)(k - 1) * op.ld + r;
        } else {
            return op.ptr + (size_t)k * op.ld + r;
        }
    }
}

// Register staging of one BMxBK operand tile (NV4 float4 per thread).
// KMAJOR == 0: thread -> (row tid/KQ + (NT/KQ) i, k 4*(tid%KQ) .. +3), KQ = BK/4
// KMAJOR == 1: thread -> (k tid/32 + (NT/32) i, row 4*(tid%32) .. +3)
// Direct products (input projection, dx) stage 16 k per tile: three
// workgroups per CU.  Split-K weight gradients stage 32: half the barriers
// and twice the MFMA work per load round (two workgroups per CU).
constexpr int kDirectBK = 16;
constexpr int kSplitBK = 32;
static_assert(BM == 128 && BN == 128 && NT == 256, "tile staging layout");

template <int KMAJOR, bool SHIFT, bool SEG, int BK, int NV4 = BM * BK / (4 * NT), int KQ = BK / 4>
__device__ __forceinline__ void load_tile(const GemmOperand& op, bool vec, int rows, int kend, int r0, int k0,
                                          int tid, float4 (&v)[NV4]) {
    if (vec && r0 + BM <= rows && k0 + BK <= kend) {
        // interior tile of a vector-capable operand (the common case; the
        // test is uniform): no per-lane bounds checks
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            const int r = KMAJOR == 0 ? r0 + tid / KQ + (NT / KQ) * i : r0 + 4 * (tid % 32);
            const int k = KMAJOR == 0 ? k0 + 4 * (tid % KQ) : k0 + tid / 32 + (NT / 32) * i;
            v[i] = *reinterpret_cast<const float4*>(elem_ptr<KMAJOR, SHIFT, SEG>(op, r, k));
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < NV4; ++i) {
        int r, k;
        if constexpr (KMAJOR == 0) {
            r = r0 + tid / KQ + (NT / KQ) * i;
            k = k0 + 4 * (tid % KQ);
        } else {
            k = k0 + tid / 32 + (NT / 32) * i;
            r = r0 + 4 * (tid % 32);
        }
        if (vec) {
            // The contiguous extent is a multiple of 4 and rows are 16-byte
            // aligned, so a float4 is entirely in or out.
            const bool in = (r < rows) && (k < kend);
            v[i] = in ? *reinterpret_cast<const float4*>(elem_ptr<KMAJOR, SHIFT, SEG>(op, r, k))
                      : make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
            float e[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int rr = KMAJOR == 0 ? r : r + c;
                const int kk = KMAJOR == 0 ? k + c : k;
                e[c] = (rr < rows && kk < kend) ? *elem_ptr<KMAJOR, SHIFT, SEG>(op, rr, kk) : 0.f;
            }
            v[i] = make_float4(e[0], e[1], e[2], e[3]);
        }
    }
}

template <int KMAJOR, int BK, int NV4 = BM * BK / (4 * NT), int KQ = BK / 4>
__device__ __forceinline__ void store_tile(float* lds, int tid, const float4 (&v)[NV4]) {
#pragma unroll
    for (int i = 0; i < NV4; ++i) {
        if constexpr (KMAJOR == 0) {
            const int r = tid / KQ + (NT / KQ) * i;
            const int k = 4 * (tid % KQ);
            lds[(k + 0) * LDSP + r] = v[i].x;
            lds[(k + 1) * LDSP + r] = v[i].y;
            lds[(k + 2) * LDSP + r] = v[i].z;
            lds[(k + 3) * LDSP + r] = v[i].w;
        } else {
            const int k = tid / 32 + (NT / 32) * i;
            const int r = 4 * (tid % 32);
            *reinterpret_cast<float4*>(lds + k * LDSP + r) = v[i];
        }
    }
}

struct GemmArgs {
    GemmOperand a, b;
    int a_vec, b_vec;      // float4 loads allowed (extent, ld and alignment)
    int m, n, k;
    int kchunk;            // k extent per split (multiple of BK)
    const float* bias;     // direct mode
    float* c;              // direct mode output
    int ldc;
    float* partial;        // split mode: [ksplit][m][n] then colsum [ksplit][m]
    int want_colsum;
    int tiles_m, tiles;    // split mode: output tiles along m, in total
    int ksplit;            // split mode: slices of this launch
    int z_off, ksplit_total;  // split mode: first slice, slices in the buffer
    SegMap c_seg;          // direct mode: output row map
};

// Split mode runs a 1-D grid of tiles * ksplit workgroups.  Workgroups are
// dealt to the 8 XCDs round robin (XCD = id % 8); when ksplit is a multiple
// of 8, the tiles of one k-chunk are given consecutive ids on one XCD, so
// the chunk's operand rows are fetched into that XCD's L2 once and re-read
// from there by the other tiles.
__device__ __forceinline__ void split_coords(const GemmArgs& p, int& bx, int& by, int& bz) {
    const int id = blockIdx.x;
    int tile;
    if (p.ksplit % 8 == 0) {
        const int xcd = id % 8, slot = id / 8;
        bz = xcd + 8 * (slot / p.tiles);
        tile = slot % p.tiles;
    } else {
        bz = id / p.tiles;
        tile = id % p.tiles;
    }
    bx = tile % p.tiles_m;
    by = tile / p.tiles_m;
}

// MFMAs of one k-tile from LDS (as, bs) into acc; the column sum of A (the
// bias gradient) rides along for split-K products.
template <int BK>
__device__ __forceinline__ void mma_tile(const float* as, const float* bs, int lane, int wm, int wn, int tid,
                                         bool colsum, float& cs, floatx16 (&acc)[2][2]) {
    if (colsum && tid < BM) {
#pragma unroll
        for (int kk = 0; kk < BK; ++kk) cs += as[kk * LDSP + tid];
    }
    // All operand fragments of the tile are read into distinct registers
    // first: reusing one set per k-step would make every step's LDS reads
    // wait for the previous step's MFMAs to consume their operands and
    // leave the matrix core idle for an LDS latency each step.
    constexpr int KS = BK / 2;
    float fa0[KS], fa1[KS], fb0[KS], fb1[KS];
#pragma unroll
    for (int q = 0; q < KS; ++q) {
        const int row = (2 * q + (lane >> 5)) * LDSP + (lane & 31);
        fa0[q] = as[row + wm * 64];
        fa1[q] = as[row + wm * 64 + 32];
        fb0[q] = bs[row + wn * 64];
        fb1[q] = bs[row + wn * 64 + 32];
    }
    // keep the scheduler from sinking the reads back between the MFMAs
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < KS; ++q) {
        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[q], fb0[q], acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[q], fb1[q], acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[q], fb0[q], acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[q], fb1[q], acc[1][1], 0, 0, 0);
    }
}

// Interior tiles of vector-capable operands with a whole number of k-tiles
// (the input projection at the GRU's shapes): operand tiles are
// prefetched two k-tiles ahead into alternating register sets.  The loads of
// tile kb+2 are issued before the MFMAs of tile kb and stored to LDS at the
// end of iteration kb+1, so a load has two MFMA bursts (~1.7 us at BK 16) to
// arrive.  Every iteration issues the same loads (past the last tile they
// re-read it), so the wait before an LDS store covers exactly the older set.
template <int AK, int BKM, bool BSHIFT, bool SEG, int BK>
__device__ __forceinline__ void mainloop_fast(const GemmArgs& p, int m0, int n0, int kbeg, int nkb, int tid,
                                              int lane, int wm, int wn, bool colsum, float& cs,
                                              float (*As)[BK * LDSP], float (*Bs)[BK * LDSP],
                                              floatx16 (&acc)[2][2]) {
    constexpr int NV4 = BM * BK / (4 * NT);
    constexpr int KQ = BK / 4;
    // per-thread base addresses at k = kbeg; a k-tile advances them by a
    // fixed stride (the row remap of SHIFT is recomputed per tile)
    auto load = [&](float4 (&ra)[NV4], float4 (&rb)[NV4], int kb) {
        const int k0 = kbeg + min(kb, nkb - 1) * BK;
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            const int ra_r = AK == 0 ? m0 + tid / KQ + (NT / KQ) * i : m0 + 4 * (tid % 32);
            const int ra_k = AK == 0 ? k0 + 4 * (tid % KQ) : k0 + tid / 32 + (NT / 32) * i;
            ra[i] = *reinterpret_cast<const float4*>(elem_ptr<AK, false, SEG>(p.a, ra_r, ra_k));
            const int rb_r = BKM == 0 ? n0 + tid / KQ + (NT / KQ) * i : n0 + 4 * (tid % 32);
            const int rb_k = BKM == 0 ? k0 + 4 * (tid % KQ) : k0 + tid / 32 + (NT / 32) * i;
            rb[i] = *reinterpret_cast<const float4*>(elem_ptr<BKM, BSHIFT, SEG>(p.b, rb_r, rb_k));
        }
    };
    float4 ra0[NV4], rb0[NV4], ra1[NV4], rb1[NV4];
    auto step = [&](int kb, int cur, float4 (&fa)[NV4], float4 (&fb)[NV4], float4 (&na)[NV4],
                    float4 (&nb)[NV4]) {
        load(fa, fb, kb + 2);
        mma_tile<BK>(As[cur], Bs[cur], lane, wm, wn, tid, colsum, cs, acc);
        if (kb + 1 < nkb) {
            store_tile<AK, BK>(As[cur ^ 1], tid, na);
            store_tile<BKM, BK>(Bs[cur ^ 1], tid, nb);
        }
        __syncthreads();
    };
    load(ra0, rb0, 0);
    load(ra1, rb1, 1);
    store_tile<AK, BK>(As[0], tid, ra0);
    store_tile<BKM, BK>(Bs[0], tid, rb0);
    __syncthreads();
    for (int kb = 0; kb < nkb; kb += 2) {
        step(kb, 0, ra0, rb0, ra1, rb1);
        if (kb + 1 < nkb) step(kb + 1, 1, ra1, rb1, ra0, rb0);
    }
}

// Any tile (edges, unaligned or odd-extent operands): one tile of register
// prefetch, per-element bounds where needed.
template <int AK, int BKM, bool BSHIFT, bool SEG, int BK>
__device__ __forceinline__ void mainloop_general(const GemmArgs& p, int m0, int n0, int kbeg, int kend, int nkb,
                                                 int tid, int lane, int wm, int wn, bool colsum, float& cs,
                                                 float (*As)[BK * LDSP], float (*Bs)[BK * LDSP],
                                                 floatx16 (&acc)[2][2]) {
    constexpr int NV4 = BM * BK / (4 * NT);
    const bool av = p.a_vec != 0, bv = p.b_vec != 0;
    float4 ra[NV4], rb[NV4];
    if (nkb > 0) {
        load_tile<AK, false, SEG, BK>(p.a, av, p.m, kend, m0, kbeg, tid, ra);
        load_tile<BKM, BSHIFT, SEG, BK>(p.b, bv, p.n, kend, n0, kbeg, tid, rb);
        store_tile<AK, BK>(As[0], tid, ra);
        store_tile<BKM, BK>(Bs[0], tid, rb);
    }
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        const int cur = kb & 1;
        const bool more = kb + 1 < nkb;
        if (more) {
            load_tile<AK, false, SEG, BK>(p.a, av, p.m, kend, m0, kbeg + (kb + 1) * BK, tid, ra);
            load_tile<BKM, BSHIFT, SEG, BK>(p.b, bv, p.n, kend, n0, kbeg + (kb + 1) * BK, tid, rb);
        }
        mma_tile<BK>(As[cur], Bs[cur], lane, wm, wn, tid, colsum, cs, acc);
        if (more) {
            store_tile<AK, BK>(As[cur ^ 1], tid, ra);
            store_tile<BKM, BK>(Bs[cur ^ 1], tid, rb);
        }
        __syncthreads();
    }
}

template <int AK, int BKM, bool BSHIFT, bool SPLIT, bool SEG, int BK = SPLIT ? kSplitBK : kDirectBK>
__global__ __launch_bounds__(NT) void gemm_f32_kernel(GemmArgs p) {
    __shared__ __attribute__((aligned(16))) float As[2][BK * LDSP];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * LDSP];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    int bx = blockIdx.x, by = blockIdx.y, bz = 0;
    if (SPLIT) split_coords(p, bx, by, bz);
    const int m0 = bx * BM;
    const int n0 = by * BN;
    const int kbeg = bz * p.kchunk;
    const int kend = min(p.k, kbeg + p.kchunk);
    const int nkb = (kend - kbeg + BK - 1) / BK;
    const bool colsum = SPLIT && p.want_colsum && by == 0;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    float cs = 0.f;

    // The two-deep prefetch pays for the input projection (row-major A and
    // B: 141 vs 145 us at c2) but not for dx (166 vs 137 us) or the split-K
    // products (257 vs 166 us): its registers cut the resident workgroups
    // per CU from three to two (one for split-K), so only that layout uses it.
    constexpr bool kFastLayout = !SPLIT && AK == 0 && BKM == 0;
    const bool fast = kFastLayout && p.a_vec && p.b_vec && m0 + BM <= p.m && n0 + BN <= p.n && nkb > 0 &&
                      (kend - kbeg) % BK == 0;
    if constexpr (kFastLayout) {
        if (fast) {
            mainloop_fast<AK, BKM, BSHIFT, SEG, BK>(p, m0, n0, kbeg, nkb, tid, lane, wm, wn, colsum, cs, As, Bs,
                                                    acc);
        } else {
            mainloop_general<AK, BKM, BSHIFT, SEG, BK>(p, m0, n0, kbeg, kend, nkb, tid, lane, wm, wn, colsum, cs,
                                                       As, Bs, acc);
        }
    } else
        mainloop_general<AK, BKM, BSHIFT, SEG, BK>(p, m0, n0, kbeg, kend, nkb, tid, lane, wm, wn, colsum, cs, As,
                                                   Bs, acc);

    // Output layout of a 32x32 MFMA block: lane l, register r holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= p.n) continue;
            const float bias = (!SPLIT && p.bias) ? p.bias[n] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m >= p.m) continue;
                if (SPLIT) {
                    p.partial[((size_t)(p.z_off + bz) * p.m + m) * p.n + n] = acc[i][j][r];
                } else {
                    p.c[(size_t)seg_map<SEG>(p.c_seg, m) * p.ldc + n] = acc[i][j][r] + bias;
                }
            }
        }
    }
    if (colsum && tid < BM && m0 + tid < p.m) {
        float* cpart = p.partial + (size_t)p.ksplit_total * p.m * p.n;
        cpart[(size_t)(p.z_off + bz) * p.m + m0 + tid] = cs;
    }
}

// out[o*ldc + n] = sum_z partial[z][(o+rot)%m][n]; colsum likewise.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partial, int ksplit,
                                                            int m, int n, int rot, float* __restrict__ c,
                                                            int ldc, float* __restrict__ colsum) {
    const size_t total = (size_t)m * n + (colsum ? m : 0);
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        if (idx < (size_t)m * n) {
            const int o = (int)(idx / n);
            const int col = (int)(idx % n);
            const int src = rot ? (o + rot) % m : o;
            float s = 0.f;
            for (int z = 0; z < ksplit; ++z) s += partial[((size_t)z * m + src) * n + col];
            c[(size_t)o * ldc + col] = s;
        } else {
            const int o = (int)(idx - (size_t)m * n);
            const int src = rot ? (o + rot) % m : o;
            const float* cpart = partial + (size_t)ksplit * m * n;
            float s = 0.f;
            for (int z = 0; z < ksplit; ++z) s += cpart[(size_t)z * m + src];
            colsum[o] = s;
        }
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A float4 along the contiguous dimension is valid when that dimension's
// extent and the leading dimension are multiples of 4 and rows are aligned.
bool vec_ok(const GemmOperand& op, int rows, int k) {
    const int extent = op.kmajor == 0 ? k : rows;
    if (extent % 4 != 0 || op.ld % 4 != 0 || !aligned16(op.ptr)) return false;
    if (op.shift_T > 0 && !aligned16(op.shift_first)) return false;
    return true;
}

template <bool SPLIT, bool SEG>
int launch_gemm_t(const GemmArgs& args, dim3 grid, hipStream_t stream) {
    const int ak = args.a.kmajor, bk = args.b.kmajor;
    const bool shift = args.b.shift_T > 0;
    if (shift && !bk) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: the row remap needs a k-major operand");
    if (SPLIT) {
        // the weight gradients: both operands k-major
        if (!ak || !bk) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: split-K products take k-major operands");
        if (shift)
            hipLaunchKernelGGL((gemm_f32_kernel<1, 1, true, true, SEG>), grid, dim3(NT), 0, stream, args);
        else
            hipLaunchKernelGGL((gemm_f32_kernel<1, 1, false, true, SEG>), grid, dim3(NT), 0, stream, args);
    } else {
        if (shift) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: the row remap is for split-K products");
        if (!ak && !bk)
            hipLaunchKernelGGL((gemm_f32_kernel<0, 0, false, false, SEG>), grid, dim3(NT), 0, stream, args);
        else if (!ak)
            hipLaunchKernelGGL((gemm_f32_kernel<0, 1, false, false, SEG>), grid, dim3(NT), 0, stream, args);
        else if (!bk)
            hipLaunchKernelGGL((gemm_f32_kernel<1, 0, false, false, SEG>), grid, dim3(NT), 0, stream, args);
        else
            hipLaunchKernelGGL((gemm_f32_kernel<1, 1, false, false, SEG>), grid, dim3(NT), 0, stream, args);
    }
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

template <bool SPLIT>
int launch_gemm(GemmArgs args, int ksplit, bool av, bool bv, hipStream_t stream) {
    const int tm = (args.m + BM - 1) / BM, tn = (args.n + BN - 1) / BN;
    args.tiles_m = tm;
    args.tiles = tm * tn;
    args.ksplit = ksplit;
    args.a_vec = av ? 1 : 0;
    args.b_vec = bv ? 1 : 0;
    if (!SPLIT) {
        args.z_off = 0;
        args.ksplit_total = 1;
    }
    const dim3 grid = SPLIT ? dim3(tm * tn * ksplit) : dim3(tm, tn);
    const bool seg = args.a.seg.len || args.b.seg.len || args.c_seg.len;
    return seg ? launch_gemm_t<SPLIT, true>(args, grid, stream) : launch_gemm_t<SPLIT, false>(args, grid, stream);
}

}  // namespace

int gemm_direct(int m, int n, int k, const GemmOperand& a, const GemmOperand& b,
                const float* bias, float* c, int ldc, hipStream_t stream, SegMap c_seg) {
    if (m <= 0 || n <= 0 || k < 0) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: m and n must be positive");
    if (!a.ptr || !b.ptr || !c) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: null operand");
    if (m > 65535 * BM || n > 65535 * BN) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "gemm: grid too large");
    GemmArgs args{};
    args.a = a;
    args.b = b;
    args.m = m;
    args.n = n;
    args.k = k;
    args.kchunk = (k + kDirectBK - 1) / kDirectBK * kDirectBK;
    args.bias = bias;
    args.c = c;
    args.ldc = ldc;
    args.c_seg = c_seg;
    return launch_gemm<false>(args, 1, vec_ok(a, m, k), vec_ok(b, n, k), stream);
}

size_t splitk_partial_floats(int m, int n, int ksplit) {
    return (size_t)ksplit * m * n + (size_t)ksplit * m;
}

int choose_ksplit(int m, int n, int k, int num_cus, int wgs_per_cu) {
    const int tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    const int target = wgs_per_cu > 0 ? wgs_per_cu * (num_cus > 0 ? num_cus : 256) : (num_cus > 0 ? num_cus : 256) / 2;
    int ks = (target + tiles - 1) / tiles;
    const int max_by_k = k / (8 * kSplitBK);  // at least 8 tiles of k per split
    if (ks > max_by_k) ks = max_by_k;
    if (ks > 64) ks = 64;
    if (ks >= 8) ks = ks / 8 * 8;       // whole k-chunks per XCD (split_coords)
    if (ks < 1) ks = 1;
    return ks;
}

int gemm_splitk_partials(int m, int n, int k, const GemmOperand& a, const GemmOperand& b, bool want_colsum,
                         float* partial, int ksplit, int z_off, int ksplit_total, hipStream_t stream) {
    if (m <= 0 || n <= 0 || k < 0) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: m and n must be positive");
    if (ksplit < 1 || z_off < 0 || z_off + ksplit > ksplit_total)
        return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: bad split slices");
    GemmArgs args{};
    args.a = a;
    args.b = b;
    args.m = m;
    args.n = n;
    args.k = k;
    const int kper = (k + ksplit - 1) / ksplit;
    args.kchunk = (kper + kSplitBK - 1) / kSplitBK * kSplitBK;
    args.partial = partial;
    args.want_colsum = want_colsum ? 1 : 0;
    args.z_off = z_off;
    args.ksplit_total = ksplit_total;
    return launch_gemm<true>(args, ksplit, vec_ok(a, m, k), vec_ok(b, n, k), stream);
}

int splitk_reduce(int m, int n, const float* partial, int ksplit_total, int rot, float* c, int ldc,
                  float* colsum, hipStream_t stream) {
    const size_t total = (size_t)m * n + (colsum ? m : 0);
    const int blocks = (int)std::min<size_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, partial, ksplit_total, m, n,
                       rot, c, ldc, colsum);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

int gemm_splitk(int m, int n, int k, const GemmOperand& a, const GemmOperand& b,
                float* c, int ldc, float* colsum, int rot,
                float* partial, int ksplit, hipStream_t stream) {
    RKA_RETURN_IF_ERR(gemm_splitk_partials(m, n, k, a, b, colsum != nullptr, partial, ksplit, 0, ksplit, stream));
    return splitk_reduce(m, n, partial, ksplit, rot, c, ldc, colsum, stream);
}

}  // namespace rka
