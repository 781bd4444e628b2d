// fp32 GEMMs of the GRU path on gfx950 matrix cores (v_mfma_f32_16x16x4_f32).
//
// One kernel template serves the four products of a layer:
//   input projection  Gx  = X W_ih^T + b_ih        (A row-major, B row-major)
//   input gradient    dX  = G_i W_ih               (A row-major, B k-major)
//   weight gradients  dW  = G^T [X | Hprev]        (A k-major,  B k-major)
// C[m,n] = sum_k A(m,k) B(n,k).  A workgroup of 4 wavefronts computes a
// 128x128 tile; each wavefront owns a 64x64 quadrant as 4x4 MFMA 16x16
// blocks; three workgroups per CU.  Tiles of 16-byte aligned operands load
// their 16-deep operand tiles straight from global memory into a three-stage
// LDS ring (global_load_lds_dwordx4); edge tiles clamp those loads to the
// operand's last row, and a k extent that is not a multiple of 16 ends with
// one k-tile read through registers into the same ring.  Operands that are
// not 16-byte aligned stage their tiles through registers into double-
// buffered LDS (range-checked buffer loads, one float per lane, in kernel
// instances of their own).  In an edge tile, a wavefront whose 64x64
// quadrant holds no output issues no MFMAs.  The LDS
// forms are chosen so that every MFMA operand read is one conflict-free
// ds_read_b128 feeding four MFMAs: a k-major tile is kept [k][row] (a lane
// reads four rows at one k), a row-major one [row][k] (four k of one row;
// swizzled in the ring, padded in the register path), and a lane's four B
// blocks are four adjacent output columns, stored as one float4 (a
// streaming store for the direct products).  At c2 inside the training
// step: input projection 119 us, dx with the weight-gradient reductions
// 110 us, the dW pair (192x256 tiles) 233 us.  Each operand layout is a
// template instance, so no product carries another's address arithmetic.
// The weight gradients (K = B*T rows) use split-K with a fixed-order
// reduction, so results are deterministic run to run; up to 8 columns past
// their last 128-column panel are summed on the VALU instead of in a tile.
#include <atomic>

#include "rka_internal.h"

namespace rka {
namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int LDSP = BM + 4;  // padded LDS row (floats); multiple of 4 for b128 stores
constexpr int NT = 256;

typedef float floatx4 __attribute__((ext_vector_type(4)));

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

__device__ __forceinline__ const float* uniform_ptr(const float* p) {
    const unsigned long long v = reinterpret_cast<uintptr_t>(p);
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return reinterpret_cast<const float*>(((unsigned long long)hi << 32) | lo);
}

template <int KMAJOR, bool SHIFT, bool SEG>
__device__ __forceinline__ const float* elem_ptr(const GemmOperand& op, int r, int k) {
    if constexpr (KMAJOR == 0) {
        return op.ptr + (size_t)seg_map<SEG>(op.seg, r) * op.ld + k;
    } else {
        k = seg_map<SEG>(op.seg, k);
        if constexpr (SHIFT) {
            const int t = k % op.shift_T;
            if constexpr (SEG) {
                // The chunked products pick the base from the two pointers
                // read as wave-uniform values: picking between the two fields
                // made the compiler copy both into a private array indexed
                // per lane (scratch loads).
                const float* first = uniform_ptr(op.shift_first);
                const float* rest = uniform_ptr(op.ptr);
                return t == 0 ? first + (size_t)(k / op.shift_T) * op.ld + r : rest + (size_t)(k - 1) * op.ld + r;
            }
            if (t == 0) return op.shift_first + (size_t)(k / op.shift_T) * op.ld + r;
            return op.ptr + (size_t)(k - 1) * op.ld + r;
        } else {
            return op.ptr + (size_t)k * op.ld + r;
        }
    }
}

// Raw buffer loads from a wave-uniform base.  The resource spans 2^31 bytes
// and a lane given the offset kOffRange is outside it and reads zero (the
// hardware's range check), so bounds-checked loads need no exec-mask
// branches (behind which the compiler waited for each load before issuing
// the next).  In-range offsets stay below 2^31 because leading dimensions are
// below 2^22 floats (checked on the host).
constexpr unsigned kOffRange = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t range_rsrc(const float* base) {
    // word 3: the 32-bit data format (a zero format would read zero), no swizzle
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)kOffRange, 0x00020000);
}
__device__ __forceinline__ float load_in_range(const float* base, unsigned off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(range_rsrc(base), off, 0, 0));
}
typedef unsigned uintx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load4_in_range(const float* base, unsigned off) {
    // (the whole vector is cast: casting its elements one by one compiled to
    // a single dword load)
    const uintx4 u = __builtin_amdgcn_raw_buffer_load_b128(range_rsrc(base), off, 0, 0);
    const floatx4 f = __builtin_bit_cast(floatx4, u);
    return make_float4(f[0], f[1], f[2], f[3]);
}

// Register staging of one BMxBK operand tile (NV4 float4 per thread).
// KMAJOR == 0: thread -> (row tid/KQ + (NT/KQ) i, k 4*(tid%KQ) .. +3), KQ = BK/4
// KMAJOR == 1: thread -> (k tid/32 + (NT/32) i, row 4*(tid%32) .. +3)
// In both, element group i starts at a wave-uniform row and k, and a lane's
// offset from that start is the same for every i.
constexpr int kDirectBK = 16;
constexpr int kSplitBK = 16;
static_assert(BM == 128 && BN == 128 && NT == 256, "tile staging layout");

template <int KMAJOR, bool SHIFT, bool SEG, int BK, int NV4 = BM * BK / (4 * NT), int KQ = BK / 4>
__device__ __forceinline__ void load_tile(const GemmOperand& op, bool vec, int rows, int kend, int r0, int k0,
                                          int tid, float4 (&v)[NV4]) {
    if (vec && r0 + BM <= rows && k0 + BK <= kend) {
        // interior tile of a vector-capable operand (the common case; the
        // test is uniform): no per-lane bounds checks
        if constexpr (KMAJOR == 1 && SHIFT && !SEG) {
            // the [h0 ; y[:, :-1]] remap with one division per tile: the
            // thread's rows k, k + NT/32, ... advance t and wrap into the next
            // sequence at t == T
            const int kk = k0 + tid / 32;
            const int r = r0 + 4 * (tid % 32);
            int b = kk / op.shift_T;
            int t = kk - b * op.shift_T;
#pragma unroll
            for (int i = 0; i < NV4; ++i) {
                const float* src = t == 0 ? op.shift_first + (size_t)b * op.ld + r
                                          : op.ptr + (size_t)(kk + (NT / 32) * i - 1) * op.ld + r;
                v[i] = *reinterpret_cast<const float4*>(src);
                t += NT / 32;
                while (t >= op.shift_T) {
                    t -= op.shift_T;
                    ++b;
                }
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            const int r = KMAJOR == 0 ? r0 + tid / KQ + (NT / KQ) * i : r0 + 4 * (tid % 32);
            const int k = KMAJOR == 0 ? k0 + 4 * (tid % KQ) : k0 + tid / 32 + (NT / 32) * i;
            v[i] = *reinterpret_cast<const float4*>(elem_ptr<KMAJOR, SHIFT, SEG>(op, r, k));
        }
        return;
    }
    if (!vec) {
        // Operands that are not float4-aligned: one float per lane, the lanes
        // of a wave on consecutive addresses of the contiguous dimension.
        // Element x = NT (4 i + c) + tid of the tile, held in component c of
        // v[i], is row x % BM at k x / BM of a k-major tile (a wave reads 64
        // rows of one k) and row x / BK at k x % BK of a row-major one (16 k
        // of four rows).  store_tile writes it back in the same order.  (The
        // float4 order below read four floats 16 bytes apart per lane:
        // 2.3-3x slower GEMMs at hidden size 129.)
        if constexpr (!SHIFT && !SEG) {
            // Element x's address is a wave-uniform base (the element's row or
            // k offset, x / NT, is the same in every lane) plus the lane's
            // offset, which is the same for every element: one VGPR of
            // addressing instead of eight 64-bit addresses per operand.
            const int lr = KMAJOR == 1 ? tid % BM : tid / BK;  // lane's row in an element group
            const int lk = KMAJOR == 1 ? tid / BM : tid % BK;  // lane's k in an element group
            const unsigned lane_off = 4u * (KMAJOR == 1 ? lk * op.ld + lr : lr * op.ld + lk);
#pragma unroll
            for (int i = 0; i < NV4; ++i) {
                float e[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int j = 4 * i + c;
                    const int gr = KMAJOR == 1 ? r0 : r0 + (NT / BK) * j;  // group's first row
                    const int gk = KMAJOR == 1 ? k0 + (NT / BM) * j : k0;  // group's first k
                    const float* base = op.ptr + (KMAJOR == 1 ? (size_t)gk * op.ld + gr : (size_t)gr * op.ld + gk);
                    const bool in = gr + lr < rows && gk + lk < kend;
                    e[c] = load_in_range(base, in ? lane_off : kOffRange);
                }
                v[i] = make_float4(e[0], e[1], e[2], e[3]);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            float e[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int x = (4 * i + c) * NT + tid;
                const int r = r0 + (KMAJOR == 1 ? x % BM : x / BK);
                const int k = k0 + (KMAJOR == 1 ? x / BM : x % BK);
                e[c] = (r < rows && k < kend) ? *elem_ptr<KMAJOR, SHIFT, SEG>(op, r, k) : 0.f;
            }
            v[i] = make_float4(e[0], e[1], e[2], e[3]);
        }
        return;
    }
    if constexpr (!SHIFT && !SEG) {
        // edge tile of a vector-capable operand: a float4 is entirely in or
        // out (the contiguous extent is a multiple of 4)
        const int lr = KMAJOR == 0 ? tid / KQ : 4 * (tid % 32);
        const int lk = KMAJOR == 0 ? 4 * (tid % KQ) : tid / 32;
        const unsigned lane_off = 4u * (KMAJOR == 0 ? lr * op.ld + lk : lk * op.ld + lr);
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            const int gr = KMAJOR == 0 ? r0 + (NT / KQ) * i : r0;
            const int gk = KMAJOR == 0 ? k0 : k0 + (NT / 32) * i;
            const float* base = op.ptr + (KMAJOR == 0 ? (size_t)gr * op.ld + gk : (size_t)gk * op.ld + gr);
            const bool in = gr + lr < rows && gk + lk < kend;
            v[i] = load4_in_range(base, in ? lane_off : kOffRange);
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
        // The contiguous extent is a multiple of 4 and rows are 16-byte
        // aligned, so a float4 is entirely in or out.
        const bool in = (r < rows) && (k < kend);
        v[i] = in ? *reinterpret_cast<const float4*>(elem_ptr<KMAJOR, SHIFT, SEG>(op, r, k))
                  : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// LDS forms of an operand tile:
//   row form ([row][k], row stride BK + 4): one ds_read_b128 gives a lane
//     the values of four consecutive k of one row;
//   k form   ([k][row], k stride LDSP): one ds_read_b128 gives four
//     consecutive rows at one k.
// A is kept in the form of its global layout (each float4 is written whole);
// B always in k form, a row-major B being transposed on the way in.
template <int LF, int BK>
constexpr int lds_tile_floats() {
    return LF == 0 ? BM * (BK + 4) : BK * LDSP;
}

template <int GK, int LF, int BK, int NV4 = BM * BK / (4 * NT), int KQ = BK / 4>
__device__ __forceinline__ void store_tile(float* lds, int tid, bool vec, const float4 (&v)[NV4]) {
    static_assert(!(GK == 1 && LF == 0), "k-major operands are staged in k form");
    if (!vec) {
        // the element order of load_tile's one-float-per-lane path
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            const float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int x = (4 * i + c) * NT + tid;
                const int r = GK == 1 ? x % BM : x / BK;
                const int k = GK == 1 ? x / BM : x % BK;
                if constexpr (LF == 0)
                    lds[r * (BK + 4) + k] = e[c];
                else
                    lds[k * LDSP + r] = e[c];
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < NV4; ++i) {
        if constexpr (GK == 0 && LF == 0) {
            const int r = tid / KQ + (NT / KQ) * i;
            *reinterpret_cast<float4*>(lds + r * (BK + 4) + 4 * (tid % KQ)) = v[i];
        } else if constexpr (GK == 0) {
            const int r = tid / KQ + (NT / KQ) * i;
            const int k = 4 * (tid % KQ);
            lds[(k + 0) * LDSP + r] = v[i].x;
            lds[(k + 1) * LDSP + r] = v[i].y;
            lds[(k + 2) * LDSP + r] = v[i].z;
            lds[(k + 3) * LDSP + r] = v[i].w;
        } else {
            const int k = tid / 32 + (NT / 32) * i;
            *reinterpret_cast<float4*>(lds + k * LDSP + 4 * (tid % 32)) = v[i];
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
    int c_vec;             // float4 stores of C / partials allowed
    float* partial;        // split mode: [ksplit][m][n] then colsum [ksplit][m]
    int want_colsum;
    int tiles_m, tiles;    // output tiles along m, in total
    int ksplit;            // split mode: slices of this launch
    int z_off, ksplit_total;  // split mode: first slice, slices in the buffer
    SegMap c_seg;          // direct mode: output row map
    unsigned long long* zero;  // direct mode: words cleared on the side (nullable)
    size_t zero_words;
    int narrow;            // last columns left to gemm_narrow_kernel (0: none)
};

// Split mode runs a 1-D grid of tiles * ksplit workgroups.  Workgroups are
// dealt to the 8 XCDs round robin (XCD = id % 8); when ksplit is a multiple
// of 8, the tiles of one k-chunk are given consecutive ids on one XCD, so
// the chunk's operand rows are fetched into that XCD's L2 once and re-read
// from there by the other tiles.
__device__ __forceinline__ void split_coords(const GemmArgs& p, int id, int& bx, int& by, int& bz) {
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

// Direct mode runs a 1-D grid of tiles.  When the row panels divide among
// the 8 XCDs (workgroup id % 8), the N-tiles of one row panel get
// consecutive ids on one XCD, so the panel's A rows are fetched from HBM
// once and re-read from that XCD's L2 by the panel's other tiles (at c2 the
// input projection's 1536 tiles run as two resident waves, and in row-panel
// order each X panel was fetched once per wave).
__device__ __forceinline__ void direct_coords(const GemmArgs& p, int id, int& bx, int& by) {
    const int tn = p.tiles / p.tiles_m;
    if (p.tiles_m % 8 == 0) {
        const int q = id / 8;
        bx = id % 8 + 8 * (q / tn);
        by = q % tn;
        return;
    }
    bx = id % p.tiles_m;
    by = id / p.tiles_m;
}

// v_mfma_f32_16x16x4_f32: lane l supplies A[l%16][k = l/16] and
// B[k = l/16][l%16]; register r of D holds D[4 (l/16) + r][l%16].  A
// wavefront computes 64x64 as 4x4 blocks.  Within a 16-deep k slab, lane
// group g = l/16 takes k = 4 g + j at MFMA step j (the same assignment for
// both operands, so every product term appears once).  Block rows:
//   A in row form: block a, MFMA row i = tile row 16 a + i;
//   A in k form:   block a, MFMA row i = tile row 4 i + a;
//   B (k form):    block b, MFMA column c = tile column 4 c + b,
// so a lane's four B blocks are four adjacent output columns (float4 stores).
// LDS forms: 0 = row form [row][BK+4]; 1 = k form [k][KS]; 2 = the
// swizzled row form of the direct-to-LDS loads (swz_slot below, BK = 16).
// A in form 2 has the block rows of the row form; B in form 2 the block
// columns of the k form.
struct NoStep {
    __device__ void operator()() const {}
};
// `mid` runs after the tile's first MFMA step (the DMA ring issues the loads
// into the stage it frees there, once the matrix cores are busy).
template <int ALF, int BK, int KS = LDSP, int BLF = 1, typename F = NoStep>
__device__ __forceinline__ void mma_tile(const float* as, const float* bs, int lane, int wm, int wn, int tid,
                                         bool colsum, float& cs, floatx4 (&acc)[4][4], F mid = F{}) {
    static_assert((ALF != 2 && BLF != 2) || BK == 16, "swizzled row form holds 16-deep tiles");
    if constexpr (ALF == 1) {
        if (colsum && tid < BM) {
            // column sums of A (bias gradients of split-K products; A in k form)
#pragma unroll
            for (int kk = 0; kk < BK; ++kk) cs += as[kk * KS + tid];
        }
    }
    const int i = lane & 15, g = lane >> 4;
    // form 2: a lane's chunk offset within its 16-row group (rows 16 a + i of A,
    // rotated columns of B), the k quad g swizzled by bits 2..3 of i
    const int sw = 16 * i + 4 * (g ^ ((i >> 2) & 3));
    constexpr int NS = BK / 16;
    // every operand fragment of the tile first (distinct registers), so the
    // MFMAs of a slab do not wait on LDS reads issued behind earlier MFMAs
    float4 fa[NS][4], fb[NS][4];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            if constexpr (ALF == 0)
                fa[q][x] = *reinterpret_cast<const float4*>(as + (wm * 64 + 16 * x + i) * (BK + 4) + 16 * q + 4 * g);
            else if constexpr (ALF == 2)
                fa[q][x] = *reinterpret_cast<const float4*>(as + 16 * (wm * 64 + 16 * x) + sw);
            else
                fa[q][x] = *reinterpret_cast<const float4*>(as + (16 * q + 4 * g + x) * KS + wm * 64 + 4 * i);
            if constexpr (BLF == 2)
                fb[q][x] = *reinterpret_cast<const float4*>(bs + 16 * (wn * 64 + 16 * x) + sw);
            else
                fb[q][x] = *reinterpret_cast<const float4*>(bs + (16 * q + 4 * g + x) * KS + wn * 64 + 4 * i);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < NS; ++q) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                // row forms: fa[q][block a] holds steps 0..3; k form: fa[q][step j] holds blocks 0..3
                const float av = ALF != 1 ? fa[q][a][j] : fa[q][j][a];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const float bv = BLF == 2 ? fb[q][b][j] : fb[q][j][b];
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[a][b], 0, 0, 0);
                }
            }
            if (q == 0 && j == 0) {
                __builtin_amdgcn_sched_barrier(0);
                mid();
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
}

// The register-staged k loop (edge tiles, unaligned operands): the next
// k-tile is loaded into registers while the MFMAs of the current one run,
// then stored to the other LDS buffer; one barrier per k-tile.  Interior
// tiles of vector-capable operands load float4 without bounds checks; edge
// tiles check per element.  UA: the kernel instance for products with an
// operand that is not float4-aligned (a_vec / b_vec read at run time);
// otherwise both operands take the float4 loads, and the one-float-per-lane
// code, whose addresses would hold ~40 more VGPRs and cost the aligned
// kernels their third workgroup per CU, is not compiled in.
template <int AK, int BKM, bool BSHIFT, bool SEG, int BK, bool UA, bool IDLE = false>
__device__ __forceinline__ void mainloop(const GemmArgs& p, int m0, int n0, int kbeg, int kend, int nkb,
                                                 int tid, int lane, int wm, int wn, bool colsum, float& cs,
                                                 float* As0, float* As1, float* Bs0, float* Bs1,
                                                 floatx4 (&acc)[4][4]) {
    constexpr int NV4 = BM * BK / (4 * NT);
    const bool av = !UA || p.a_vec != 0, bv = !UA || p.b_vec != 0;
    float4 ra[NV4], rb[NV4];
    if (nkb > 0) {
        load_tile<AK, false, SEG, BK>(p.a, av, p.m, kend, m0, kbeg, tid, ra);
        load_tile<BKM, BSHIFT, SEG, BK>(p.b, bv, p.n, kend, n0, kbeg, tid, rb);
        store_tile<AK, AK, BK>(As0, tid, av, ra);
        store_tile<BKM, 1, BK>(Bs0, tid, bv, rb);
    }
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        float* as = (kb & 1) ? As1 : As0;
        float* bs = (kb & 1) ? Bs1 : Bs0;
        float* as_n = (kb & 1) ? As0 : As1;
        float* bs_n = (kb & 1) ? Bs0 : Bs1;
        const bool more = kb + 1 < nkb;
        if (more) {
            load_tile<AK, false, SEG, BK>(p.a, av, p.m, kend, m0, kbeg + (kb + 1) * BK, tid, ra);
            load_tile<BKM, BSHIFT, SEG, BK>(p.b, bv, p.n, kend, n0, kbeg + (kb + 1) * BK, tid, rb);
        }
        if constexpr (!IDLE) mma_tile<AK, BK>(as, bs, lane, wm, wn, tid, colsum, cs, acc);
        if (more) {
            store_tile<AK, AK, BK>(as_n, tid, av, ra);
            store_tile<BKM, 1, BK>(bs_n, tid, bv, rb);
        }
        __syncthreads();
    }
}

// Interior tiles of vector-capable operands, whole k-tiles: the operand
// tiles go from global memory straight to LDS (global_load_lds_dwordx4, 16
// bytes per lane, a wave's 64 lanes filling 1 KB of a 8 KB tile) through a
// ring of three stages, so tile kb+2 is in flight while tile kb is
// consumed, without staging registers.  One barrier per k-tile: it follows
// a wait for this wave's part of stage kb (the next stage's four loads may
// stay in flight) and precedes the loads into the stage consumed two tiles
// ago.  The barrier is the bare s_barrier (no fence): the wait covers this
// wave's loads, and every wave waits before it.
//
// The wave's 64 lanes each copy 16 bytes from src to LDS address
// M0 + 16 * lane, M0 = the wave's destination (wave-uniform).  Written as
// inline assembly so the compiler does not place a wait for every
// outstanding LDS load before each LDS read (it cannot tell the stages
// apart); the loop below waits on the vector-memory counter itself.  The
// s_nop covers the one wait state an M0 write needs before an LDS-DMA load.
// (M0 is declared clobbered; no other code of these kernels uses it, which
// the compiler's reserved-register warning cannot know.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const float* src, float* lds_dst) {
    const unsigned m0v = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_dst);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0v)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

constexpr int kDmaStages = 3;
constexpr int kDmaTile = 16 * BM;  // floats per operand tile

// Source of 16-byte chunk s (0..511) of a stage's operand tile, rows r0..,
// k k0..k0+15.  A load writes chunk s where it lands, so the LDS form is
// chosen by which global chunk each lane fetches:
//   k-major operand: k form [16][128] unpadded, chunk s = k row s/32,
//     rows 4 (s%32) .. +3;
//   row-major operand: swizzled row form, chunk s = tile row t = s/4 (for B
//     the rotated column: t = 64 (n/64) + 16 (n%4) + (n%64)/4), k quad
//     (s%4) ^ ((t/4)%4).  The 16 lanes of one ds_read_b128 (one k quad g,
//     rows 16a + i of A or columns 4i + b of B) then fall on 16 distinct
//     4-bank groups.  (rocprofv3 counts 4 bank-conflict cycles per such
//     read; a swizzle that also spreads every 8-lane group over 128 bytes
//     left that count and the run time unchanged.)
// R: rows of the tile (k form: R / 4 chunks per k row).  CLAMP (edge
// tiles): a chunk past the operand's last row reads the last row (k form:
// the last four, `rows` being a multiple of 4 there), so every load stays
// inside the operand; the products of those rows land in outputs that are
// not stored.
template <int KMAJOR, bool SHIFT, bool SEG, bool ROT, int R = BM, bool CLAMP = false>
__device__ __forceinline__ const float* dma_src(const GemmOperand& op, int r0, int k0, int s, int rows = 0) {
    if constexpr (KMAJOR == 1) {
        int r = r0 + 4 * (s % (R / 4));
        if constexpr (CLAMP) r = min(r, rows - 4);
        return elem_ptr<1, SHIFT, SEG>(op, r, k0 + s / (R / 4));
    } else {
        const int t = s >> 2;
        const int kq = (s & 3) ^ ((t >> 2) & 3);
        const int row = ROT ? (t & ~63) | ((t & 15) << 2) | ((t >> 4) & 3) : t;
        int r = r0 + row;
        if constexpr (CLAMP) r = min(r, rows - 1);
        return elem_ptr<0, false, SEG>(op, r, k0 + 4 * kq);
    }
}

// s_waitcnt vmcnt(n) with expcnt / lgkmcnt left at their maxima (gfx9
// encoding: vmcnt bits 3:0); n is wave-uniform.  n above 15 waits for
// everything (never less than asked).
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
        case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
        case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
        case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
        case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
        case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
        case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
        case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
        case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
        case 9: __builtin_amdgcn_s_waitcnt(0x0F79); break;
        case 10: __builtin_amdgcn_s_waitcnt(0x0F7A); break;
        case 11: __builtin_amdgcn_s_waitcnt(0x0F7B); break;
        case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
        case 13: __builtin_amdgcn_s_waitcnt(0x0F7D); break;
        case 14: __builtin_amdgcn_s_waitcnt(0x0F7E); break;
        case 15: __builtin_amdgcn_s_waitcnt(0x0F7F); break;
        default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    }
}

// A last k-tile of fewer than 16 (k extent or split chunk not a multiple of
// 16) takes the same ring stage and LDS form: its chunks are read with
// bounds-checked float4 loads (zero past kend) and written with
// ds_write_b128 where the DMA would have put them, so every k-tile meets
// the same MFMA code.  Edge tiles clamp their loads (dma_src).  IDLE: a
// wavefront whose 64x64 quadrant holds no output issues its share of the
// loads and the barriers but no MFMAs.
template <int AK, int BKM, bool BSHIFT, bool SEG, bool IDLE = false>
__device__ __forceinline__ void mainloop_dma(const GemmArgs& p, int m0, int n0, int kbeg, int kend, int tid, int lane,
                                             int wm, int wn, bool colsum, float& cs, float* smem,
                                             floatx4 (&acc)[4][4]) {
    const int wave = tid >> 6;
    const int nkw = (kend - kbeg) / 16;                 // whole k-tiles
    const int nkb = (kend - kbeg + 15) / 16;            // with the short last one
    auto a_stage = [&](int st) { return smem + st * 2 * kDmaTile; };
    auto b_stage = [&](int st) { return smem + st * 2 * kDmaTile + kDmaTile; };
    auto issue = [&](int kb, int st) {
        const int k0 = kbeg + kb * 16;
        if (kb < nkw) {
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                const int s0 = 64 * (2 * wave + d);  // first chunk of this wave's 1 KB block
                lds_dma16(dma_src<AK, false, SEG, false, BM, true>(p.a, m0, k0, s0 + lane, p.m),
                          a_stage(st) + 4 * s0);
                lds_dma16(dma_src<BKM, BSHIFT, SEG, true, BM, true>(p.b, n0, k0, s0 + lane, p.n),
                          b_stage(st) + 4 * s0);
            }
            return;
        }
        // the short last k-tile: chunk s of a k-major operand is k row s / 32,
        // of a row-major one k quad kq (dma_src's swizzle); a chunk past kend
        // is zero (k extents of row-major float4 operands are multiples of 4)
        float4 v[4];
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const int sc = 64 * (2 * wave + d) + lane;
            const int ka = AK == 1 ? k0 + sc / 32 : k0 + 4 * ((sc & 3) ^ ((sc >> 4) & 3));
            const int kb2 = BKM == 1 ? k0 + sc / 32 : k0 + 4 * ((sc & 3) ^ ((sc >> 4) & 3));
            v[2 * d] = ka < kend ? *reinterpret_cast<const float4*>(
                                       dma_src<AK, false, SEG, false, BM, true>(p.a, m0, k0, sc, p.m))
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
            v[2 * d + 1] = kb2 < kend ? *reinterpret_cast<const float4*>(
                                            dma_src<BKM, BSHIFT, SEG, true, BM, true>(p.b, n0, k0, sc, p.n))
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        // the ring's DMA loads are counted on the same counter: wait for all
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const int s0 = 64 * (2 * wave + d);
            *reinterpret_cast<float4*>(a_stage(st) + 4 * (s0 + lane)) = v[2 * d];
            *reinterpret_cast<float4*>(b_stage(st) + 4 * (s0 + lane)) = v[2 * d + 1];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };
    for (int kb = 0; kb < kDmaStages - 1 && kb < nkb; ++kb) issue(kb, kb);
    for (int kb = 0; kb < nkb; ++kb) {
        // this wave's four loads of stage kb are done once at most those of
        // the later stages already issued (up to kDmaStages - 2) are
        // outstanding
        wait_vmcnt(4 * min(kDmaStages - 2, nkb - 1 - kb));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        // the stage consumed at kb - 1 is free: every wave is past its reads
        // of it (the barrier).  Row-major A (the direct products): refilled
        // after this stage's first MFMA step (dx at c2: 110-112 vs 113-114
        // us); k-major A (the split-K column sums) before the MFMAs, which
        // keeps those kernels at three workgroups per CU.
        auto refill = [&]() {
            if (kb + kDmaStages - 1 < nkb) issue(kb + kDmaStages - 1, (kb + kDmaStages - 1) % kDmaStages);
        };
        if constexpr (AK == 1 || IDLE) refill();
        if constexpr (!IDLE)
            mma_tile<AK == 1 ? 1 : 2, 16, BM, BKM == 1 ? 1 : 2>(a_stage(kb % kDmaStages), b_stage(kb % kDmaStages),
                                                               lane, wm, wn, tid, colsum, cs, acc, [&]() {
                                                                   if constexpr (AK == 0) refill();
                                                               });
    }
}

// LDS floats of one workgroup: the three-stage ring or the two register-path
// buffers, whichever is larger.
template <int AK, int BK>
constexpr int gemm_smem_floats() {
    constexpr int AF = lds_tile_floats<AK, BK>();
    constexpr int BF = lds_tile_floats<1, BK>();
    return BK == 16 && kDmaStages * 2 * kDmaTile > 2 * AF + 2 * BF ? kDmaStages * 2 * kDmaTile : 2 * AF + 2 * BF;
}

// Epilogue of one output tile: acc[a][b][r] is C(row(a, 4 g + r), n0 + 64 wn
// + 4 c + b); a lane's four b values are one float4 of a C row (a partial
// row of slice bz in split mode).
template <int AK, bool SPLIT, bool SEG>
__device__ __forceinline__ void store_c(const GemmArgs& p, int m0, int n0, int bz, int wm, int wn, int lane,
                                        const floatx4 (&acc)[4][4]) {
    const int c = lane & 15, g = lane >> 4;
    const int n = n0 + wn * 64 + 4 * c;
    float4 bias4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!SPLIT && p.bias) {
        if (n + 3 < p.n) {
            bias4 = make_float4(p.bias[n], p.bias[n + 1], p.bias[n + 2], p.bias[n + 3]);
        } else {
            bias4.x = n < p.n ? p.bias[n] : 0.f;
            bias4.y = n + 1 < p.n ? p.bias[n + 1] : 0.f;
            bias4.z = n + 2 < p.n ? p.bias[n + 2] : 0.f;
        }
    }
    const bool vec_store = p.c_vec && n + 3 < p.n;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int lr = 4 * g + r;  // MFMA row within block a
            const int m = m0 + wm * 64 + (AK == 0 ? 16 * a + lr : 4 * lr + a);
            if (m >= p.m || n >= p.n) continue;
            float4 v = make_float4(acc[a][0][r], acc[a][1][r], acc[a][2][r], acc[a][3][r]);
            float* dst;
            if (SPLIT) {
                dst = p.partial + ((size_t)(p.z_off + bz) * p.m + m) * p.n + n;
            } else {
                v.x += bias4.x;
                v.y += bias4.y;
                v.z += bias4.z;
                v.w += bias4.w;
                dst = p.c + (size_t)seg_map<SEG>(p.c_seg, m) * p.ldc + n;
            }
            if (vec_store) {
                if (!SPLIT) {
                    // streaming store: C is written once and not re-read by
                    // this kernel (the output write costs ~4 us less at c2)
                    const floatx4 vv = {v.x, v.y, v.z, v.w};
                    __builtin_nontemporal_store(vv, reinterpret_cast<floatx4*>(dst));
                } else {
                    *reinterpret_cast<float4*>(dst) = v;
                }
            } else {
                dst[0] = v.x;
                if (n + 1 < p.n) dst[1] = v.y;
                if (n + 2 < p.n) dst[2] = v.z;
                if (n + 3 < p.n) dst[3] = v.w;
            }
        }
    }
}

// One output tile (bx, by) of k-chunk bz.
template <int AK, int BKM, bool BSHIFT, bool SPLIT, bool SEG, int BK, bool UA>
__device__ __forceinline__ void gemm_tile(const GemmArgs& p, int bx, int by, int bz, float* smem) {
    constexpr int AF = lds_tile_floats<AK, BK>();
    constexpr int BF = lds_tile_floats<1, BK>();
    constexpr bool kDma = BK == 16;
    float* As0 = smem;
    float* As1 = smem + AF;
    float* Bs0 = smem + 2 * AF;
    float* Bs1 = smem + 2 * AF + BF;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int m0 = bx * BM;
    const int n0 = by * BN;
    const int kbeg = bz * p.kchunk;
    const int kend = min(p.k, kbeg + p.kchunk);
    const int nkb = (kend - kbeg + BK - 1) / BK;
    const bool colsum = SPLIT && p.want_colsum && by == 0;

    floatx4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};
    float cs = 0.f;

    // an edge tile's wavefront whose 64x64 quadrant holds no output loads its
    // share of the operand tiles for the others and issues no MFMAs (its rows
    // are past p.m, so it has no column sums to store either)
    const bool idle = m0 + 64 * wm >= p.m || n0 + 64 * wn >= p.n - p.narrow;
    if (kDma && (!UA || (p.a_vec && p.b_vec))) {
        // both operands float4-capable (always so in the aligned instances)
        if (idle) {
            mainloop_dma<AK, BKM, BSHIFT, SEG, true>(p, m0, n0, kbeg, kend, tid, lane, wm, wn, false, cs, smem, acc);
            return;
        }
        mainloop_dma<AK, BKM, BSHIFT, SEG>(p, m0, n0, kbeg, kend, tid, lane, wm, wn, colsum, cs, smem, acc);
    } else {
        if (idle) {
            mainloop<AK, BKM, BSHIFT, SEG, BK, UA, true>(p, m0, n0, kbeg, kend, nkb, tid, lane, wm, wn, false, cs, As0,
                                                         As1, Bs0, Bs1, acc);
            return;
        }
        mainloop<AK, BKM, BSHIFT, SEG, BK, UA>(p, m0, n0, kbeg, kend, nkb, tid, lane, wm, wn, colsum, cs, As0, As1, Bs0,
                                           Bs1, acc);
    }
    store_c<AK, SPLIT, SEG>(p, m0, n0, bz, wm, wn, lane, acc);
    if (colsum && tid < BM && m0 + tid < p.m) {
        float* cpart = p.partial + (size_t)p.ksplit_total * p.m * p.n;
        cpart[(size_t)(p.z_off + bz) * p.m + m0 + tid] = cs;
    }
}

template <int AK, int BKM, bool BSHIFT, bool SPLIT, bool SEG, bool UA, int BK = SPLIT ? kSplitBK : kDirectBK>
__global__ __launch_bounds__(NT) void gemm_f32_kernel(GemmArgs p) {
    __shared__ __attribute__((aligned(16))) float smem[gemm_smem_floats<AK, BK>()];
    int bx, by, bz = 0;
    if (SPLIT) {
        split_coords(p, blockIdx.x, bx, by, bz);
    } else {
        direct_coords(p, blockIdx.x, bx, by);
        for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < p.zero_words; i += (size_t)gridDim.x * NT)
            p.zero[i] = 0ull;
    }
    gemm_tile<AK, BKM, BSHIFT, SPLIT, SEG, BK, UA>(p, bx, by, bz, smem);
}

// Two split-K products of k-major operands in one launch: workgroups
// [0, tiles0 * ksplit0) take the first, the rest the second (the weight
// gradients dW_hh, whose B operand is row-remapped, and dW_ih).  One launch
// of both at half the slices each keeps three workgroups per CU with half
// the partial sums and one ramp-up and tail instead of two.
template <bool SHIFT0, bool SEG, bool UA>
__global__ __launch_bounds__(NT) void gemm_f32_pair_kernel(GemmArgs p0, GemmArgs p1) {
    __shared__ __attribute__((aligned(16))) float smem[gemm_smem_floats<1, kSplitBK>()];
    const int blocks0 = p0.tiles * p0.ksplit;
    int bx, by, bz;
    if ((int)blockIdx.x < blocks0) {
        split_coords(p0, blockIdx.x, bx, by, bz);
        gemm_tile<1, 1, SHIFT0, true, SEG, kSplitBK, UA>(p0, bx, by, bz, smem);
    } else {
        split_coords(p1, blockIdx.x - blocks0, bx, by, bz);
        gemm_tile<1, 1, false, true, SEG, kSplitBK, UA>(p1, bx, by, bz, smem);
    }
}

// ------------------------------------- large-tile weight-gradient pair ---
// The two split-K weight-gradient products (both operands k-major) with
// workgroups of WMW x WNW wavefronts, each wavefront computing a 64x64
// sub-tile exactly as above (the same LDS forms and MFMA order, so every
// partial sum equals the 128x128 kernel's bit for bit): a workgroup tile is
// (64 WMW) x (64 WNW), one (tile, k-slice) item per workgroup and one
// workgroup per CU.  At c2 the 3H = 768 gate rows and the 256 columns of
// each product are four 192x256 tiles, 32 k-slices each, 256 items in all.
// A 192x256 tile loads 28 KB of operands per 16-deep stage for 1.57 MFLOP,
// against 16 KB for 0.52 MFLOP with 128x128 tiles; twelve wavefronts keep
// three per SIMD, as three 128x128 workgroups per CU do.  The operand tiles
// go straight to LDS through a ring of BigTile::D stages (five: 140 KB).
// Measured at c2 (same box, three alternating pairs): 234.5 vs 240.5 us.
// The same workgroups for the direct products (256x192 tiles for the
// input projection, 128x256 for the input gradient, one workgroup per CU)
// measured slower than three 128x128 workgroups per CU: 125 vs 120 us and
// 126 vs 110 us.
template <int WMW, int WNW>
struct BigTile {
    static constexpr int BM = 64 * WMW, BN = 64 * WNW, NW = WMW * WNW, NT = 64 * NW;
    static constexpr int ACH = BM / 16, BCH = BN / 16, CH = ACH + BCH;  // 1 KB wave loads per stage
    static constexpr int STAGE = 16 * (BM + BN);                        // floats per ring stage
    // ring stages: as many as 160 KB of LDS holds, at most 6
    static constexpr int D = 163840 / (STAGE * 4) < 6 ? 163840 / (STAGE * 4) : 6;
    static constexpr int SMEM_BYTES = D * STAGE * 4;
    static_assert(D >= 3, "the ring needs three stages");
};


// One item (split_coords(p, id)) of a split-K product of k-major operands.
template <int WMW, int WNW, bool BSHIFT>
__device__ __forceinline__ void big_split_item(const GemmArgs& p, int id, float* smem) {
    using T = BigTile<WMW, WNW>;
    constexpr int D = T::D;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WMW, wn = wave / WMW;
    const int nw = (T::CH - wave + T::NW - 1) / T::NW;  // this wave's loads per stage
    int bx, by, bz;
    split_coords(p, id, bx, by, bz);
    const int m0 = bx * T::BM, n0 = by * T::BN, kbeg = bz * p.kchunk;
    const int nkb = p.kchunk / 16;
    const bool colsum = p.want_colsum && by == 0;
    auto issue = [&](int kb) {
        const int k0 = kbeg + 16 * kb;
        float* st = smem + (kb % D) * T::STAGE;
        for (int c = wave; c < T::CH; c += T::NW) {
            if (c < T::ACH)
                lds_dma16(dma_src<1, false, false, false, T::BM>(p.a, m0, k0, 64 * c + lane), st + 256 * c);
            else
                lds_dma16(dma_src<1, BSHIFT, false, false, T::BN>(p.b, n0, k0, 64 * (c - T::ACH) + lane),
                          st + 16 * T::BM + 256 * (c - T::ACH));
        }
    };
    for (int kb = 0; kb < D - 1 && kb < nkb; ++kb) issue(kb);
    const int i = lane & 15, g = lane >> 4;
    floatx4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};
    float cs = 0.f;
    for (int kb = 0; kb < nkb; ++kb) {
        // stage kb has landed once at most the later stages already issued
        // (up to D - 2 of them, nw loads each) are outstanding
        wait_vmcnt(nw * min(D - 2, nkb - 1 - kb));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        const float* as = smem + (kb % D) * T::STAGE;
        const float* bs = as + 16 * T::BM;
        // operand fragments of this stage (the k forms and order of
        // mma_tile), then the first MFMA step, so the matrix cores start
        // before the loads into the freed stage are addressed and issued
        float4 fa[4], fb[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            fa[x] = *reinterpret_cast<const float4*>(as + (4 * g + x) * T::BM + wm * 64 + 4 * i);
            fb[x] = *reinterpret_cast<const float4*>(bs + (4 * g + x) * T::BN + wn * 64 + 4 * i);
        }
        auto mstep = [&](int j) {
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[j][a], fb[j][b], acc[a][b], 0, 0, 0);
        };
        __builtin_amdgcn_sched_barrier(0);
        mstep(0);
        __builtin_amdgcn_sched_barrier(0);
        // the stage consumed at kb - 1 is free: every wave is past its reads
        if (kb + D - 1 < nkb) issue(kb + D - 1);
        if (colsum && tid < T::BM) {
            // column sums of A (the bias gradients), in k order
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) cs += as[kk * T::BM + tid];
        }
        __builtin_amdgcn_sched_barrier(0);
        mstep(1);
        mstep(2);
        mstep(3);
    }
    store_c<1, true, false>(p, m0, n0, bz, wm, wn, lane, acc);
    if (colsum && tid < T::BM) {
        float* cpart = p.partial + (size_t)p.ksplit_total * p.m * p.n;
        cpart[(size_t)(p.z_off + bz) * p.m + m0 + tid] = cs;
    }
}

// The two weight-gradient products, one item per workgroup: items
// [0, tiles0 * ksplit0) of the first, then the second's.
template <int WMW, int WNW, bool SHIFT0>
__global__ __launch_bounds__(64 * WMW * WNW) void gemm_big_pair_kernel(GemmArgs p0, GemmArgs p1) {
    extern __shared__ __attribute__((aligned(16))) float big_smem[];
    const int items0 = p0.tiles * p0.ksplit;
    if ((int)blockIdx.x < items0)
        big_split_item<WMW, WNW, SHIFT0>(p0, blockIdx.x, big_smem);
    else
        big_split_item<WMW, WNW, false>(p1, blockIdx.x - items0, big_smem);
}

// out[o*ldc + n] = sum_z partial[z][(o+rot)%m][n]; colsum likewise.  With
// vec, a team of kTeam threads (consecutive lanes) sums one float4 of a row:
// member r takes slices r, r + kTeam, ... in order, then the team's sums are
// added as a fixed tree, so the order is the same on every run.
constexpr int kTeam = 8;
struct ReduceJob {
    const float* partial;
    int ksplit, m, n, rot;
    float* c;
    int ldc;
    float* colsum;
    int vec;
    size_t items, total;  // row items (float4 or float), then m column sums
};

__device__ __forceinline__ void reduce_item(const ReduceJob& j, size_t idx, int member) {
    const int m = j.m, n = j.n, ksplit = j.ksplit;
    if (idx < j.items) {
        const size_t per_row = j.vec ? (size_t)(n / 4) : (size_t)n;
        const int o = (int)(idx / per_row);
        const int src = j.rot ? (o + j.rot) % m : o;
        if (j.vec) {
            const int col = 4 * (int)(idx % per_row);
            const float* pp = j.partial + (size_t)src * n + col;
            float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int z = member; z < ksplit; z += kTeam) {
                const float4 v = *reinterpret_cast<const float4*>(pp + (size_t)z * m * n);
                s4.x += v.x;
                s4.y += v.y;
                s4.z += v.z;
                s4.w += v.w;
            }
#pragma unroll
            for (int off = 1; off < kTeam; off <<= 1) {
                s4.x += __shfl_xor(s4.x, off, kTeam);
                s4.y += __shfl_xor(s4.y, off, kTeam);
                s4.z += __shfl_xor(s4.z, off, kTeam);
                s4.w += __shfl_xor(s4.w, off, kTeam);
            }
            if (member == 0) *reinterpret_cast<float4*>(j.c + (size_t)o * j.ldc + col) = s4;
        } else {
            const int col = (int)(idx % per_row);
            float sum = 0.f;
            for (int z = member; z < ksplit; z += kTeam) sum += j.partial[((size_t)z * m + src) * n + col];
#pragma unroll
            for (int off = 1; off < kTeam; off <<= 1) sum += __shfl_xor(sum, off, kTeam);
            if (member == 0) j.c[(size_t)o * j.ldc + col] = sum;
        }
    } else {
        const int o = (int)(idx - j.items);
        const int src = j.rot ? (o + j.rot) % m : o;
        const float* cpart = j.partial + (size_t)ksplit * m * n;
        float sum = 0.f;
        for (int z = member; z < ksplit; z += kTeam) sum += cpart[(size_t)z * m + src];
#pragma unroll
        for (int off = 1; off < kTeam; off <<= 1) sum += __shfl_xor(sum, off, kTeam);
        if (member == 0) j.colsum[o] = sum;
    }
}

// The reductions of one or two split-K products by `blocks` workgroups of
// 256 threads (this one is number `block`): team items [0, j0.total) belong
// to the first, the rest to the second (j1.total = 0 for one product).  A
// team's idx is uniform over its kTeam lanes, so the shuffles stay within
// one job.
__device__ __forceinline__ void reduce_range(const ReduceJob& j0, const ReduceJob& j1, int block, int blocks) {
    constexpr int kTeamsPerBlock = 256 / kTeam;
    const int member = threadIdx.x % kTeam;
    const size_t teams = (size_t)blocks * kTeamsPerBlock;
    const size_t total = j0.total + j1.total;
    for (size_t idx = (size_t)block * kTeamsPerBlock + threadIdx.x / kTeam; idx < total; idx += teams) {
        if (idx < j0.total)
            reduce_item(j0, idx, member);
        else
            reduce_item(j1, idx - j0.total, member);
    }
}

__global__ __launch_bounds__(256) void splitk_reduce_kernel(ReduceJob j0, ReduceJob j1) {
    reduce_range(j0, j1, blockIdx.x, gridDim.x);
}

// A direct product (workgroups [0, p.tiles), 128x128 tiles as in
// gemm_f32_kernel) and the reductions of one or two split-K products (the
// remaining workgroups) in one launch.  The backward's input gradient and
// its weight-gradient reductions are independent: the reductions stream
// partial sums from HBM while the product keeps the matrix cores busy, on
// the workgroup slots the product's tiles leave free.
template <int AK, int BKM, bool UA>
__global__ __launch_bounds__(NT) void gemm_direct_reduce_kernel(GemmArgs p, ReduceJob j0, ReduceJob j1) {
    static_assert(NT == 256, "reduction teams assume 256-thread workgroups");
    __shared__ __attribute__((aligned(16))) float smem[gemm_smem_floats<AK, kDirectBK>()];
    if ((int)blockIdx.x >= p.tiles) {
        reduce_range(j0, j1, (int)blockIdx.x - p.tiles, (int)gridDim.x - p.tiles);
        return;
    }
    int bx, by;
    direct_coords(p, blockIdx.x, bx, by);
    gemm_tile<AK, BKM, false, false, false, kDirectBK, UA>(p, bx, by, 0, smem);
}

// ------------------------------------------------- narrow last columns ---
// A split-K product whose n is whole 128-column panels plus w <= kNarrowMax
// columns (the weight gradients at odd hidden sizes: n = H = 129) runs its
// tiles over the panels only: a tile for the last w columns would spend 128
// columns of MFMA work on w.  Those columns are summed here on the VALU, in
// a fixed order (deterministic, though not bitwise a tile's sums).  A block
// is 64 rows and four wavefronts.  Per 256-deep k slab, wavefront q sums k in
// [64q, 64q + 64) of it for its 64 rows: lanes are rows, so each k is one
// coalesced row segment of the k-major A.  At the end the four partial
// sums are added in the order q = 0..3, and each k-chunk's sums go into the
// product's partial buffer, which the reduction adds in the same fixed order
// as the tiles' partials.  Blocks [0, blocks0) take p0, the rest p1 (the
// weight-gradient pair).  The same summation for the direct products' last
// columns, run after their tiles, measured slower than the edge tiles it
// replaced (dx at hidden size 129: 101 vs 85 us).
constexpr int kNarrowMax = 8;
constexpr int kNarrowSlab = 256;  // k per LDS slab

template <bool BSHIFT>
__device__ __forceinline__ void narrow_block(const GemmArgs& p, int id, float* lds) {
    float (*bs)[kNarrowMax] = reinterpret_cast<float (*)[kNarrowMax]>(lds);  // [kNarrowSlab][8]
    float* part = lds + kNarrowSlab * kNarrowMax;                            // [4][64][8]
    const int n0 = p.n - p.narrow;
    const int mblocks = (p.m + 63) / 64;
    const int mb = id % mblocks, z = id / mblocks;
    const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
    const int m = mb * 64 + lane;
    const int kbeg = z * p.kchunk;
    const int kend = min(p.k, kbeg + p.kchunk);
    float acc[kNarrowMax];
#pragma unroll
    for (int j = 0; j < kNarrowMax; ++j) acc[j] = 0.f;
    for (int k0 = kbeg; k0 < kend; k0 += kNarrowSlab) {
        for (int i = threadIdx.x; i < kNarrowSlab * kNarrowMax; i += 256) {
            const int kk = i / kNarrowMax, j = i % kNarrowMax;
            const int k = k0 + kk;
            bs[kk][j] = (j < p.narrow && k < kend) ? *elem_ptr<1, BSHIFT, false>(p.b, n0 + j, k) : 0.f;
        }
        __syncthreads();
        const int kq = k0 + 64 * q;
        const int kn = max(0, min(64, kend - kq));
        if (m < p.m) {
            const float* a = p.a.ptr + (size_t)kq * p.a.ld + m;
#pragma unroll 8
            for (int kk = 0; kk < kn; ++kk) {
                const float av = a[(size_t)kk * p.a.ld];
#pragma unroll
                for (int j = 0; j < kNarrowMax; ++j) acc[j] = fmaf(av, bs[64 * q + kk][j], acc[j]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < kNarrowMax; ++j) part[(q * 64 + lane) * kNarrowMax + j] = acc[j];
    __syncthreads();
    if (q != 0 || m >= p.m) return;
#pragma unroll
    for (int j = 0; j < kNarrowMax; ++j) {
        if (j < p.narrow) {
            float v = part[lane * kNarrowMax + j];
            v += part[(64 + lane) * kNarrowMax + j];
            v += part[(128 + lane) * kNarrowMax + j];
            v += part[(192 + lane) * kNarrowMax + j];
            p.partial[((size_t)(p.z_off + z) * p.m + m) * p.n + n0 + j] = v;
        }
    }
}

constexpr int kNarrowSmemBytes = (kNarrowSlab + 4 * 64) * kNarrowMax * (int)sizeof(float);

template <bool BSHIFT0>
__global__ __launch_bounds__(256) void gemm_narrow_kernel(GemmArgs p0, GemmArgs p1, int blocks0) {
    __shared__ __attribute__((aligned(16))) float smem[kNarrowSmemBytes / sizeof(float)];
    const int id = (int)blockIdx.x;
    if (id < blocks0)
        narrow_block<BSHIFT0>(p0, id, smem);
    else
        narrow_block<false>(p1, id - blocks0, smem);
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

// Leading dimensions are below 2^22 floats: the bounds-checked tile loads
// address a lane's element (at most 63 ld + 15 floats from a wave-uniform
// base) with a 32-bit byte offset below 2^31.
int check_ld(const GemmOperand& a, const GemmOperand& b) {
    constexpr int kMaxLd = 1 << 22;
    if (a.ld < 0 || b.ld < 0 || a.ld >= kMaxLd || b.ld >= kMaxLd)
        return fail(RKA_ERR_UNSUPPORTED_SHAPE, "gemm: leading dimensions must be below 2^22");
    return 0;
}

// Columns of a split-K product past its last whole 128-column panel that
// gemm_narrow_kernel takes instead of a tile (0: the tiles take every column).
int narrow_cols(int n) {
    const int r = n % BN;
    return n > BN && r > 0 && r <= kNarrowMax ? r : 0;
}

// The narrow columns of the weight-gradient pair (after the tiles' launch).
int launch_narrow_pair(const GemmArgs& p0, const GemmArgs& p1, bool shift0, hipStream_t stream) {
    auto blocks = [](const GemmArgs& p) -> long long {
        return p.narrow ? (long long)((p.m + 63) / 64) * p.ksplit : 0;
    };
    const long long b0 = blocks(p0), b1 = blocks(p1);
    if (b0 + b1 == 0) return 0;
    if (b0 + b1 > 0x7fffffff) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "gemm: grid too large");
    const dim3 grid((unsigned)(b0 + b1));
    if (shift0)
        hipLaunchKernelGGL((gemm_narrow_kernel<true>), grid, dim3(256), 0, stream, p0, p1, (int)b0);
    else
        hipLaunchKernelGGL((gemm_narrow_kernel<false>), grid, dim3(256), 0, stream, p0, p1, (int)b0);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

template <int AK, int BKM, bool BSHIFT, bool SPLIT, bool SEG>
void launch_gemm_kernel(const GemmArgs& args, dim3 grid, hipStream_t stream) {
    if (args.a_vec && args.b_vec)
        hipLaunchKernelGGL((gemm_f32_kernel<AK, BKM, BSHIFT, SPLIT, SEG, false>), grid, dim3(NT), 0, stream, args);
    else
        hipLaunchKernelGGL((gemm_f32_kernel<AK, BKM, BSHIFT, SPLIT, SEG, true>), grid, dim3(NT), 0, stream, args);
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
            launch_gemm_kernel<1, 1, true, true, SEG>(args, grid, stream);
        else
            launch_gemm_kernel<1, 1, false, true, SEG>(args, grid, stream);
    } else {
        if (shift) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: the row remap is for split-K products");
        if (!ak && !bk)
            launch_gemm_kernel<0, 0, false, false, SEG>(args, grid, stream);
        else if (!ak)
            launch_gemm_kernel<0, 1, false, false, SEG>(args, grid, stream);
        else if (!bk)
            launch_gemm_kernel<1, 0, false, false, SEG>(args, grid, stream);
        else
            launch_gemm_kernel<1, 1, false, false, SEG>(args, grid, stream);
    }
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

template <bool SPLIT>
void finish_args(GemmArgs& args, int ksplit, bool av, bool bv) {
    const int tm = (args.m + BM - 1) / BM, tn = (args.n - args.narrow + BN - 1) / BN;
    args.tiles_m = tm;
    args.tiles = tm * tn;
    args.ksplit = ksplit;
    args.a_vec = av ? 1 : 0;
    args.b_vec = bv ? 1 : 0;
    if (!SPLIT) {
        args.z_off = 0;
        args.ksplit_total = 1;
    }
}

template <bool SPLIT>
int launch_gemm(GemmArgs args, int ksplit, bool av, bool bv, hipStream_t stream) {
    finish_args<SPLIT>(args, ksplit, av, bv);
    const int tm = args.tiles_m, tn = args.tiles / args.tiles_m;
    const dim3 grid(SPLIT ? tm * tn * ksplit : tm * tn);
    const bool seg = args.a.seg.len || args.b.seg.len || args.c_seg.len;
    return seg ? launch_gemm_t<SPLIT, true>(args, grid, stream) : launch_gemm_t<SPLIT, false>(args, grid, stream);
}

std::atomic<int> g_gemm_tiles{RKA_GEMM_TILES_AUTO};

}  // namespace

int set_gemm_tiles(int mode) {
    if (mode != RKA_GEMM_TILES_AUTO && mode != RKA_GEMM_TILES_128)
        return fail(RKA_ERR_INVALID_ARGUMENT, "rka_set_gemm_tiles: mode must be 0 or 1");
    g_gemm_tiles.store(mode);
    return 0;
}

int gemm_direct(int m, int n, int k, const GemmOperand& a, const GemmOperand& b,
                const float* bias, float* c, int ldc, hipStream_t stream, SegMap c_seg,
                unsigned long long* zero, size_t zero_words) {
    if (m <= 0 || n <= 0 || k < 0) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: m and n must be positive");
    if (!a.ptr || !b.ptr || !c) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: null operand");
    if ((long long)((m + BM - 1) / BM) * ((n + BN - 1) / BN) > 0x7fffffff) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "gemm: grid too large");
    RKA_RETURN_IF_ERR(check_ld(a, b));
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
    args.c_vec = (ldc % 4 == 0 && aligned16(c)) ? 1 : 0;
    args.c_seg = c_seg;
    args.zero = zero;
    args.zero_words = zero ? zero_words : 0;
    return launch_gemm<false>(args, 1, vec_ok(a, m, k), vec_ok(b, n, k), stream);
}

size_t splitk_partial_floats(int m, int n, int ksplit) {
    return (size_t)ksplit * m * n + (size_t)ksplit * m;
}

int choose_ksplit(int m, int n, int k, int num_cus, int wgs_per_cu) {
    const int tiles = ((m + BM - 1) / BM) * ((n - narrow_cols(n) + BN - 1) / BN);
    const int target = wgs_per_cu > 0 ? wgs_per_cu * (num_cus > 0 ? num_cus : 256) : (num_cus > 0 ? num_cus : 256) / 2;
    int ks = (target + tiles - 1) / tiles;
    const int max_by_k = k / (8 * kSplitBK);  // at least 8 tiles of k per split
    if (ks > max_by_k) ks = max_by_k;
    if (ks > 64) ks = 64;
    if (ks >= 8) ks = ks / 8 * 8;       // whole k-chunks per XCD (split_coords)
    if (ks < 1) ks = 1;
    return ks;
}

namespace {
int split_args(int m, int n, int k, const GemmOperand& a, const GemmOperand& b, bool want_colsum, float* partial,
               int ksplit, int z_off, int ksplit_total, bool narrow, GemmArgs* out) {
    if (m <= 0 || n <= 0 || k < 0) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: m and n must be positive");
    if (ksplit < 1 || z_off < 0 || z_off + ksplit > ksplit_total)
        return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: bad split slices");
    if (!a.kmajor || !b.kmajor) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: split-K products take k-major operands");
    RKA_RETURN_IF_ERR(check_ld(a, b));
    GemmArgs& args = *out;
    args = GemmArgs{};
    args.a = a;
    args.b = b;
    args.m = m;
    args.n = n;
    args.k = k;
    const int kper = (k + ksplit - 1) / ksplit;
    args.kchunk = (kper + kSplitBK - 1) / kSplitBK * kSplitBK;
    args.partial = partial;
    args.c_vec = (n % 4 == 0 && aligned16(partial)) ? 1 : 0;
    args.want_colsum = want_colsum ? 1 : 0;
    args.z_off = z_off;
    args.ksplit_total = ksplit_total;
    args.narrow = narrow ? narrow_cols(n) : 0;
    finish_args<true>(args, ksplit, vec_ok(a, m, k), vec_ok(b, n, k));
    return 0;
}

// The weight-gradient pair in 192x256 tiles (3H = 768 gate rows in four
// tiles, n = H or I = 256 in one), one item (tile, k-slice) per workgroup.
// Every k-slice must be whole 16-deep stages of the same length.
int try_big_pair(GemmArgs a0, GemmArgs a1, bool shift0, hipStream_t stream, bool* launched) {
    *launched = false;
    if (g_gemm_tiles.load(std::memory_order_relaxed) != RKA_GEMM_TILES_AUTO) return 0;
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    using T = BigTile<3, 4>;
    int items = 0;
    for (GemmArgs* g : {&a0, &a1}) {
        if (!g->a_vec || !g->b_vec || !g->c_vec || g->kchunk <= 0 || g->k != g->ksplit * g->kchunk) return 0;
        if (g->m % T::BM != 0 || g->n % T::BN != 0) return 0;
        g->tiles_m = g->m / T::BM;
        g->tiles = g->tiles_m * (g->n / T::BN);
        items += g->tiles * g->ksplit;
    }
    if (dev->num_cus <= 0 || items % dev->num_cus != 0) return 0;
    *launched = true;
    auto kern = shift0 ? gemm_big_pair_kernel<3, 4, true> : gemm_big_pair_kernel<3, 4, false>;
    RKA_RETURN_IF_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, T::SMEM_BYTES));
    hipLaunchKernelGGL(kern, dim3(items), dim3(T::NT), T::SMEM_BYTES, stream, a0, a1);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}
}  // namespace

int gemm_splitk_partials(int m, int n, int k, const GemmOperand& a, const GemmOperand& b, bool want_colsum,
                         float* partial, int ksplit, int z_off, int ksplit_total, hipStream_t stream) {
    GemmArgs args;
    RKA_RETURN_IF_ERR(split_args(m, n, k, a, b, want_colsum, partial, ksplit, z_off, ksplit_total, false, &args));
    return launch_gemm<true>(args, ksplit, args.a_vec != 0, args.b_vec != 0, stream);
}

int gemm_splitk_pair_partials(const SplitProduct& p0, const SplitProduct& p1, hipStream_t stream) {
    GemmArgs a0, a1;
    RKA_RETURN_IF_ERR(split_args(p0.m, p0.n, p0.k, p0.a, p0.b, p0.colsum != nullptr, p0.partial, p0.ksplit, 0,
                                 p0.ksplit, true, &a0));
    RKA_RETURN_IF_ERR(split_args(p1.m, p1.n, p1.k, p1.a, p1.b, p1.colsum != nullptr, p1.partial, p1.ksplit, 0,
                                 p1.ksplit, true, &a1));
    if (p1.b.shift_T > 0) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: only the first product of a pair is remapped");
    const bool seg = a0.a.seg.len || a0.b.seg.len || a1.a.seg.len || a1.b.seg.len;
    if (seg) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: pair products take whole operands");
    bool launched = false;
    RKA_RETURN_IF_ERR(try_big_pair(a0, a1, p0.b.shift_T > 0, stream, &launched));
    if (launched) return 0;
    const dim3 grid(a0.tiles * a0.ksplit + a1.tiles * a1.ksplit);
    const bool ua = !(a0.a_vec && a0.b_vec && a1.a_vec && a1.b_vec);
    if (p0.b.shift_T > 0) {
        if (ua)
            hipLaunchKernelGGL((gemm_f32_pair_kernel<true, false, true>), grid, dim3(NT), 0, stream, a0, a1);
        else
            hipLaunchKernelGGL((gemm_f32_pair_kernel<true, false, false>), grid, dim3(NT), 0, stream, a0, a1);
    } else {
        if (ua)
            hipLaunchKernelGGL((gemm_f32_pair_kernel<false, false, true>), grid, dim3(NT), 0, stream, a0, a1);
        else
            hipLaunchKernelGGL((gemm_f32_pair_kernel<false, false, false>), grid, dim3(NT), 0, stream, a0, a1);
    }
    RKA_RETURN_IF_HIP(hipGetLastError());
    return launch_narrow_pair(a0, a1, p0.b.shift_T > 0, stream);
}

namespace {
ReduceJob reduce_job(int m, int n, const float* partial, int ksplit_total, int rot, float* c, int ldc,
                     float* colsum) {
    ReduceJob j{};
    j.partial = partial;
    j.ksplit = ksplit_total;
    j.m = m;
    j.n = n;
    j.rot = rot;
    j.c = c;
    j.ldc = ldc;
    j.colsum = colsum;
    j.vec = (n % 4 == 0 && ldc % 4 == 0 && aligned16(partial) && aligned16(c)) ? 1 : 0;
    j.items = (size_t)m * (j.vec ? n / 4 : n);
    j.total = j.items + (colsum ? m : 0);
    return j;
}

int launch_reduce(const ReduceJob& j0, const ReduceJob& j1, hipStream_t stream) {
    const size_t total = j0.total + j1.total;
    const int blocks = (int)std::min<size_t>((total * kTeam + 255) / 256, 8192);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(std::max(blocks, 1)), dim3(256), 0, stream, j0, j1);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

ReduceJob reduce_job(const SplitProduct& p) {
    return reduce_job(p.m, p.n, p.partial, p.ksplit, p.rot, p.c, p.ldc, p.colsum);
}
}  // namespace

int splitk_reduce(const SplitProduct& p, hipStream_t stream) {
    return launch_reduce(reduce_job(p), ReduceJob{}, stream);
}

int splitk_reduce_pair(const SplitProduct& p0, const SplitProduct& p1, hipStream_t stream) {
    return launch_reduce(reduce_job(p0), reduce_job(p1), stream);
}

namespace {
template <int AK, int BKM>
void launch_direct_reduce(const GemmArgs& args, const ReduceJob& j0, const ReduceJob& j1, dim3 grid,
                          hipStream_t stream) {
    if (args.a_vec && args.b_vec)
        hipLaunchKernelGGL((gemm_direct_reduce_kernel<AK, BKM, false>), grid, dim3(NT), 0, stream, args, j0, j1);
    else
        hipLaunchKernelGGL((gemm_direct_reduce_kernel<AK, BKM, true>), grid, dim3(NT), 0, stream, args, j0, j1);
}
}  // namespace

int gemm_direct_reduce_pair(int m, int n, int k, const GemmOperand& a, const GemmOperand& b, float* c, int ldc,
                            const SplitProduct& p0, const SplitProduct& p1, hipStream_t stream) {
    if (m <= 0 || n <= 0 || k < 0) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: m and n must be positive");
    if (!a.ptr || !b.ptr || !c) return fail(RKA_ERR_INVALID_ARGUMENT, "gemm: null operand");
    RKA_RETURN_IF_ERR(check_ld(a, b));
    if (a.seg.len || b.seg.len || b.shift_T > 0) {
        RKA_RETURN_IF_ERR(splitk_reduce_pair(p0, p1, stream));
        return gemm_direct(m, n, k, a, b, nullptr, c, ldc, stream);
    }
    const DeviceInfo* dev = nullptr;
    RKA_RETURN_IF_ERR(current_device_info(&dev));
    GemmArgs args{};
    args.a = a;
    args.b = b;
    args.m = m;
    args.n = n;
    args.k = k;
    args.kchunk = (k + kDirectBK - 1) / kDirectBK * kDirectBK;
    args.c = c;
    args.ldc = ldc;
    args.c_vec = (ldc % 4 == 0 && aligned16(c)) ? 1 : 0;
    finish_args<false>(args, 1, vec_ok(a, m, k), vec_ok(b, n, k));
    // one reducing workgroup per CU: with the product's tiles at up to two
    // per CU they run beside them, in the third workgroup slot
    const long reducers = dev->num_cus > 0 ? dev->num_cus : 256;
    if ((long long)args.tiles + reducers > 0x7fffffff) return fail(RKA_ERR_UNSUPPORTED_SHAPE, "gemm: grid too large");
    const dim3 grid((unsigned)(args.tiles + reducers));
    const ReduceJob j0 = reduce_job(p0), j1 = reduce_job(p1);
    if (!a.kmajor && !b.kmajor)
        launch_direct_reduce<0, 0>(args, j0, j1, grid, stream);
    else if (!a.kmajor)
        launch_direct_reduce<0, 1>(args, j0, j1, grid, stream);
    else if (!b.kmajor)
        launch_direct_reduce<1, 0>(args, j0, j1, grid, stream);
    else
        launch_direct_reduce<1, 1>(args, j0, j1, grid, stream);
    RKA_RETURN_IF_HIP(hipGetLastError());
    return 0;
}

int splitk_reduce(int m, int n, const float* partial, int ksplit_total, int rot, float* c, int ldc,
                  float* colsum, hipStream_t stream) {
    return launch_reduce(reduce_job(m, n, partial, ksplit_total, rot, c, ldc, colsum), ReduceJob{}, stream);
}

}  // namespace rka
