// kernels_linear.hip - dense linear layer on MFMA for bf16 / fp16 storage.
//
// y[r][o] = bias[o] + sum_c x[r][c] * W[o][c], optionally followed by SiLU
// (src/ops/sparse/trellis_sparse_cpu.c:122-171; weight [Co][Ci], :143).
// fp32 accumulation on v_mfma_f32_16x16x32_{bf16,f16}; bias and SiLU are
// applied in fp32 before the one rounding to the storage type (SiLU through
// the hardware exp2 / reciprocal instructions).
//
// A block owns a 128-row x BN-channel output tile at a time and walks its
// share of the tiles (tile lb, lb + G, ... for logical block lb of G), so the
// operand prefetch runs on from one tile into the next without a drain.  Per
// K step of 32 channels:
//  * the tile's 128 rows x 32 channels of x (8 KB) are fetched once by the
//    block, four neighbouring lanes reading one row's 64 bytes, and stored two
//    steps ahead into a 3-slot LDS ring in the bank-conflict-free a_granule
//    layout; each wavefront reads its row blocks' fragments one step ahead;
//  * each wavefront fetches its own channels' weight fragments straight into
//    registers, DEPTH steps ahead.
// 8 wavefronts = 2 row groups (4 row blocks of 16 each) x 4 channel groups.
// Weights use the grouped packing of the compacted conv (packed column
// g*WN + nt*16 + l holds channel g*WN + l*NT + nt), so a lane's results for a
// row are NT adjacent channels; a finished tile is staged in LDS and stored
// in whole 16-byte chunks.
#include "tsh_internal.h"
#include "mfma_common.h"

namespace tsh {
namespace {

template <int DT, int BN, int UPB, int DEPTH>
__global__ void __launch_bounds__(512) k_linear_mfma(const typename Store<DT>::T * __restrict__ x,
                                                     const typename Store<DT>::T * __restrict__ w16,
                                                     const float * __restrict__ bias,
                                                     typename Store<DT>::T * __restrict__ y, int64_t n, int ci,
                                                     int co, int n_col_tiles, int n_tiles, int silu) {
    using T = typename Store<DT>::T;
    using V = typename Mfma<DT>::V;
    constexpr int NTHR = 512;
    constexpr int BM = 128;          // rows per tile
    constexpr int BK = 32;           // input channels per K step
    constexpr int RG = 2;            // row groups
    constexpr int CG = 4;            // channel groups
    constexpr int WN = BN / CG;      // channels per wavefront
    constexpr int NT = WN / 16;      // MFMA column tiles per wavefront
    constexpr int QB = 8 / RG;       // row blocks per wavefront
    constexpr int SPU = DEPTH / UPB; // steps per tile when a block holds UPB tiles
    static_assert(NT >= 1 && WN % 16 == 0, "channel groups of whole 16-column tiles");
    static_assert((UPB == 1 || UPB == 2 || UPB == 4) && (DEPTH == 4 || DEPTH == 8) && SPU >= 2, "step blocks");
    constexpr int CHUNKS = BN / 8;       // 16-byte chunks per output row of the tile
    constexpr int OSTRIDE = BN + 8;      // staged row stride (elements): rows 4 apart land 64 bytes apart in the banks
    static_assert(BM * CHUNKS % NTHR == 0, "whole store passes");
    __shared__ __attribute__((aligned(16))) T s_a[3][BM * BK];
    __shared__ __attribute__((aligned(16))) T s_out[BM * OSTRIDE];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int rh = wave % RG, ch = wave / RG;
    const int l16 = lane & 15, lg = lane >> 4;
    const int G = (int) gridDim.x;
    const int lb = (int) xcd_remap(blockIdx.x, G);
    const int U = (n_tiles - lb + G - 1) / G;  // tiles of this block (>= 1: G <= n_tiles)
    const int KS = ci / BK;

    // This thread's x piece: row arow of the tile, 16-byte chunk achunk.
    const int arow = (t >> 6) * 16 + a_quad_row((t >> 2) & 15), achunk = t & 3;
    const int a_st = ((t >> 6) * 64 + a_granule(arow & 15, achunk)) * 8;
    const int a_ld = (rh * 64 + a_granule(l16, lg)) * 8;
    constexpr int A_QSTRIDE = RG * 64 * 8;
    const int64_t bstep = (int64_t) 4 * co * 8;  // elements between consecutive K steps' weights
    const int64_t blane = ((int64_t) lg * co + ch * WN + l16) * 8;

    // Operand addresses of the next block of DEPTH steps: tile tu + r / SPU,
    // K step tps + r % SPU for step r (past the last tile: the last again).
    const T * pa[UPB];
    const T * pb[UPB];
    auto tile_of = [&](int u) -> int { return lb + (u < U ? u : U - 1) * G; };
    auto target = [&](int tu0, int tps) {
#pragma unroll
        for (int uo = 0; uo < UPB; ++uo) {
            const int tile = tile_of(tu0 + uo);
            const int rt = tile / n_col_tiles;
            const int ct = tile - rt * n_col_tiles;
            int64_t row = (int64_t) rt * BM + arow;
            row = row < n ? row : n - 1;  // rows past the end read the last row; never stored
            pa[uo] = x + row * ci + tps * BK + achunk * 8;
            pb[uo] = w16 + ((int64_t) tps * 4 * co + (int64_t) ct * BN) * 8 + blane;
        }
    };
    auto load_a = [&](V & a, int r) { a = *(const V *) (pa[r / SPU] + (r % SPU) * BK); };
    auto load_b = [&](V * b, int r) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) b[nt] = *(const V *) (pb[r / SPU] + (r % SPU) * bstep + nt * 16 * 8);
    };
    auto store_a = [&](int slot, const V & a) { *(V *) (&s_a[slot][a_st]) = a; };
    auto read_a = [&](V * f, int slot) {
#pragma unroll
        for (int q = 0; q < QB; ++q) f[q] = *(const V *) (&s_a[slot][a_ld + q * A_QSTRIDE]);
    };

    V ra[DEPTH];      // x pieces in flight
    V rb[DEPTH][NT];  // weights of the block's steps (refilled with the next block's)
    V af[2][QB];      // x fragments of step g in af[g & 1]
    f32x4 acc[QB][NT];
#pragma unroll
    for (int q = 0; q < QB; ++q)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Epilogue of tile u: bias, SiLU and the one rounding in registers; the
    // tile is then staged in LDS and leaves as whole 16-byte chunks (the lanes'
    // own results are only NT adjacent channels, and stores that narrow halve
    // the write bandwidth).  The accumulators restart at zero.
    auto finish = [&](int u) {
        using Out = T __attribute__((ext_vector_type(NT)));
        const int tile = tile_of(u);
        const int rt = tile / n_col_tiles;
        const int ct = tile - rt * n_col_tiles;
        const int c0 = ch * WN + l16 * NT;  // channel within the tile
        float bv[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) bv[nt] = bias != nullptr ? bias[ct * BN + c0 + nt] : 0.0f;
#pragma unroll
        for (int q = 0; q < QB; ++q) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = (rh + RG * q) * 16 + lg * 4 + i;
                Out o;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    float v = acc[q][nt][i] + bv[nt];
                    // Hardware exp2 and reciprocal (about 1 ulp each), far
                    // inside the 16-bit storage rounding.
                    if (silu) v = v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
                    if constexpr (DT == kBF16) {
                        o[nt] = __builtin_bit_cast(uint16_t, (__bf16) v);  // v_cvt_pk_bf16_f32, RNE
                    } else {
                        o[nt] = (T) v;
                    }
                }
                *(Out *) (&s_out[r * OSTRIDE + c0]) = o;
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        lds_barrier();
        // Row r's chunks are read rotated by r, so each group of 16 lanes
        // touches every bank granule once; together they still write the
        // row's whole span.
#pragma unroll
        for (int p = 0; p < BM * CHUNKS / NTHR; ++p) {
            const int e = t + p * NTHR;
            const int r = e / CHUNKS;
            const int j = (e + r) % CHUNKS;
            const int64_t row = (int64_t) rt * BM + r;
            const int4 v = *(const int4 *) (&s_out[r * OSTRIDE + j * 8]);
            if (row < n) *(int4 *) (y + row * co + ct * BN + j * 8) = v;
        }
    };

    // Block 0: x of steps 0 and 1 straight into LDS slots 0 and 1, steps 2 ..
    // DEPTH-1 into ring slots 2 .. DEPTH-1; weights of steps 0 .. DEPTH-1.
    target(0, 0);
    load_a(ra[0], 0);
    store_a(0, ra[0]);
    load_a(ra[1], 1);
    store_a(1, ra[1]);
#pragma unroll
    for (int r = 2; r < DEPTH; ++r) load_a(ra[r], r);
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) load_b(rb[r], r);
    lds_barrier();
    read_a(af[0], 0);

    int aslot = 0;  // LDS slot of the current step's x (step g: g % 3)
    for (int cb = 0; cb < U; cb += UPB) {
        int s0 = 0;
        do {
            if constexpr (UPB == 1) {
                const bool last = s0 + DEPTH >= KS;
                target(last ? cb + 1 : cb, last ? 0 : s0 + DEPTH);
            } else {
                target(cb + UPB, 0);
            }
#pragma unroll
            for (int r = 0; r < DEPTH; ++r) {
                const int s1 = aslot == 2 ? 0 : aslot + 1;  // next step's x
                const int s2 = s1 == 2 ? 0 : s1 + 1;        // step after: held step g-1
                // Fragments of the next step and x of step g + 2 into the slot
                // every wavefront finished reading before the last barrier,
                // both issued ahead of the MFMAs.
                read_a(af[(r + 1) & 1], s1);
                store_a(s2, ra[(r + 2) % DEPTH]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < QB; ++q)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        acc[q][nt] = Mfma<DT>::mac(af[r & 1][q], rb[r][nt], acc[q][nt]);
                load_a(ra[r], r);
                load_b(rb[r], r);
                aslot = s1;
                lds_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (UPB > 1) {
                    // A tile ends inside the block; a tile past the last one
                    // (odd tile count) multiplied repeated data and is dropped.
                    if (r % SPU == SPU - 1) {
                        if (cb + r / SPU < U) {
                            finish(cb + r / SPU);
                        } else {
#pragma unroll
                            for (int q = 0; q < QB; ++q)
#pragma unroll
                                for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
                        }
                    }
                }
            }
            s0 += DEPTH;
        } while (s0 < KS);
        if constexpr (UPB == 1) finish(cb);
    }
}

template <int DT, int BN, int UPB, int DEPTH>
hipError_t launch_linear_t(const void * x, const void * w16, const float * bias, void * y, int64_t n, int ci, int co,
                           int silu, int cus, hipStream_t s) {
    using T = typename Store<DT>::T;
    const int64_t row_tiles = (n + 127) / 128;
    const int64_t col_tiles = co / BN;
    const int64_t tiles = row_tiles * col_tiles;
    // One resident block per CU (512 threads; the register ring allows two
    // wavefronts per SIMD); each walks every G-th tile.
    if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
    const int64_t grid = tiles < cus ? tiles : cus;
    k_linear_mfma<DT, BN, UPB, DEPTH><<<(unsigned) grid, 512, 0, s>>>(
        (const T *) x, (const T *) w16, bias, (T *) y, n, ci, co, (int) col_tiles, (int) tiles, silu);
    return hipGetLastError();
}

template <int DT>
hipError_t launch_linear_dt(const void * x, const void * w16, const float * bias, void * y, int64_t n, int ci, int co,
                            int silu, int cus, hipStream_t s) {
    // Blocks of 8 steps (64 KB of x in flight per CU) when a tile is a whole
    // number of them (Ci % 256 == 0), else 4; Ci = 64 puts two 2-step tiles in
    // a block.
#define TSH_LINEAR(BNV)                                                                                     \
    do {                                                                                                    \
        if (ci == 64) return launch_linear_t<DT, BNV, 2, 4>(x, w16, bias, y, n, ci, co, silu, cus, s);      \
        if (ci % 256 == 0) return launch_linear_t<DT, BNV, 1, 8>(x, w16, bias, y, n, ci, co, silu, cus, s); \
        return launch_linear_t<DT, BNV, 1, 4>(x, w16, bias, y, n, ci, co, silu, cus, s);                    \
    } while (0)
    if (co % 128 == 0) TSH_LINEAR(128);
    TSH_LINEAR(64);
#undef TSH_LINEAR
}
// Narrow outputs (Co <= 16: the subdivide logits, Ci -> 8): one wavefront
// per 16-row block at a time.  The block's KS A fragments come straight from
// the rows (four lanes per 64-byte segment), all loads issued before the
// MFMAs; the B fragments are the [co][ci] weights' rows read from cache (the
// columns past Co are zero); bias and SiLU in fp32; lanes of the Co valid
// columns store.
template <int DT, int KS>
__global__ void __launch_bounds__(256) k_linear_narrow(const typename Store<DT>::T * __restrict__ x,
                                                       const typename Store<DT>::T * __restrict__ w,
                                                       const float * __restrict__ bias,
                                                       typename Store<DT>::T * __restrict__ y, int64_t n, int co,
                                                       int silu) {
    using V = typename Mfma<DT>::V;
    constexpr int CI = KS * 32;
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15, lg = lane >> 4;
    const int64_t waves = (int64_t) gridDim.x * (blockDim.x >> 6);
    const int64_t wid = (int64_t) blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const bool colok = l16 < co;
    V b[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) b[s] = colok ? *(const V *) (w + (int64_t) l16 * CI + s * 32 + lg * 8) : V{};
    const float bv = (colok && bias != nullptr) ? bias[l16] : 0.0f;
    const int64_t blocks16 = (n + 15) / 16;
    for (int64_t rb = wid; rb < blocks16; rb += waves) {
        const int64_t row = rb * 16 + l16;
        V a[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) a[s] = row < n ? *(const V *) (x + row * CI + s * 32 + lg * 8) : V{};
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) acc = Mfma<DT>::mac(a[s], b[s], acc);
        if (colok) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t r = rb * 16 + lg * 4 + i;
                float v = acc[i] + bv;
                if (silu) v = v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
                if (r < n) Store<DT>::st_signed(y, r * co + l16, v);
            }
        }
    }
}

template <int DT>
hipError_t launch_narrow_dt(const void * x, const void * w16, const float * bias, void * y, int64_t n, int ci, int co,
                            int silu, int cus, hipStream_t s) {
    using T = typename Store<DT>::T;
    const int64_t blocks16 = (n + 15) / 16;
    int64_t grid = (blocks16 + 3) / 4;
    if (grid > (int64_t) cus * 16) grid = (int64_t) cus * 16;
    if (grid < 1) grid = 1;
#define TSH_NARROW(KSV)                                                                                          \
    k_linear_narrow<DT, KSV><<<(unsigned) grid, 256, 0, s>>>((const T *) x, (const T *) w16, bias, (T *) y, n, co, \
                                                            silu)
    switch (ci) {
        case 32: TSH_NARROW(1); break;
        case 64: TSH_NARROW(2); break;
        case 128: TSH_NARROW(4); break;
        case 256: TSH_NARROW(8); break;
        case 512: TSH_NARROW(16); break;
        default: TSH_NARROW(32); break;
    }
#undef TSH_NARROW
    return hipGetLastError();
}
}  // namespace

bool linear_narrow_supported(int dtype, int ci, int co) {
    return (dtype == kF16 || dtype == kBF16) && co >= 1 && co <= 16 &&
           (ci == 32 || ci == 64 || ci == 128 || ci == 256 || ci == 512 || ci == 1024);
}

hipError_t launch_linear_narrow(int dtype, const void * x, const void * w16, const float * bias, void * y, int64_t n,
                                int ci, int co, int silu, int cus, hipStream_t s) {
    if (!linear_narrow_supported(dtype, ci, co) || n <= 0 || cus <= 0) return hipErrorInvalidValue;
    if (dtype == kBF16) return launch_narrow_dt<kBF16>(x, w16, bias, y, n, ci, co, silu, cus, s);
    return launch_narrow_dt<kF16>(x, w16, bias, y, n, ci, co, silu, cus, s);
}

int linear_mfma_group(int co) { return (co % 128 == 0 ? 128 : 64) / 4 / 16; }

bool linear_mfma_supported(int dtype, int ci, int co) {
    return (dtype == kF16 || dtype == kBF16) && (ci == 64 || (ci > 0 && ci % 128 == 0)) && co > 0 && co % 64 == 0;
}

hipError_t launch_linear_mfma(int dtype, const void * x, const void * w16, const float * bias, void * y, int64_t n,
                              int ci, int co, int silu, int cus, hipStream_t s) {
    if (!linear_mfma_supported(dtype, ci, co) || n <= 0 || cus <= 0) {
        return hipErrorInvalidValue;
    }
    if (dtype == kBF16) return launch_linear_dt<kBF16>(x, w16, bias, y, n, ci, co, silu, cus, s);
    return launch_linear_dt<kF16>(x, w16, bias, y, n, ci, co, silu, cus, s);
}

}  // namespace tsh
