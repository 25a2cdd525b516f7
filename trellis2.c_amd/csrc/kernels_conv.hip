// kernels_conv.hip - 3x3x3 submanifold sparse convolution for gfx950.
//
// out[i][o] = bias[o] + sum_k sum_c x[nbr[i][k]][c] * W[o][k][c]
// (src/ops/sparse/trellis_sparse_cpu.c:324-373; weight [Co][27][Ci], :361).
//
// Three schedules, each deterministic:
//
//  * generic  - VALU, any channel counts, any storage type.  For each output
//               it follows the reference's operation order exactly: start at
//               the bias, then per valid offset in k order a sequentially
//               rounded fp32 dot product (no fused multiply-add) added to the
//               row.  With fp32 storage the result is bit-identical to the
//               reference CPU backend.
//  * masked   - bf16/fp16 storage, Ci % 32 == 0, Co % 64 == 0.  Implicit GEMM
//               on v_mfma_f32_16x16x32_{bf16,f16} with fp32 accumulation over
//               the dense neighbour table.  A block owns 64 output rows x
//               64/128 output channels; each wavefront owns 32 rows x 32/64
//               channels.  For each offset the lanes gather their source rows
//               straight into MFMA A fragments (16 contiguous bytes per lane)
//               and read pre-packed weight fragments; row groups of 16 with no
//               valid neighbour skip the offset, others multiply zeros for
//               their missing neighbours.
//  * os64     - bf16/fp16 storage, Ci = Co = 64 (the compact schedule's
//               choice for that shape): output-stationary over the same pair
//               lists, sums in registers for all 27 offsets, no tile sums.
//  * compact  - bf16/fp16 storage, Ci = 64 or Ci % 128 == 0, Co % 64 == 0 or
//               Co = 16 / 32 (one 16/32-channel block).  The same MFMA
//               tiles driven by the kernel map's compacted per-tile pair
//               lists, so the MFMA rows are valid (src, dst) pairs only; sums
//               of a 256-row tile stay in LDS until one final store.  Blocks
//               of 128 output channels run k_conv_mfma_wreg (weights in
//               registers, feature rows shared through LDS), blocks of 64,
//               32 or 16 k_conv_mfma_stream (weights shared through LDS).
#include <type_traits>

#include "tsh_internal.h"
#include "mfma_common.h"

namespace tsh {
namespace {

// ---------------------------------------------------------------------------
// Generic VALU kernel: 16 TM rows x 64 channels per 256-lane block, each
// lane TM rows x 4 channels (TM = 1 for small row counts, for more blocks).  Every output is formed in the reference's order:
// bias, then per offset k (rows with a neighbour at k only) a partial sum
// over the input channels in ascending order, mul and add rounded
// separately, added to the running sum.  The block's 32 x 27 neighbour rows
// are staged once; offsets no row of the block has are skipped.  The (k,
// 32-channel chunk) tiles run through a double-buffered LDS stage, the next
// tile's gathers loaded into registers while the current one is multiplied,
// one barrier per tile.
// ---------------------------------------------------------------------------
template <int DT, int TM>
__global__ void __launch_bounds__(256) k_conv_generic(const typename Store<DT>::T * __restrict__ x,
                                                      const int32_t * __restrict__ nbr,
                                                      const float * __restrict__ w32,
                                                      const float * __restrict__ bias,
                                                      typename Store<DT>::T * __restrict__ y, int64_t n, int ci,
                                                      int co) {
#pragma clang fp contract(off)
    constexpr int BM = 16 * TM, BN = 64, BK = 32;
    constexpr int AQ = BM * BK / 256;  // A elements per lane and tile
    __shared__ float s_a[2][BM][BK + 1];
    __shared__ __attribute__((aligned(16))) float s_b[2][BK][BN];
    __shared__ int32_t s_nbr[BM * 27];
    __shared__ int32_t s_klist[27];
    __shared__ int32_t s_nk;
    const int t = threadIdx.x;
    const int tx = t & 15, ty = t >> 4;
    const int64_t row0 = (int64_t) blockIdx.x * BM;
    const int col0 = blockIdx.y * BN;
    const int rows = (int) ((n - row0) < BM ? (n - row0) : BM);
    // The block's neighbour rows: rows * 27 consecutive entries.
    for (int e = t; e < BM * 27; e += 256) s_nbr[e] = e < rows * 27 ? nbr[row0 * 27 + e] : -1;
    __syncthreads();
    if (t < 64) {
        // Offsets some row of the block has, in ascending order (a ballot
        // per offset, then a prefix count).
        const int k = t;
        bool has = false;
        if (k < 27) {
            for (int r = 0; r < BM; ++r) has = has || s_nbr[r * 27 + k] >= 0;
        }
        const uint64_t bal = __ballot(has);
        if (has) s_klist[__popcll(bal & ((1ull << t) - 1ull))] = k;
        if (t == 0) s_nk = __popcll(bal);
    }
    __syncthreads();
    const int nk = s_nk;
    const int nchunk = (ci + BK - 1) / BK;
    const int tiles = nk * nchunk;

    float acc[TM][4];
    float part[TM][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = col0 + tx * 4 + j;
        const float b = (bias != nullptr && col < co) ? bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = b;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) part[i][j] = 0.0f;

    // Tile it = (k = s_klist[it / nchunk], c0 = (it % nchunk) * BK).
    float ra[AQ], rb[8];
    auto fetch = [&](int it) {
        const int k = s_klist[it / nchunk];
        const int c0 = (it % nchunk) * BK;
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int e = t + q * 256;
            const int r = e >> 5, c = e & 31;
            const int32_t src = s_nbr[r * 27 + k];
            ra[q] = (src >= 0 && c0 + c < ci) ? Store<DT>::ld(x, (int64_t) src * ci + c0 + c) : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int e = t + q * 256;
            const int c = e >> 6, o = e & 63;
            rb[q] = (c0 + c < ci && col0 + o < co) ? w32[((int64_t) k * ci + c0 + c) * co + col0 + o] : 0.0f;
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int e = t + q * 256;
            s_a[buf][e >> 5][e & 31] = ra[q];
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int e = t + q * 256;
            s_b[buf][e >> 6][e & 63] = rb[q];
        }
    };
    if (tiles > 0) {
        fetch(0);
        stage(0);
    }
    __syncthreads();
    for (int it = 0; it < tiles; ++it) {
        const int buf = it & 1;
        if (it + 1 < tiles) fetch(it + 1);
        const int k = s_klist[it / nchunk];
        const int c0 = (it % nchunk) * BK;
        const int kmax = (ci - c0) < BK ? (ci - c0) : BK;
        // Channels in groups of 4: the group's LDS reads are all issued
        // before its multiplies, so one LDS latency covers four channels;
        // the sums still run channel by channel.
        const int kmax4 = kmax & ~3;
        for (int c = 0; c < kmax4; c += 4) {
            float a[4][TM];
            float4 b[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
                for (int i = 0; i < TM; ++i) a[u][i] = s_a[buf][ty * TM + i][c + u];
                b[u] = *(const float4 *) &s_b[buf][c + u][tx * 4];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float bb[4] = {b[u].x, b[u].y, b[u].z, b[u].w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int i = 0; i < TM; ++i) part[i][j] = part[i][j] + a[u][i] * bb[j];
            }
        }
        for (int c = kmax4; c < kmax; ++c) {
            float a[TM];
#pragma unroll
            for (int i = 0; i < TM; ++i) a[i] = s_a[buf][ty * TM + i][c];
            const float4 b = *(const float4 *) &s_b[buf][c][tx * 4];
            const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < TM; ++i) part[i][j] = part[i][j] + a[i] * bb[j];
        }
        if (it % nchunk == nchunk - 1) {
            // Offset k done: rows with a neighbour at k add their partial sum
            // (the reference skips the offset for the others, it does not add
            // a zero).
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                if (s_nbr[(ty * TM + i) * 27 + k] >= 0) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = acc[i][j] + part[i][j];
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) part[i][j] = 0.0f;
            }
        }
        // The other buffer was last read by the previous tile, before the
        // previous barrier.
        if (it + 1 < tiles) stage(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int64_t r = row0 + ty * TM + i;
        if (r >= n) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = col0 + tx * 4 + j;
            if (col < co) Store<DT>::st(y, r * co + col, acc[i][j]);
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA kernel (bf16 / fp16 storage).
// ---------------------------------------------------------------------------
// WR wavefronts split the rows (32 each), 4/WR the BN channels: WR = 2 for
// 64/128-channel blocks, WR = 4 for the narrow outputs (16 or 32 channels,
// e.g. the encoder's S2C conv to co/8 channels), whose one column group is
// the whole output.
template <int DT, int BN, int WR>
__global__ void __launch_bounds__(256) k_conv_mfma_masked(const typename Store<DT>::T * __restrict__ x,
                                                          const int32_t * __restrict__ nbr,
                                                          const uint32_t * __restrict__ mask,
                                                          const typename Store<DT>::T * __restrict__ w16,
                                                          const float * __restrict__ bias,
                                                          typename Store<DT>::T * __restrict__ y, int64_t n, int ci,
                                                          int co, int64_t n_col_tiles) {
    using V = typename Mfma<DT>::V;
    constexpr int BM = 32 * WR;
    constexpr int WN = BN / (4 / WR);  // channels per wavefront
    constexpr int NT = WN / 16;        // 16-wide MFMA column tiles per wavefront
    static_assert(NT >= 1 && WN % 16 == 0, "column split");
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wr = wave % WR, wc = wave / WR;
    const int64_t grid = (int64_t) gridDim.x;
    const int64_t logical = xcd_remap(blockIdx.x, grid);
    const int64_t row_tile = logical / n_col_tiles;
    const int col_tile = (int) (logical % n_col_tiles);
    const int64_t row0 = row_tile * BM + wr * 32;
    const int colw = col_tile * BN + wc * WN;
    const int l16 = lane & 15, lg = lane >> 4;
    const int ci8 = ci >> 3;

    f32x4 acc[2][NT];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[m][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    int64_t arow[2];
    uint32_t amask[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        arow[m] = row0 + m * 16 + l16;
        amask[m] = arow[m] < n ? mask[arow[m]] : 0u;
    }
    // Offsets any of this wavefront's rows need.
    uint32_t need = amask[0] | amask[1];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) need |= __shfl_xor(need, d);

    const V zero = V{};
    for (int k = 0; k < 27; ++k) {
        if (((need >> k) & 1u) == 0) {
            continue;
        }
        int32_t src[2];
        bool live[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            src[m] = ((amask[m] >> k) & 1u) ? nbr[arow[m] * 27 + k] : -1;
            live[m] = __ballot(src[m] >= 0) != 0;
        }
        const typename Store<DT>::T * wk = w16 + (int64_t) k * ci8 * co * 8;
        for (int c0 = 0; c0 < ci; c0 += 32) {
            V a[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                a[m] = src[m] >= 0 ? *(const V *) (x + (int64_t) src[m] * ci + c0 + lg * 8) : zero;
            }
            const int g = (c0 >> 3) + lg;
            V b[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                b[j] = *(const V *) (wk + ((int64_t) g * co + colw + j * 16 + l16) * 8);
            }
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                if (!live[m]) continue;
#pragma unroll
                for (int j = 0; j < NT; ++j) acc[m][j] = Mfma<DT>::mac(a[m], b[j], acc[m][j]);
            }
        }
    }
    // Epilogue: bias, round to storage, store.
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int col = colw + j * 16 + l16;
        const float bv = bias != nullptr ? bias[col] : 0.0f;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t r = row0 + m * 16 + lg * 4 + i;
                if (r < n) Store<DT>::st(y, r * co + col, acc[m][j][i] + bv);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Compacted MFMA kernel (bf16 / fp16 storage), streamed.
//
// A block owns one 256-row map tile x BN output channels; the fp32 sums of
// those rows live in LDS.  The kernel map's tile-major pair lists give, for
// each offset k, the tile's valid (src, dst) pairs in destination order.  The
// block walks "units" (offset k, up to 128 of its pairs): the centre offset's
// first, whose flushes store (every row of the tile has one centre pair, so
// the sums need no clearing), then the others in k order; each unit
// is Ci/32 K steps of MFMA work over 16-pair row blocks, so the MFMA row
// dimension runs over valid pairs only.  NW wavefronts (8: two per SIMD, so
// one's VALU and LDS work overlaps the other's MFMAs) are split into RG row
// groups and NW/RG channel groups; wavefront w multiplies row blocks
// w % RG + RG q of the unit by channel group w / RG.  The default, RG = 8,
// gives each wavefront one row block and all BN channels, so no feature row
// is fetched twice.
//
// Steps are processed in blocks of DEPTH (Ci/32 is a multiple of DEPTH, so a
// block never straddles two units).  Operands are fetched one block ahead:
//  * A (gathered feature rows) goes global -> registers; the row addresses of
//    the target block are formed once per block from the unit's source list.
//  * B (the unit's weight slice, 32 channels x BN per step) is fetched once
//    per block into registers, stored into a 3-slot LDS ring two steps before
//    use and read into fragments one step before use by every wavefront, which
//    halves the weight bytes through the vector memory path and keeps LDS
//    latency off the MFMA stream.
// One barrier per step, after the step's MFMAs are issued, publishes the
// weights stored during the step; it orders LDS only, so the register rings
// stay in flight across it and the matrix cores run while wavefronts wait.
//
// Weights use the grouped packing: packed column ch*WN + nt*16 + l16 holds
// output channel ch*WN + l16*NT + nt, so each lane's MFMA results for a row
// are NT adjacent channels and a unit's results reach the LDS sums as one
// vector read-modify-write per row.  Padding rows of a unit (past its count)
// multiply a repeated valid pair and are added into a spare row.  Within a
// unit a destination occurs at most once and units are applied in order, so
// the result is deterministic.  The tile's rows are written once at the end.
// ---------------------------------------------------------------------------
// Shape of the streamed schedule: wavefronts per block, and row groups among
// them (the rest split the block's channels).
#ifndef TSH_STREAM_WAVES
#define TSH_STREAM_WAVES 8
#endif
#ifndef TSH_STREAM_ROW_GROUPS
#define TSH_STREAM_ROW_GROUPS 8
#endif

template <int DT, int BN, int DEPTH, int NW, int RG, int UPB>
__global__ void __launch_bounds__(64 * NW) k_conv_mfma_stream(const typename Store<DT>::T * __restrict__ x,
                                                               const int32_t * __restrict__ pair_src,
                                                               const uint8_t * __restrict__ pair_dst,
                                                               const int32_t * __restrict__ tile_off,
                                                               const int32_t * __restrict__ tile_counts,
                                                               const typename Store<DT>::T * __restrict__ w16,
                                                               const float * __restrict__ bias,
                                                               typename Store<DT>::T * __restrict__ y, int64_t n,
                                                               int ci, int co, int64_t n_col_tiles) {
    using T = typename Store<DT>::T;
    using V = typename Mfma<DT>::V;
    constexpr int TM = kMapTile;     // rows per block = rows per kernel-map tile
    constexpr int BK = 32;           // input channels per K step
    constexpr int NTHR = 64 * NW;
    // Row groups RG: wavefront w takes row blocks w % RG + RG * q of a unit
    // and channel group w / RG.
    constexpr int CG = NW / RG;      // channel groups
    constexpr int WN = BN / CG;      // channels per wavefront
    constexpr int NT = WN / 16;      // MFMA column tiles per wavefront
    constexpr int QB = 8 / RG;       // row blocks per wavefront per unit
    constexpr int PASS = 128;        // pairs per unit
    constexpr int MAX_UNITS = 27 * (TM / PASS);
    constexpr int BSLOT = 4 * BN * 8;      // weight elements per step: [4 channel groups][BN][8]
    constexpr int BUNITS = 4 * BN;         // 16-byte pieces of a step's weights
    constexpr int BLOADS = (BUNITS + NTHR - 1) / NTHR;  // pieces per thread
    static_assert(NW == 4 || NW == 8, "4 or 8 wavefronts");
    static_assert((RG == 2 || RG == 4 || RG == 8) && NW % RG == 0 && NT >= 1, "row groups");
    constexpr int QF = QB < 2 ? QB : 2;  // row blocks per flush batch
    static_assert(DEPTH == 4 || DEPTH == 8, "block of 4 or 8 steps");
    static_assert(UPB == 1 || UPB == 2, "units per block");
    constexpr int RING = UPB == 1 ? 4 : 8;  // unit-list slots: the current block's units and two blocks ahead
    static_assert(BUNITS % NTHR == 0 || BUNITS < NTHR, "weight pieces split evenly or fit one round");
    __shared__ float s_acc[(TM + 1) * BN];      // row TM absorbs padding rows
    __shared__ __attribute__((aligned(16))) T s_b[3][BSLOT];
    __shared__ int32_t s_rsrc[RING][PASS];
    __shared__ uint16_t s_rdst[RING][PASS];     // tile-local dst row, TM for padding
    __shared__ int32_t s_uk[MAX_UNITS], s_ustart[MAX_UNITS], s_ucnt[MAX_UNITS];
    __shared__ int32_t s_cnt[27], s_start[27];
    __shared__ int32_t s_units;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int rh = wave % RG, ch = wave / RG;
    const int l16 = lane & 15, lg = lane >> 4;
    const int64_t logical = xcd_remap(blockIdx.x, (int64_t) gridDim.x);
    const int64_t tile = logical / n_col_tiles;
    const int64_t row0 = tile * TM;
    const int col0 = (int) (logical % n_col_tiles) * BN;
    const int ci8 = ci >> 3;
    const int KS = ci / BK;

    // The centre offset pairs every row of the tile with exactly one row
    // (itself, or the last duplicate of its coordinates), and the kernel map
    // packs its list first in the tile's region, dst ascending.  So the
    // first CU units are the centre's: their lists sit at known places, and
    // together they write every row of the tile once, which is why their
    // flushes store instead of adding and the tile sums need no clearing.
    const int tile_rows = (int) ((n - row0) < TM ? (n - row0) : TM);
    const int CU = (tile_rows + PASS - 1) / PASS;
    const int64_t region = tile * TM * 27;
    const int le = t & (PASS - 1);
    // Entry pos of this thread's list: sources (threads 0..PASS-1) or the
    // destinations' rows within the map tile (threads PASS..2 PASS-1).
    auto list_at = [&](int64_t pos) -> int32_t { return t < PASS ? pair_src[pos] : (int32_t) pair_dst[pos]; };
    // One round trip for the tile's counts and starts and the centre units'
    // lists among the first 2 UPB units (the ring fill below).
    int32_t cnt_v = 0, off_v = 0;
    if (t < 27) {
        cnt_v = tile_counts[tile * 27 + t];
        off_v = tile_off[tile * 27 + t];
    }
    int32_t ring_v[2 * UPB];
#pragma unroll
    for (int j = 0; j < 2 * UPB; ++j) {
        const int cj = tile_rows - j * PASS < PASS ? tile_rows - j * PASS : PASS;
        ring_v[j] = (t < 2 * PASS && j < CU) ? list_at(region + j * PASS + (le < cj ? le : cj - 1)) : 0;
    }
    if (t < 27) {
        s_cnt[t] = cnt_v;
        s_start[t] = off_v;
    }
    lds_barrier();
    // Unit table: offset k contributes ceil(count / PASS) units, the centre
    // offset's first, then the others in k order (the packing order): lane p
    // of wavefront 0 takes the p-th offset of that order, and a scan of the
    // unit counts gives each offset's first unit.
    if (t < 64) {
        const int k = t == 0 ? 13 : (t <= 13 ? t - 1 : t);
        const int c = t < 27 ? s_cnt[k] : 0;
        const int nu = (c + PASS - 1) / PASS;
        int incl = nu;
#pragma unroll
        for (int d = 1; d < 32; d <<= 1) {
            const int o = __shfl_up(incl, d);
            if (lane >= d) incl += o;
        }
        int u = incl - nu;
#pragma unroll 1
        for (int p = 0; p < c; p += PASS, ++u) {
            s_uk[u] = k;
            s_ustart[u] = s_start[k] + p;
            s_ucnt[u] = c - p < PASS ? c - p : PASS;
        }
        if (t == 26) s_units = incl;
    }
    lds_barrier();
    const int U = s_units;
    if (U == 0) return;  // unreachable for a tile with rows: the centre offset pairs every row with itself

    // Unit lists, staged two blocks ahead in a ring of RING slots (threads
    // 0..127 carry src entries, 128..255 dst entries).  Padding entries
    // repeat the unit's last pair, so every gather stays in range; past the
    // last unit the last unit is loaded again (never used).
    auto list_load = [&](int u) -> int32_t {
        if (t >= 2 * PASS) return 0;
        const int lu = u < U ? u : U - 1;
        const int c = s_ucnt[lu];
        return list_at(s_ustart[lu] + (le < c ? le : c - 1));
    };
    auto list_store = [&](int u, int32_t v) {
        if (t < PASS) {
            s_rsrc[u & (RING - 1)][le] = v;
        } else if (t < 2 * PASS) {
            const int c = s_ucnt[u < U ? u : U - 1];
            s_rdst[u & (RING - 1)][le] = (uint16_t) (le < c ? v : TM);
        }
    };
#pragma unroll
    for (int j = 0; j < 2 * UPB; ++j) list_store(j, j < CU ? ring_v[j] : list_load(j));
    int32_t lv[UPB];
#pragma unroll
    for (int j = 0; j < UPB; ++j) lv[j] = list_load(2 * UPB + j);
    lds_barrier();

    // Operand addresses of one block of DEPTH steps, which covers UPB units
    // of SPU steps each (UPB > 1 only when a unit is shorter than a block):
    // unit tu + r / SPU, K step tps + r % SPU for step r (past the last unit:
    // the last unit again).  A row q of step r is at pa[r/SPU][q] +
    // (r%SPU)*BK; the thread's weight pieces at pb[r/SPU] + (r%SPU)*bstep +
    // piece offset.
    constexpr int SPU = DEPTH / UPB;
    const int64_t bstep = (int64_t) 4 * co * 8;  // elements between consecutive K steps' weights
    int64_t boff[BLOADS];
#pragma unroll
    for (int h = 0; h < BLOADS; ++h) {
        const int u = t + h * NTHR;
        boff[h] = ((int64_t) (u / BN) * co + u % BN) * 8;
    }
    const T * pa[UPB][QB];
    const T * pb[UPB];
    // A rows are fetched straight in MFMA operand order (lane i + 16 c reads
    // 16 bytes c of row i of the row block).  Fetching them in the lane order
    // of a coalesced load (four neighbouring lanes per 64-byte segment) and
    // moving them to operand order with ds_bpermute moved the vector memory
    // path's bytes faster in a microbenchmark, but the permutes cost more:
    // the S2C block's 64 -> 16 conv took 0.304 ms that way, 0.270 ms this way.
    auto target = [&](int tu0, int tps) {
#pragma unroll
        for (int uo = 0; uo < UPB; ++uo) {
            const int tu = tu0 + uo < U ? tu0 + uo : U - 1;
            const int slot = tu & (RING - 1);
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                const int32_t src = s_rsrc[slot][(rh + RG * q) * 16 + l16];
                pa[uo][q] = x + (int64_t) src * ci + tps * BK + lg * 8;
            }
            pb[uo] = w16 + ((int64_t) (s_uk[tu] * ci8 + tps * 4) * co + col0) * 8;
        }
    };
    constexpr bool B_ALL = BUNITS >= NTHR;  // every thread has a weight piece
    auto load_a = [&](V * a, int r) {
#pragma unroll
        for (int q = 0; q < QB; ++q) a[q] = *(const V *) (pa[r / SPU][q] + (r % SPU) * BK);
    };
    auto load_b = [&](V * b, int r) {
        if (B_ALL || t < BUNITS) {
#pragma unroll
            for (int h = 0; h < BLOADS; ++h) b[h] = *(const V *) (pb[r / SPU] + (r % SPU) * bstep + boff[h]);
        }
    };
    auto store_b = [&](int slot, const V * b) {
        if (B_ALL || t < BUNITS) {
#pragma unroll
            for (int h = 0; h < BLOADS; ++h) *(V *) (&s_b[slot][(t + h * NTHR) * 8]) = b[h];
        }
    };

    V ra[DEPTH][QB];  // A fragments in flight
    V rw[DEPTH][BLOADS];
    V rf[2][NT];  // weight fragments of step g in rf[g & 1]
    f32x4 acc[QB][NT];
#pragma unroll
    for (int q = 0; q < QB; ++q)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Flush: add a unit's products into the tile sums.  The lane's NT
    // columns are adjacent (grouped weight packing), so each row is one
    // vector read-modify-write; padding rows go to the spare row TM.  Within
    // a unit every valid destination occurs once, and no other wavefront
    // touches these columns of these rows before the next barrier.  Rows are
    // read in batches before any is written back, so the LDS round trips
    // overlap (the compiler cannot reorder a read past a write to a possibly
    // equal row).
    auto flush = [&](int unit) {
        const int slot = unit & (RING - 1);
        const bool first = unit < CU;  // a centre unit: its rows' first sums
        using Row = float __attribute__((ext_vector_type(NT)));
#pragma unroll
        for (int q0 = 0; q0 < QB; q0 += QF) {
            Row * dst[QF][4];
            Row v[QF][4];
#pragma unroll
            for (int qq = 0; qq < QF; ++qq) {
                const ushort4 d = *(const ushort4 *) &s_rdst[slot][(rh + RG * (q0 + qq)) * 16 + lg * 4];
                const int rows[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[qq][i] = (Row *) (s_acc + rows[i] * BN + ch * WN + l16 * NT);
            }
            if (first) {
#pragma unroll
                for (int qq = 0; qq < QF; ++qq)
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[qq][i] = (Row) 0.0f;
            } else {
#pragma unroll
                for (int qq = 0; qq < QF; ++qq)
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[qq][i] = *dst[qq][i];
            }
#pragma unroll
            for (int qq = 0; qq < QF; ++qq)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) v[qq][i][nt] += acc[q0 + qq][nt][i];
                    *dst[qq][i] = v[qq][i];
                }
#pragma unroll
            for (int qq = 0; qq < QF; ++qq)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[q0 + qq][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };

    // Block 0: every fetch of its DEPTH steps issued first, in the order the
    // main loop issues them (step r: weights, then A), so that the loop's
    // memory waits, which must hold for its first pass as for the later
    // ones, stay those of a full DEPTH-step look-ahead; then the weights of
    // steps 0 and 1 into LDS slots 0 and 1 (one round trip for the block).
    target(0, 0);
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) {
        load_b(rw[r], r);
        load_a(ra[r], r);
    }
    store_b(0, rw[0]);
    store_b(1, rw[1]);
    lds_barrier();
    {
        const T * bs = &s_b[0][(lg * BN + ch * WN + l16) * 8];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) rf[0][nt] = *(const V *) (bs + nt * 16 * 8);
    }

    int bslot = 0;  // LDS slot of the current step's weights (step g: g % 3)
    for (int cb = 0; cb < U; cb += UPB) {
        // The lists of the units two blocks ahead become visible at this
        // block's first barrier; their first readers are the next block's
        // target computation.
#pragma unroll
        for (int j = 0; j < UPB; ++j) {
            list_store(cb + 2 * UPB + j, lv[j]);
            lv[j] = list_load(cb + 3 * UPB + j);
        }
        int s0 = 0;
        do {
            // This block prefetches the next one: same unit unless s0 is the
            // unit's last block (always the next units when UPB > 1).
            if constexpr (UPB == 1) {
                const bool last = s0 + DEPTH >= KS;
                target(last ? cb + 1 : cb, last ? 0 : s0 + DEPTH);
            } else {
                target(cb + UPB, 0);
            }
#pragma unroll
            for (int r = 0; r < DEPTH; ++r) {
                const int s1 = bslot == 2 ? 0 : bslot + 1;  // next step's weights
                const int s2 = s1 == 2 ? 0 : s1 + 1;        // step after: held step g-1
                // Fragments of the next step (stored two steps ago, published
                // by the previous step's barrier).
                const T * bs = &s_b[s1][(lg * BN + ch * WN + l16) * 8];
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) rf[(r + 1) & 1][nt] = *(const V *) (bs + nt * 16 * 8);
#pragma unroll
                for (int q = 0; q < QB; ++q)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        acc[q][nt] = Mfma<DT>::mac(ra[r][q], rf[r & 1][nt], acc[q][nt]);
                // Weights of step g + 2 (fetched two steps ago) into the slot
                // whose fragments every wavefront read before the last barrier.
                store_b(s2, rw[(r + 2) % DEPTH]);
                load_b(rw[r], r);
                load_a(ra[r], r);
                bslot = s1;
                lds_barrier();
                // Keep each step's loads in its step: the scheduler would
                // otherwise sink the whole ring's loads below the last MFMA.
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (UPB > 1) {
                    // A unit ends inside the block; a unit past the last one
                    // (odd unit count) multiplied repeated data and is dropped.
                    if (r % SPU == SPU - 1 && cb + r / SPU < U) flush(cb + r / SPU);
                    if (r % SPU == SPU - 1) {
#pragma unroll
                        for (int q = 0; q < QB; ++q)
#pragma unroll
                            for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
                    }
                }
            }
            s0 += DEPTH;
        } while (s0 < KS);
        if constexpr (UPB == 1) flush(cb);
    }
    lds_barrier();
    // Epilogue: bias, round to the storage type, 16-byte coalesced stores.
    constexpr int CHUNKS = BN / 8;
    for (int e = t; e < TM * CHUNKS; e += NTHR) {
        const int rr = e / CHUNKS, cc = (e % CHUNKS) * 8;
        const int64_t row = row0 + rr;
        if (row >= n) continue;
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = s_acc[rr * BN + cc + u] + (bias != nullptr ? bias[col0 + cc + u] : 0.0f);
        *(int4 *) (y + row * co + col0 + cc) = pack_chunk<DT>(v);
    }
}

// ---------------------------------------------------------------------------
// Compacted MFMA kernel with the weights in registers.
//
// Same units, tile sums in LDS, flush and epilogue as k_conv_mfma_stream, with
// the two operands' staging paths exchanged:
//  * A (the unit's gathered feature rows: 128 rows x 32 channels per step,
//    8 KB) is fetched once per step by the whole block, one 16-byte piece per
//    thread with four neighbouring lanes reading one row's 64 bytes, and
//    stored into a 3-slot LDS ring two steps before use; each wavefront reads
//    its row blocks' MFMA fragments one step before use.  The ring's layout
//    (a_granule) keeps both the coalesced store and the fragment reads free
//    of bank conflicts, and no lane transpose is needed.
//  * B (the weights) never passes through LDS: each wavefront fetches its own
//    channels' fragments straight into registers one block of DEPTH steps
//    ahead and multiplies them there.
// With RG row groups a step reads 64/RG KB of A fragments from LDS and fetches
// RG x 8 KB of weights (each row group fetches all BN channels); RG = 2 (each
// wavefront: 4 row blocks x 32 channels) balances the two.  Blocks of DEPTH =
// 8 steps (when a unit is a whole number of them) give the gathers six steps
// between fetch and use.
// With Co % 256 == 0 a block covers 256 channels over half a map tile (TMR =
// 128 rows; the 128 x 256 tile sums take the LDS that 256 x 128 take): each
// offset's list is split where its destinations leave the first 128 rows, a
// wavefront holds 64 rows x 64 channels, and every barrier, fragment read and
// gather serves twice the MFMAs.  With 4-step units (Ci % 256 != 0) a block
// of 4 wavefronts covers half a tile with 64-pair units, so that two blocks
// share a CU.  A row's sums are formed in the same order in every layout, so
// all of them give bit-identical outputs.
// ---------------------------------------------------------------------------

// Sum over the 16 lanes of a DPP row, left in every lane of the row:
// rotations by 8, 4, 2 and 1 within the row (row_ror), each one VALU add.
__device__ __forceinline__ float row16_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
    return v;
}

static_assert(kLayoutSlots == 64, "one layout statistics slot per lane");

template <int DT, int BN, int RG, int UPB, int DEPTH, int TMR, int NW, int AP = 1, bool PACK64 = false>
__global__ void __launch_bounds__(64 * NW, NW * AP == 8 ? 1 : 2) k_conv_mfma_wreg(const typename Store<DT>::T * __restrict__ x,
                                                        const int32_t * __restrict__ pair_src,
                                                        const uint8_t * __restrict__ pair_dst,
                                                        const int32_t * __restrict__ tile_off,
                                                        const int32_t * __restrict__ tile_counts,
                                                        const uint32_t * __restrict__ mask,
                                                        const typename Store<DT>::T * __restrict__ w16,
                                                        const float * __restrict__ bias,
                                                        typename Store<DT>::T * __restrict__ y, int64_t n, int ci,
                                                        int co, ConvEpilogue epi, int layout_sel,
                                                        const int32_t * __restrict__ layout_stats) {
    using T = typename Store<DT>::T;
    using V = typename Mfma<DT>::V;
    // NW wavefronts; a unit holds AP 16-row blocks per wavefront.
    constexpr int NTHR = 64 * NW;
    constexpr int TM = TMR;          // rows per block: a kernel-map tile, or half of one
    constexpr int HALVES = kMapTile / TM;
    static_assert(HALVES == 1 || (HALVES == 2 && UPB == 1), "whole or half map tiles");
    constexpr int BK = 32;           // input channels per K step
    constexpr int CG = NW / RG;      // channel groups
    constexpr int WN = BN / CG;      // channels per wavefront
    constexpr int NT = WN / 16;      // MFMA column tiles per wavefront
    constexpr int PASS = 16 * NW * AP;  // pairs per unit
    constexpr int QB = NW * AP / RG;    // row blocks per wavefront per unit
    constexpr int MAX_UNITS = 27 * (TM / PASS);
    constexpr int QF = QB < 2 ? QB : 2;  // row blocks per flush batch
    constexpr int RING = UPB == 1 ? 4 : 8;
    constexpr int SPU = DEPTH / UPB;
    static_assert((RG == 1 || RG == 2 || RG == 4) && NT >= 1 && WN % 16 == 0, "row groups");
    static_assert(PASS * 4 == NTHR * AP && (AP == 1 || AP == 2), "AP 16-byte A pieces per thread and step");
    static_assert(2 * PASS <= NTHR, "a thread per src and dst list entry");
    static_assert(UPB == 1 || UPB == 2, "units per block");
    static_assert(DEPTH == 4 || DEPTH == 8, "block of 4 or 8 steps");
    __shared__ float s_acc[(TM + 1) * BN];      // row TM absorbs padding rows
    __shared__ __attribute__((aligned(16))) T s_a[3][PASS * BK];
    __shared__ int32_t s_rsrc[RING][PASS];
    __shared__ uint16_t s_rdst[RING][PASS];     // tile-local dst row, TM for padding
    __shared__ int32_t s_uk[MAX_UNITS], s_ustart[MAX_UNITS], s_ucnt[MAX_UNITS];
    __shared__ int32_t s_cnt[27], s_start[27];
    __shared__ int32_t s_units;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int rh = wave % RG, ch = wave / RG;
    const int l16 = lane & 15, lg = lane >> 4;
    // Layout choice for Co % 256 == 0 (layout_sel 1: this launch runs the
    // conv if the 256-column layout takes it, 2: if the 128-column one does).
    // The 256-column blocks cover half tiles with one unit per offset and
    // half, the 128-column ones whole tiles with one unit per offset, two
    // where more than half the tile's rows have a neighbour at the offset.
    // The kernel map counts, over all tiles, the offsets with pairs and
    // those with more than 128.  On dense sets (about 1 in 2 with more than
    // 128) the wide layout's MFMAs per fetched byte win, on sparse ones
    // (about 1 in 20) its half-empty units lose to the narrow layout's
    // fuller ones.  The crossover moves with Ci (measured): the wide layout
    // runs from 4 in 10 with Ci >= 512 (config 5: 0.52, wide 5 % faster),
    // from 6 in 10 with Ci <= 256 (0.49 and 0.56: narrow 5 and 1-2 % faster).
    if (layout_sel != 0) {
        // Lane l holds slot l of both sums (kLayoutSlots == 64 slots each).
        int32_t offsets = layout_stats[threadIdx.x & 63], busy = layout_stats[64 + (threadIdx.x & 63)];
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            offsets += __shfl_xor(offsets, d);
            busy += __shfl_xor(busy, d);
        }
        if ((10 * busy >= (ci <= 256 ? 6 : 4) * offsets) != (layout_sel == 1)) return;
    }
    const int64_t logical = xcd_remap(blockIdx.x, (int64_t) gridDim.x);
    // Column block slowest, then tile, then half: an XCD's range of blocks
    // covers few column blocks, so each XCD fetches few columns' weights.
    const int64_t row_tiles = ((n + kMapTile - 1) / kMapTile) * HALVES;
    const int64_t tile = (logical % row_tiles) / HALVES;
    const int half = HALVES == 1 ? 0 : (int) (logical % HALVES);
    const int64_t row0 = tile * kMapTile + half * TM;
    const int col0 = (int) (logical / row_tiles) * BN;
    if (row0 >= n) return;  // the empty second half of a short last tile
    const int ci8 = ci >> 3;
    const int KS = ci / BK;

    // Epilogue operands fetched now, so that their latency hides under the
    // main loop: this thread's residual chunks (add epilogue).  Thread t
    // handles chunk column cc of rows rr0 + p * (NTHR / CHUNKS) in the
    // epilogue; a block reads these residual rows before it writes the same
    // rows of y, so y may be the residual buffer.
    constexpr int CHUNKS = BN / 8;
    constexpr int PASSES = TM * CHUNKS / NTHR;
    static_assert(NTHR % CHUNKS == 0 && 64 % CHUNKS == 0 && (TM * CHUNKS) % NTHR == 0, "whole rows per wavefront");
    const int cc = (t % CHUNKS) * 8;
    const int rr0 = t / CHUNKS;
    union Chunk {
        int4 v;
        T h[8];
    };
    Chunk res[PASSES];
    if (epi.mode == kEpiAdd) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int64_t row = row0 + rr0 + p * (NTHR / CHUNKS);
            res[p].v = row < n ? *(const int4 *) ((const T *) epi.residual + row * co + col0 + cc) : int4{0, 0, 0, 0};
        }
    }

    // The centre offset pairs every row of the tile with exactly one row
    // (itself, or the last duplicate of its coordinates), and the kernel map
    // packs its list first in the tile's region, dst ascending.  So the
    // first CU units are the centre's: their lists sit at known places, and
    // together they write every row of the tile once, which is why their
    // flushes store instead of adding and the tile sums need no clearing.
    const int tile_rows = (int) ((n - row0) < TM ? (n - row0) : TM);
    const int CU = (tile_rows + PASS - 1) / PASS;
    // The centre list holds one entry per row of the map tile, in row
    // order, so this block's rows start `half * TM` entries into it.
    const int64_t region = tile * kMapTile * 27 + half * TM;
    const int le = t & (PASS - 1);
    // Entry pos of this thread's list: sources (threads 0..PASS-1) or the
    // destinations' rows within the map tile (threads PASS..2 PASS-1; this
    // block's rows start at half * TM of the tile).
    auto list_at = [&](int64_t pos) -> int32_t { return t < PASS ? pair_src[pos] : (int32_t) pair_dst[pos]; };
    const int32_t list_bias = half * TM;
    // One round trip for the tile's counts and starts and the centre units'
    // lists among the first 2 UPB units (the ring fill below).
    int32_t cnt_v = 0, off_v = 0;
    if (t < 27) {
        cnt_v = tile_counts[tile * 27 + t];
        off_v = tile_off[tile * 27 + t];
    }
    int32_t ring_v[2 * UPB];
#pragma unroll
    for (int j = 0; j < 2 * UPB; ++j) {
        const int cj = tile_rows - j * PASS < PASS ? tile_rows - j * PASS : PASS;
        ring_v[j] = (t < 2 * PASS && j < CU) ? list_at(region + j * PASS + (le < cj ? le : cj - 1)) : 0;
    }
    if (t < 27) {
        s_cnt[t] = cnt_v;
        s_start[t] = off_v;
    }
    // Half tiles: each offset's list (destinations ascending) splits where
    // its destinations leave the first half, after as many entries as the
    // first half's rows have a neighbour at that offset (mask ballots).
    __shared__ int32_t s_lo[HALVES == 2 ? 27 * 2 : 1];
    if constexpr (HALVES == 2) {
        if (t < TM) {
            const int64_t r = tile * kMapTile + t;
            const uint32_t mr = r < n ? mask[r] : 0u;
#pragma unroll 1
            for (int k = 0; k < 27; ++k) {
                const int c = __popcll(__ballot((mr >> k) & 1u));
                if (lane == 0) s_lo[k * 2 + (t >> 6)] = c;
            }
        }
    }
    lds_barrier();
    // Unit table: offset k contributes ceil(count / PASS) units, the centre
    // offset's first, then the others in k order (the packing order): lane p
    // of wavefront 0 takes the p-th offset of that order, and a scan of the
    // unit counts gives each offset's first unit.
    if (t < 64) {
        const int k = t == 0 ? 13 : (t <= 13 ? t - 1 : t);
        int c = t < 27 ? s_cnt[k] : 0;
        int start = t < 27 ? s_start[k] : 0;
        if constexpr (HALVES == 2) {
            if (t < 27) {
                const int lo = s_lo[k * 2] + s_lo[k * 2 + 1];
                start += half ? lo : 0;
                c = half ? c - lo : lo;
            }
        }
        const int nu = (c + PASS - 1) / PASS;
        int incl = nu;
#pragma unroll
        for (int d = 1; d < 32; d <<= 1) {
            const int o = __shfl_up(incl, d);
            if (lane >= d) incl += o;
        }
        int u = incl - nu;
#pragma unroll 1
        for (int p = 0; p < c; p += PASS, ++u) {
            s_uk[u] = k;
            s_ustart[u] = start + p;
            s_ucnt[u] = c - p < PASS ? c - p : PASS;
        }
        if (t == 26) s_units = incl;
    }
    lds_barrier();
    const int U = s_units;
    if (U == 0) return;  // unreachable for a tile with rows: the centre offset pairs every row with itself

    // Unit lists, staged two blocks ahead in a ring of RING slots (threads
    // 0..127 carry src entries, 128..255 dst entries).  Padding entries
    // repeat the unit's last pair, so every gather stays in range; past the
    // last unit the last unit is loaded again (never used).
    auto list_load = [&](int u) -> int32_t {
        if (t >= 2 * PASS) return 0;
        const int lu = u < U ? u : U - 1;
        const int c = s_ucnt[lu];
        return list_at(s_ustart[lu] + (le < c ? le : c - 1));
    };
    auto list_store = [&](int u, int32_t v) {
        if (t < PASS) {
            s_rsrc[u & (RING - 1)][le] = v;
        } else if (t < 2 * PASS) {
            const int c = s_ucnt[u < U ? u : U - 1];
            s_rdst[u & (RING - 1)][le] = (uint16_t) (le < c ? v - list_bias : TM);
        }
    };
#pragma unroll
    for (int j = 0; j < 2 * UPB; ++j) list_store(j, j < CU ? ring_v[j] : list_load(j));
    int32_t lv[UPB];
#pragma unroll
    for (int j = 0; j < UPB; ++j) lv[j] = list_load(2 * UPB + j);
    lds_barrier();

    // This thread's A pieces: wavefront w fetches and stores row blocks w +
    // NW p (p < AP) of the unit; quad j of the wavefront (lanes 4j .. 4j+3)
    // fetches row a_quad_row(j) of the block, lane 4j + c its chunk c.
    // Fragment q of this lane: chunk lg of row l16 of row block rh + RG q.
    const int achunk = t & 3;
    int arow[AP], a_st[AP];
#pragma unroll
    for (int p = 0; p < AP; ++p) {
        arow[p] = ((t >> 6) + NW * p) * 16 + a_quad_row((t >> 2) & 15);
        a_st[p] = (((t >> 6) + NW * p) * 64 + a_granule(arow[p] & 15, achunk)) * 8;
    }
    const int a_ld = (rh * 64 + a_granule(l16, lg)) * 8;
    constexpr int A_QSTRIDE = RG * 64 * 8;

    // Operand addresses of the next block of DEPTH steps, which covers UPB
    // units of SPU steps each: unit tu + r / SPU, K step tps + r % SPU for
    // step r (past the last unit: the last unit again).
    const int64_t bstep = (int64_t) 4 * co * 8;  // elements between consecutive K steps' weights
    const int64_t blane = ((int64_t) lg * co + ch * WN + l16) * 8;
    const T * pa[UPB][AP];
    const T * pb[UPB];
    auto target = [&](int tu0, int tps) {
#pragma unroll
        for (int uo = 0; uo < UPB; ++uo) {
            const int tu = tu0 + uo < U ? tu0 + uo : U - 1;
#pragma unroll
            for (int p = 0; p < AP; ++p) {
                const int32_t src = s_rsrc[tu & (RING - 1)][arow[p]];
                pa[uo][p] = x + (int64_t) src * ci + tps * BK + achunk * 8;
            }
            pb[uo] = w16 + ((int64_t) (s_uk[tu] * ci8 + tps * 4) * co + col0) * 8 + blane;
        }
    };
    auto load_a = [&](V (&a)[AP], int r) {
#pragma unroll
        for (int p = 0; p < AP; ++p) a[p] = *(const V *) (pa[r / SPU][p] + (r % SPU) * BK);
    };
    auto load_b = [&](V * b, int r) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) b[nt] = *(const V *) (pb[r / SPU] + (r % SPU) * bstep + nt * 16 * 8);
    };
    auto store_a = [&](int slot, const V (&a)[AP]) {
#pragma unroll
        for (int p = 0; p < AP; ++p) *(V *) (&s_a[slot][a_st[p]]) = a[p];
    };
    auto read_a = [&](V * f, int slot) {
#pragma unroll
        for (int q = 0; q < QB; ++q) f[q] = *(const V *) (&s_a[slot][a_ld + q * A_QSTRIDE]);
    };

    V ra[DEPTH][AP];  // A pieces in flight
    V rb[DEPTH][NT];  // weights of the block's steps (refilled with the next block's)
    V af[2][QB];      // A fragments of step g in af[g & 1]
    f32x4 acc[QB][NT];
#pragma unroll
    for (int q = 0; q < QB; ++q)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Tile-sum column of this lane's products (NT consecutive floats).  With
    // the weights packed for WN-channel wavefronts (channel b * WN + l * NT + j
    // at packed position b * WN + 16 * j + l) the tile sums are in channel
    // order.  PACK64: the weights are packed for 64-channel wavefronts (the
    // 256-column layout's) and this kernel's wavefronts take 32 of those
    // packed columns each, channels 64 b + 4 l + 2 h + j (h = ch % 2) for
    // lane l's product j; they are written at ch * 32 + 2 l + j all the same,
    // so that a row's writes stay contiguous, and the epilogue reorders.
    static_assert(!PACK64 || WN == 32, "packing for 64-channel wavefronts read by 32-channel ones");
    const int acc_col = ch * WN + l16 * NT;
    // Flush: add a unit's products into the tile sums (as in
    // k_conv_mfma_stream: one vector read-modify-write per row, padding rows
    // into the spare row TM, reads batched ahead of the writes).
    auto flush = [&](int unit) {
        const int slot = unit & (RING - 1);
        const bool first = unit < CU;  // a centre unit: its rows' first sums
        using Row = float __attribute__((ext_vector_type(NT)));
#pragma unroll
        for (int q0 = 0; q0 < QB; q0 += QF) {
            Row * dst[QF][4];
            Row v[QF][4];
#pragma unroll
            for (int qq = 0; qq < QF; ++qq) {
                const ushort4 d = *(const ushort4 *) &s_rdst[slot][(rh + RG * (q0 + qq)) * 16 + lg * 4];
                const int rows[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[qq][i] = (Row *) (s_acc + rows[i] * BN + acc_col);
            }
            if (first) {
#pragma unroll
                for (int qq = 0; qq < QF; ++qq)
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[qq][i] = (Row) 0.0f;
            } else {
#pragma unroll
                for (int qq = 0; qq < QF; ++qq)
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[qq][i] = *dst[qq][i];
            }
#pragma unroll
            for (int qq = 0; qq < QF; ++qq)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) v[qq][i][nt] += acc[q0 + qq][nt][i];
                    *dst[qq][i] = v[qq][i];
                }
#pragma unroll
            for (int qq = 0; qq < QF; ++qq)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[q0 + qq][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };

    // Block 0: every fetch of its DEPTH steps issued first, in the order the
    // main loop issues them (step r: A piece, then weights), so that the
    // loop's memory waits, which must hold for its first pass as for the
    // later ones, stay those of a full DEPTH-step look-ahead; then the A of
    // steps 0 and 1 into LDS slots 0 and 1 (one round trip for the block).
    target(0, 0);
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) {
        load_a(ra[r], r);
        load_b(rb[r], r);
    }
    store_a(0, ra[0]);
    store_a(1, ra[1]);
    lds_barrier();
    read_a(af[0], 0);

    int aslot = 0;  // LDS slot of the current step's A (step g: g % 3)
    for (int cb = 0; cb < U; cb += UPB) {
#pragma unroll
        for (int j = 0; j < UPB; ++j) {
            list_store(cb + 2 * UPB + j, lv[j]);
            lv[j] = list_load(cb + 3 * UPB + j);
        }
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
                const int s1 = aslot == 2 ? 0 : aslot + 1;  // next step's A
                const int s2 = s1 == 2 ? 0 : s1 + 1;        // step after: held step g-1
                // Fragments of the next step (stored two steps ago, published
                // by the previous step's barrier).
                read_a(af[(r + 1) & 1], s1);
                // A of step g + 2 (fetched DEPTH - 2 steps ago) into the slot
                // whose fragments every wavefront read before the last
                // barrier.  Both LDS operations are issued ahead of the MFMAs
                // so that they run under them, and so is the fetch of step
                // g + DEPTH's A into the register stored two steps ago (0.7 %
                // faster than after the MFMAs).
                store_a(s2, ra[(r + 2) % DEPTH]);
                load_a(ra[r], r);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < QB; ++q)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        acc[q][nt] = Mfma<DT>::mac(af[r & 1][q], rb[r][nt], acc[q][nt]);
                // Refill: the next block's weights in place of the ones just
                // used.
                load_b(rb[r], r);
                aslot = s1;
                lds_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (UPB > 1) {
                    if (r % SPU == SPU - 1 && cb + r / SPU < U) flush(cb + r / SPU);
                    if (r % SPU == SPU - 1) {
#pragma unroll
                        for (int q = 0; q < QB; ++q)
#pragma unroll
                            for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
                    }
                }
            }
            s0 += DEPTH;
        } while (s0 < KS);
        if constexpr (UPB == 1) flush(cb);
    }
    // Epilogue: bias, one rounding to the storage type; then the optional
    // row norm (+ SiLU) or residual add on the rounded values, rounded again.
    // A row's CHUNKS 16-byte chunks sit in CHUNKS consecutive lanes (each
    // thread keeps its chunk column on every pass), so the norm's sums are
    // DPP row reductions over those lanes (a DPP row is 16 lanes); every
    // thread takes part in them (rows past n are computed and not stored).
    // Bias, scale and shift are fetched before the barrier so that their
    // latency overlaps the last accumulator flush; the residual chunks were
    // fetched at the start.
    static_assert(CHUNKS == 16 || BN != 128, "a row's chunks fill one DPP row (the norm runs for BN = 128 only)");
    // Missing scale / shift are 1 and 0 (exact in r * g + b).
    float bv[8], gv[8], sv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        bv[u] = bias != nullptr ? bias[col0 + cc + u] : 0.0f;
        gv[u] = epi.gamma != nullptr ? epi.gamma[col0 + cc + u] : 1.0f;
        sv[u] = epi.beta != nullptr ? epi.beta[col0 + cc + u] : 0.0f;
    }
    lds_barrier();
    // One copy of the pass loop per epilogue kind, so that no kind pays for
    // another's arithmetic.
    auto passes = [&](auto mode_c, auto silu_c) {
        constexpr int MODE = decltype(mode_c)::value;
        constexpr bool SILU = decltype(silu_c)::value;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int rr = rr0 + p * (NTHR / CHUNKS);
            const int64_t row = row0 + rr;
            // Whole 16-byte chunks through the packed conversions: sum +
            // bias, rounded to the storage type (and widened again).
            float v[8];
            if constexpr (PACK64) {
                // Channels cc .. cc + 7 (64 b + 4 l + j, l = 2 q', 2 q' + 1):
                // j = 0, 1 at 64 b + 4 q' .. + 3, j = 2, 3 at 64 b + 32 + 4 q'.
                const int c0 = rr * BN + (cc & ~63) + (cc & 63) / 2;
                const float4 lo = *(const float4 *) &s_acc[c0];
                const float4 hi = *(const float4 *) &s_acc[c0 + 32];
                const float t8[8] = {lo.x, lo.y, hi.x, hi.y, lo.z, lo.w, hi.z, hi.w};
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = t8[u] + bv[u];
            } else {
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = s_acc[rr * BN + cc + u] + bv[u];
            }
            int4 o = pack_chunk<DT>(v);
            if constexpr (MODE == kEpiNorm) {
                unpack_chunk<DT>(o, v);
                float sum = 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u) sum += v[u];
                const float mean = row16_sum(sum) / (float) BN;
                float q = 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u) q += (v[u] - mean) * (v[u] - mean);
                const float inv = 1.0f / sqrtf(row16_sum(q) / (float) BN + epi.eps);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    float r = (v[u] - mean) * inv;
                    r = r * gv[u] + sv[u];
                    if constexpr (SILU) r = r * __builtin_amdgcn_rcpf(1.0f + __expf(-r));
                    v[u] = r;
                }
                o = pack_chunk<DT>(v);
            } else if constexpr (MODE == kEpiAdd) {
                float rv[8];
                unpack_chunk<DT>(o, v);
                unpack_chunk<DT>(res[p].v, rv);
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] += rv[u];
                o = pack_chunk<DT>(v);
            }
            if (row < n) *(int4 *) (y + row * co + col0 + cc) = o;
        }
    };
    using kNone = std::integral_constant<int, kEpiNone>;
    using kNorm = std::integral_constant<int, kEpiNorm>;
    using kAdd = std::integral_constant<int, kEpiAdd>;
    if (epi.mode == kEpiNorm) {
        if constexpr (BN == 128) {
            if (epi.silu) {
                passes(kNorm(), std::true_type());
            } else {
                passes(kNorm(), std::false_type());
            }
        }
    } else if (epi.mode == kEpiAdd) {
        passes(kAdd(), std::false_type());
    } else {
        passes(kNone(), std::false_type());
    }
}

// ---------------------------------------------------------------------------
// Output-stationary MFMA kernel for Ci = 64 (bf16 / fp16 storage).
//
// The compacted kernels add each 128-pair unit's products into fp32 tile sums
// in LDS; with Ci = 64 a unit is only two K steps, so that read-modify-write
// (Co x 8 bytes per pair) costs more than the unit's MFMAs.  Here every row's
// sums stay in registers for all 27 offsets: a block owns one 256-row map
// tile (4 wavefronts x 64 rows, lane = row), a wavefront 4 row blocks of 16
// x all Co = 64 channels.  For offset k each row's source is read from the
// tile's pair list for k (its rank among the tile's rows with a neighbour at
// k comes from ballots of the row masks), and the 16 source rows of a row
// block are loaded straight into MFMA operand order (lane i + 16 c: chunk c
// of row i's 64-byte K step); a row without a neighbour at k multiplies
// zeros.  (Loading each row's 64 bytes with four neighbouring lanes and
// moving them to operand order with ds_bpermute, 4 per fragment, measured
// 15 % slower: config 4, 1.196 -> 1.036 ms.)  The loads are raw buffer loads over x: a missing neighbour gets an
// offset past the buffer's end, which the hardware answers with zeros and no
// memory request, so no branch guards a load and the compiler's memory waits
// keep the two-offset look-ahead (a guarded load made it wait for each
// offset's loads almost at once).  The offset's 8 KB of weights are shared
// through a double-buffered LDS slot: one barrier per offset.  Each row's 27 sources are fetched in one
// round trip at the start; operand loads run two offsets ahead.  No unit
// lists, no tile sums, no flushes: the MFMA rows include the rows without a
// neighbour (27 N row-offsets against P), which is the price of keeping the
// sums in registers.  (Sorting each tile's rows by mask, so that 16-row
// blocks without a neighbour at k could be skipped, measured slower.)
// ---------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256, 2) k_conv_os64(const typename Store<DT>::T * __restrict__ x,
                                                      const int32_t * __restrict__ pair_src,
                                                      const int32_t * __restrict__ tile_off,
                                                      const uint32_t * __restrict__ mask,
                                                      const typename Store<DT>::T * __restrict__ w16,
                                                      const float * __restrict__ bias,
                                                      typename Store<DT>::T * __restrict__ y, int64_t n) {
    using T = typename Store<DT>::T;
    using V = typename Mfma<DT>::V;
    constexpr int CI = 64, CO = 64;
    // The weights come in conv_stream_group(64, 64)'s packing, which this
    // kernel reads with g = 4: lane l16 owns channels 4 l16 .. 4 l16 + 3.
    static_assert(64 / (TSH_STREAM_WAVES / TSH_STREAM_ROW_GROUPS) / 16 == 4,
                  "k_conv_os64 needs the 64-channel grouped packing with g = 4");
    constexpr int QB = 4;                      // row blocks per wavefront
    constexpr int NT = CO / 16;                // column tiles (grouped packing: lane's NT columns adjacent)
    constexpr int WSLOT = (CI / 8) * CO * 8;   // weight elements per offset
    constexpr int WPT = WSLOT * 2 / 16 / 256;  // 16-byte weight pieces per thread per offset
    static_assert(WPT == 2, "8 KB of weights per offset over 256 threads");
    __shared__ __attribute__((aligned(16))) T s_w[2][WSLOT];
    __shared__ int32_t s_cnt[27][4];
    __shared__ int32_t s_off[27];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    const int64_t tile = xcd_remap(blockIdx.x, (int64_t) gridDim.x);
    const int64_t row0 = tile * kMapTile;
    const int64_t my_row = row0 + wave * 64 + lane;
    const uint32_t m = my_row < n ? mask[my_row] : 0u;
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    if (t < 27) s_off[t] = tile_off[tile * 27 + t];
    // Rows of each wavefront with a neighbour at k, for the ranks below.
#pragma unroll 1
    for (int k = 0; k < 27; ++k) {
        const int c = __popcll(__ballot((m >> k) & 1u));
        if (lane == 0) s_cnt[k][wave] = c;
    }
    // Weights of offsets 0 (into slot 0) and 1 (in registers).
    V wreg[WPT];
#pragma unroll
    for (int j = 0; j < WPT; ++j) wreg[j] = *(const V *) (w16 + (int64_t) (t + j * 256) * 8);
#pragma unroll
    for (int j = 0; j < WPT; ++j) *(V *) &s_w[0][(t + j * 256) * 8] = wreg[j];
#pragma unroll
    for (int j = 0; j < WPT; ++j) wreg[j] = *(const V *) (w16 + WSLOT + (int64_t) (t + j * 256) * 8);
    lds_barrier();

    // Source rows of this lane's row at every offset (or -1), all fetched
    // in one round trip: the row's rank in the tile's list for k is the
    // count of earlier rows with a neighbour at k.
    int32_t src[27];
#pragma unroll
    for (int k = 0; k < 27; ++k) {
        const uint64_t bk = __ballot((m >> k) & 1u);
        int base = 0;
        for (int w = 0; w < wave; ++w) base += s_cnt[k][w];
        src[k] = ((m >> k) & 1u) ? pair_src[s_off[k] + base + __popcll(bk & lt)] : -1;
    }
    // A fragments of offset k: row block q, K step f; lane i + 16 c holds 16
    // bytes (chunk c of the step) of row i of the block.  Byte offsets into x
    // per row block, prepared one offset before their loads so that the
    // shuffles' latency stays off the load path.
    constexpr int AHEAD = 2;  // offsets whose A loads are in flight
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc((void *) x, 0, (int) (n * CI * (int64_t) sizeof(T)), 0x00020000);
    V ra[AHEAD + 1][QB][2];
    uint32_t voff[QB];
    auto prep_a = [&](int32_t src) {
#pragma unroll
        for (int q = 0; q < QB; ++q) {
            const int32_t sq = __shfl(src, q * 16 + l16);
            voff[q] = sq >= 0 ? (uint32_t) sq * (uint32_t) (CI * sizeof(T)) + (uint32_t) lg * 16u : 0x80000000u;
        }
    };
    auto load_a = [&](V (&a)[QB][2]) {
#pragma unroll
        for (int q = 0; q < QB; ++q)
#pragma unroll
            for (int f = 0; f < 2; ++f)
                a[q][f] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(xres, voff[q] + f * 64u, 0, 0));
    };
    f32x4 acc[QB][NT];
#pragma unroll
    for (int q = 0; q < QB; ++q)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < AHEAD; ++k) {
        prep_a(src[k]);
        load_a(ra[k]);
    }
    prep_a(src[AHEAD]);
#pragma unroll
    for (int k = 0; k < 27; ++k) {
        const int cur = k & 1;
        const int ar = k % (AHEAD + 1);
        if (k + AHEAD < 27) load_a(ra[(k + AHEAD) % (AHEAD + 1)]);
        if (k + AHEAD + 1 < 27) prep_a(src[k + AHEAD + 1]);
        // Keeps the loads just issued ahead of this offset's weight reads and
        // MFMAs (the scheduler would interleave them).
        __builtin_amdgcn_sched_barrier(0);
        // Weight fragments of offset k: K step f, column tile nt.
        V bw[2][NT];
        const T * ws = &s_w[cur][0];
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) bw[f][nt] = *(const V *) (ws + ((f * 4 + lg) * CO + nt * 16 + l16) * 8);
#pragma unroll
        for (int q = 0; q < QB; ++q)
#pragma unroll
            for (int f = 0; f < 2; ++f) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[q][nt] = Mfma<DT>::mac(ra[ar][q][f], bw[f][nt], acc[q][nt]);
            }
        // Offset k + 1's weights into the other slot (read last at offset
        // k - 1, before the previous barrier); offset k + 2's into registers.
        if (k + 1 < 27) {
#pragma unroll
            for (int j = 0; j < WPT; ++j) *(V *) &s_w[cur ^ 1][(t + j * 256) * 8] = wreg[j];
        }
        if (k + 2 < 27) {
#pragma unroll
            for (int j = 0; j < WPT; ++j)
                wreg[j] = *(const V *) (w16 + (int64_t) (k + 2) * WSLOT + (int64_t) (t + j * 256) * 8);
        }
        lds_barrier();
    }
    // Epilogue: bias, round, store; lane holds rows 4 lg + i of each row
    // block, channels 4 l16 .. 4 l16 + 3 (grouped packing).
    float bv[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) bv[nt] = bias != nullptr ? bias[l16 * NT + nt] : 0.0f;
#pragma unroll
    for (int q = 0; q < QB; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t row = row0 + wave * 64 + q * 16 + lg * 4 + i;
            if (row >= n) continue;
            union {
                uint2 u;
                T h[4];
            } o;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) o.h[nt] = round_to_store<DT>(acc[q][nt][i] + bv[nt]);
            *(uint2 *) (y + row * CO + l16 * NT) = o.u;
        }
}

}  // namespace

hipError_t launch_conv_generic(int dtype, const void * x, const int32_t * nbr, const float * w32, const float * bias,
                               void * y, int64_t n, int ci, int co, hipStream_t s) {
    // Two rows per lane, or one (twice the blocks) when the whole conv is
    // fewer than 1024 tiles of 32 rows x 32 input channels x 64 outputs: the
    // GPU then runs short of blocks (config 1, 64 -> 64: 0.192 -> 0.169 ms;
    // larger convs measured slower with one row per lane).
    const int64_t tiles32 = (n + 31) / 32 * ((co + 63) / 64) * ((ci + 31) / 32);
    const int tm = tiles32 < 1024 ? 1 : 2;
    const dim3 grid((unsigned) ((n + 16 * tm - 1) / (16 * tm)), (unsigned) ((co + 63) / 64));
#define TSH_GENERIC(DTV, TYPE, TMV)                                                                           \
    k_conv_generic<DTV, TMV><<<grid, 256, 0, s>>>((const TYPE *) x, nbr, w32, bias, (TYPE *) y, n, ci, co)
    switch (dtype) {
        case kF32:
            if (tm == 2) TSH_GENERIC(kF32, float, 2); else TSH_GENERIC(kF32, float, 1);
            break;
        case kF16:
            if (tm == 2) TSH_GENERIC(kF16, _Float16, 2); else TSH_GENERIC(kF16, _Float16, 1);
            break;
        case kBF16:
            if (tm == 2) TSH_GENERIC(kBF16, uint16_t, 2); else TSH_GENERIC(kBF16, uint16_t, 1);
            break;
        default:
            return hipErrorInvalidValue;
    }
#undef TSH_GENERIC
    return hipGetLastError();
}

bool conv_mfma_supported(int dtype, int ci, int co) {
    return (dtype == kF16 || dtype == kBF16) && ci > 0 && co > 0 && ci % 32 == 0 &&
           (co % 64 == 0 || co == 16 || co == 32);
}

hipError_t launch_conv_mfma_masked(int dtype, const void * x, const int32_t * nbr, const uint32_t * mask,
                                   const void * w16, const float * bias, void * y, int64_t n, int ci, int co,
                                   hipStream_t s) {
    if (!conv_mfma_supported(dtype, ci, co)) {
        return hipErrorInvalidValue;
    }
    const int bn = (co % 128 == 0) ? 128 : (co % 64 == 0 ? 64 : co);
    const int bm = bn >= 64 ? 64 : 128;
    const int64_t row_tiles = (n + bm - 1) / bm;
    const int64_t col_tiles = co / bn;
    const int64_t grid = row_tiles * col_tiles;
    if (grid > 0x7fffffffLL) {
        return hipErrorInvalidValue;
    }
#define TSH_LAUNCH(DTV, TYPE, BNV, WRV)                                                                       \
    k_conv_mfma_masked<DTV, BNV, WRV><<<(unsigned) grid, 256, 0, s>>>((const TYPE *) x, nbr, mask,               \
                                                                       (const TYPE *) w16, bias, (TYPE *) y, n, ci, \
                                                                       co, col_tiles)
    if (dtype == kBF16) {
        if (bn == 128) TSH_LAUNCH(kBF16, uint16_t, 128, 2);
        else if (bn == 64) TSH_LAUNCH(kBF16, uint16_t, 64, 2);
        else if (bn == 32) TSH_LAUNCH(kBF16, uint16_t, 32, 4);
        else TSH_LAUNCH(kBF16, uint16_t, 16, 4);
    } else {
        if (bn == 128) TSH_LAUNCH(kF16, _Float16, 128, 2);
        else if (bn == 64) TSH_LAUNCH(kF16, _Float16, 64, 2);
        else if (bn == 32) TSH_LAUNCH(kF16, _Float16, 32, 4);
        else TSH_LAUNCH(kF16, _Float16, 16, 4);
    }
#undef TSH_LAUNCH
    return hipGetLastError();
}


bool conv_wide_supported(int ci, int co) { return co % 256 == 0 && ci % 128 == 0; }

int conv_stream_group(int ci, int co) {
    // 256-channel blocks over half map tiles and 128-channel blocks run
    // k_conv_mfma_wreg (2 row groups x 4 channel groups of 64 or 32),
    // 64-channel blocks k_conv_mfma_stream; 16- and 32-channel outputs are
    // one block of co channels there.
    if (conv_wide_supported(ci, co)) return 256 / 4 / 16;
    if (co % 128 == 0) return 128 / 4 / 16;
    if (co == 16 || co == 32) return co / (TSH_STREAM_WAVES / TSH_STREAM_ROW_GROUPS) / 16;
    return 64 / (TSH_STREAM_WAVES / TSH_STREAM_ROW_GROUPS) / 16;
}

bool conv_stream_supported(int dtype, int ci, int co) {
    // A unit (Ci/32 K steps) spans a whole number of 4-step blocks, or two
    // units (Ci = 64) make one block.
    return conv_mfma_supported(dtype, ci, co) && (co % 64 == 0 || co == 16 || co == 32) &&
           (ci % 128 == 0 || ci == 64);
}

namespace {
template <int DT, int BN, int DEPTH, int NW, int RG, int UPB, bool PACK64 = false>
hipError_t launch_stream_t(const void * x, const int32_t * pair_src, const uint8_t * pair_dst,
                           const int32_t * tile_off, const int32_t * tile_counts, const uint32_t * mask,
                           const void * w16, const float * bias, void * y, int64_t n, int ci, int co, hipStream_t s,
                           const ConvEpilogue & epi, int layout_sel = 0, const int32_t * layout_stats = nullptr) {
    using T = typename Store<DT>::T;
    const int64_t tiles = (n + kMapTile - 1) / kMapTile;
    const int64_t col_tiles = co / BN;
    const int64_t grid = tiles * col_tiles * (BN == 256 ? 2 : 1);
    if (grid > 0x7fffffffLL) {
        return hipErrorInvalidValue;
    }
    if constexpr (BN == 256) {
        // Half map tiles (the tile sums of 128 rows x 256 channels fill the
        // LDS as 256 x 128 do); 4-step blocks keep the weight ring in the
        // register budget.
        if (epi.mode == kEpiNorm || UPB != 1 || ci % 128 != 0) return hipErrorInvalidValue;
        k_conv_mfma_wreg<DT, 256, 2, 1, 4, kMapTile / 2, 8><<<(unsigned) grid, 512, 0, s>>>(
            (const T *) x, pair_src, pair_dst, tile_off, tile_counts, mask, (const T *) w16, bias, (T *) y, n, ci,
            co, epi, layout_sel, layout_stats);
    } else if constexpr (BN == 128) {
        // Weights in registers; blocks of 8 steps when a unit is a whole
        // number of them (Ci % 256 == 0), else 4.
        if (UPB == 1 && (ci % 256 != 0 || (PACK64 && ci == 256))) {
            // 4-step units (Ci = 128, 384, ...): half map tiles, 64-pair
            // units and 4 wavefronts, so that two blocks (81 KB of LDS each)
            // share a CU and one's barriers overlap the other's MFMAs
            // (config 2: 0.636 -> 0.602 ms; 8-step units measured 1.5 %
            // slower this way and keep whole tiles).  On the sparse sets that
            // take this layout for Co % 256 == 0, Ci = 256 runs half tiles
            // too (the encoder's 256 -> 256 and the up-blocks' 256 -> 1024:
            // 1.4-3.6 % faster; Ci = 512 was 4-10 % slower).
            const int64_t hgrid = tiles * col_tiles * 2;
            if (hgrid > 0x7fffffffLL) return hipErrorInvalidValue;
            k_conv_mfma_wreg<DT, BN, 1, 1, 4, kMapTile / 2, 4, 1, PACK64><<<(unsigned) hgrid, 256, 0, s>>>(
                (const T *) x, pair_src, pair_dst, tile_off, tile_counts, mask, (const T *) w16, bias, (T *) y, n, ci,
                co, epi, layout_sel, layout_stats);
        } else if (UPB == 1) {
            k_conv_mfma_wreg<DT, BN, 2, UPB, UPB == 1 ? 8 : 4, kMapTile, 8, 1, PACK64><<<(unsigned) grid, 512, 0, s>>>(
                (const T *) x, pair_src, pair_dst, tile_off, tile_counts, mask, (const T *) w16, bias, (T *) y, n,
                ci, co, epi, layout_sel, layout_stats);
        } else {
            if (PACK64 || layout_sel != 0) return hipErrorInvalidValue;  // Ci = 64 never takes the 256-column layout
            k_conv_mfma_wreg<DT, BN, 2, UPB, 4, kMapTile, 8><<<(unsigned) grid, 512, 0, s>>>(
                (const T *) x, pair_src, pair_dst, tile_off, tile_counts, mask, (const T *) w16, bias, (T *) y, n,
                ci, co, epi, 0, nullptr);
        }
    } else {
        if (epi.mode != kEpiNone) return hipErrorInvalidValue;  // 64-channel blocks: plain epilogue only
        k_conv_mfma_stream<DT, BN, DEPTH, NW, RG, UPB><<<(unsigned) grid, 64 * NW, 0, s>>>(
            (const T *) x, pair_src, pair_dst, tile_off, tile_counts, (const T *) w16, bias, (T *) y, n, ci, co,
            col_tiles);
    }
    return hipGetLastError();
}

template <int DT>
hipError_t launch_stream_dt(const void * x, const int32_t * pair_src, const uint8_t * pair_dst,
                            const int32_t * tile_off, const int32_t * tile_counts, const uint32_t * mask,
                            const void * w16, const float * bias, void * y, int64_t n, int ci, int co, hipStream_t s,
                            const ConvEpilogue & epi, const int32_t * layout_stats) {
    const bool wide = co % 128 == 0;
    const bool pair = ci == 64;  // two 2-step units per 4-step block
#define TSH_STREAM(BNV, UV)                                                                                      \
    launch_stream_t<DT, BNV, 4, TSH_STREAM_WAVES, TSH_STREAM_ROW_GROUPS, UV>(x, pair_src, pair_dst, tile_off,     \
                                                                           tile_counts, mask, w16, bias, y, n, ci, \
                                                                           co, s, epi)
    if (conv_wide_supported(ci, co) && epi.mode != kEpiNorm) {
        // The 256-column layout or the 128-column one, as the kernel map's
        // statistics decide on the device (layout_sel): both are launched,
        // over the same 64-channel weight packing, and the one not chosen
        // returns at once.  A row's sums are formed in the same order in both.
        const hipError_t e = launch_stream_t<DT, 256, 4, TSH_STREAM_WAVES, TSH_STREAM_ROW_GROUPS, 1>(
            x, pair_src, pair_dst, tile_off, tile_counts, mask, w16, bias, y, n, ci, co, s, epi, 1, layout_stats);
        if (e != hipSuccess) return e;
        return launch_stream_t<DT, 128, 4, TSH_STREAM_WAVES, TSH_STREAM_ROW_GROUPS, 1, true>(
            x, pair_src, pair_dst, tile_off, tile_counts, mask, w16, bias, y, n, ci, co, s, epi, 2, layout_stats);
    }
    if (wide) return pair ? TSH_STREAM(128, 2) : TSH_STREAM(128, 1);
    if (co == 16) return pair ? TSH_STREAM(16, 2) : TSH_STREAM(16, 1);
    if (co == 32) return pair ? TSH_STREAM(32, 2) : TSH_STREAM(32, 1);
    return pair ? TSH_STREAM(64, 2) : TSH_STREAM(64, 1);
#undef TSH_STREAM
}
}  // namespace

// The gathers address x through a buffer resource whose byte range is an
// int32: up to 2^31 / 128 rows (16.7M voxels); beyond that the compacted
// streamed kernel runs instead.
bool conv_os_supported(int dtype, int ci, int co, int64_t n) {
    return (dtype == kF16 || dtype == kBF16) && ci == 64 && co == 64 && n > 0 && n <= (int64_t) INT32_MAX / 128;
}

hipError_t launch_conv_os(int dtype, const void * x, const int32_t * pair_src, const int32_t * tile_off,
                          const uint32_t * mask, const void * w16, const float * bias, void * y, int64_t n, int ci,
                          int co, hipStream_t s) {
    if (!conv_os_supported(dtype, ci, co, n)) return hipErrorInvalidValue;
    const int64_t tiles = (n + kMapTile - 1) / kMapTile;
    if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
    if (dtype == kBF16) {
        k_conv_os64<kBF16><<<(unsigned) tiles, 256, 0, s>>>((const uint16_t *) x, pair_src, tile_off, mask,
                                                            (const uint16_t *) w16, bias, (uint16_t *) y, n);
    } else {
        k_conv_os64<kF16><<<(unsigned) tiles, 256, 0, s>>>((const _Float16 *) x, pair_src, tile_off, mask,
                                                           (const _Float16 *) w16, bias, (_Float16 *) y, n);
    }
    return hipGetLastError();
}

hipError_t launch_conv_mfma_stream(int dtype, const void * x, const int32_t * pair_src, const uint8_t * pair_dst,
                                   const int32_t * tile_off, const int32_t * tile_counts, const uint32_t * mask,
                                   const void * w16, const float * bias, void * y, int64_t n, int ci, int co,
                                   hipStream_t s, const ConvEpilogue & epi, const int32_t * layout_stats) {
    if (!conv_stream_supported(dtype, ci, co) || (epi.mode == kEpiNorm && co != 128) ||
        (epi.mode != kEpiNone && co % 128 != 0) || layout_stats == nullptr) {
        return hipErrorInvalidValue;
    }
    if (dtype == kBF16) {
        return launch_stream_dt<kBF16>(x, pair_src, pair_dst, tile_off, tile_counts, mask, w16, bias, y, n, ci, co, s,
                                       epi, layout_stats);
    }
    return launch_stream_dt<kF16>(x, pair_src, pair_dst, tile_off, tile_counts, mask, w16, bias, y, n, ci, co, s, epi,
                                  layout_stats);
}

}  // namespace tsh
