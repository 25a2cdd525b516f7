// tsh_internal.h - internal declarations of the MI355X sparse-voxel backend.
//
// Not part of the C ABI.  Shared between the backend translation unit
// (vtable, memory, caches) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "trellis_sparse_hip.h"

namespace tsh {

enum Dtype : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

inline size_t dtype_bytes(int dt) { return dt == kF32 ? 4u : 2u; }

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet), usable on host and device.
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return (uint16_t) ((u >> 16) | 0x40u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t) (u >> 16);
}
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t) h << 16);
}

// Storage-type load/store with fp32 arithmetic.
template <int DT> struct Store;
template <> struct Store<kF32> {
    using T = float;
    __device__ static float ld(const T * p, int64_t i) { return p[i]; }
    __device__ static void st(T * p, int64_t i, float v) { p[i] = v; }
    __device__ static void st_signed(T * p, int64_t i, float v) { p[i] = v; }
};
// st_signed: the same rounding, except that a positive value which rounds to
// +0 is stored as the smallest positive subnormal, so that v > 0 holds for
// the stored value exactly when it held for v.  Used where a sign decides
// something downstream (uploads and the linear slot, whose 8-wide output is
// the subdivide logits: child s exists iff logit > 0).
template <> struct Store<kF16> {
    using T = _Float16;
    __device__ static float ld(const T * p, int64_t i) { return (float) p[i]; }
    __device__ static void st(T * p, int64_t i, float v) { p[i] = (_Float16) v; }
    __device__ static void st_signed(T * p, int64_t i, float v) {
        const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16) v);
        p[i] = __builtin_bit_cast(_Float16, (uint16_t) ((v > 0.0f && h == 0) ? 1 : h));
    }
};
template <> struct Store<kBF16> {
    using T = uint16_t;
    __device__ static float ld(const T * p, int64_t i) { return bf16_to_f32(p[i]); }
    // Round to nearest even with the hardware conversion (NaN stays NaN).
    __device__ static void st(T * p, int64_t i, float v) { p[i] = __builtin_bit_cast(uint16_t, (__bf16) v); }
    __device__ static void st_signed(T * p, int64_t i, float v) {
        const uint16_t h = __builtin_bit_cast(uint16_t, (__bf16) v);
        p[i] = (v > 0.0f && h == 0) ? (uint16_t) 1 : h;
    }
};

// A 16-byte chunk of 16-bit storage values (8 of them) to fp32 and back,
// with round-to-nearest-even on the way back.
template <int DT> __device__ inline void unpack_chunk(const int4 & c, float * v) {
    static_assert(DT != kF32, "16-bit storage");
    const uint32_t w[4] = {(uint32_t) c.x, (uint32_t) c.y, (uint32_t) c.z, (uint32_t) c.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if constexpr (DT == kBF16) {
            v[2 * k] = __builtin_bit_cast(float, w[k] << 16);
            v[2 * k + 1] = __builtin_bit_cast(float, w[k] & 0xffff0000u);
        } else {
            v[2 * k] = (float) __builtin_bit_cast(_Float16, (uint16_t) (w[k] & 0xffffu));
            v[2 * k + 1] = (float) __builtin_bit_cast(_Float16, (uint16_t) (w[k] >> 16));
        }
    }
}

template <int DT> __device__ inline typename Store<DT>::T round_to_store(float v) {
    if constexpr (DT == kBF16) {
        return __builtin_bit_cast(uint16_t, (__bf16) v);
    } else {
        return (typename Store<DT>::T) v;
    }
}

template <int DT> __device__ inline int4 pack_chunk(const float * v) {
    static_assert(DT != kF32, "16-bit storage");
    union {
        int4 c;
        typename Store<DT>::T h[8];
    } u;
#pragma unroll
    for (int k = 0; k < 8; ++k) u.h[k] = round_to_store<DT>(v[k]);
    return u.c;
}

// Work split of a rulebook build / conv: rows per tile of the kernel map.
constexpr int kMapTile = 256;
constexpr int kBrickCells = 64;  // 4x4x4 cells per brick
// Build counters: [1] duplicate flag, [4] internal-error flags, the brick
// count (statistics) summed over kBrickCounters counters from
// counters[kBrickCounter], and the conv layout statistics from
// counters[kLayoutStats]: over the map tiles, the offsets with pairs (summed
// over kLayoutSlots counters), then the offsets with more than kMapTile / 2
// pairs (the next kLayoutSlots).  Spread over slots because one address that
// every tile adds to serialises the kernel map.
constexpr int kBrickCounters = 64;
constexpr int kBrickCounter = 64;
constexpr int kLayoutSlots = 64;
constexpr int kLayoutStats = kBrickCounter + kBrickCounters;
constexpr int kCounterInts = kLayoutStats + 2 * kLayoutSlots;

struct Backend;

// Device-side scratch handed out by the backend's pool.
struct DevMem {
    void * ptr = nullptr;
    size_t bytes = 0;
};

}  // namespace tsh

// Opaque ABI types, defined here for the backend.
struct trellis_sparse_buffer {
    void * ptr;
    size_t count;   // elements
    size_t bytes;   // count * element size
    size_t cap;     // bytes actually reserved (pool size class)
    int dtype;      // tsh::Dtype of the storage, or -1 for raw int32
};

struct trellis_sparse_rulebook {
    int64_t n;
    int32_t * coords;        // device [n][4]
    tsh::DevMem coords_mem;  // owned copy (empty when borrowed from a C2S map)
    // Brick hash: open-addressed uint64 keys (b, x>>2, y>>2, z>>2)+1 -> brick index.
    int64_t table_slots;
    tsh::DevMem table;       // brick table: [table_slots] x {uint64 key, int32 idx, pad}
    tsh::DevMem pool;        // int32  [cap_bricks][64] voxel rows, -1 = empty
    tsh::DevMem counters;    // int32  [kCounterInts]: [1] duplicate flag, [4] internal-error flags, [64..] brick counts, [128..] layout statistics
    // Kernel map.
    tsh::DevMem nbr;         // int32  [n][27]
    tsh::DevMem mask;        // uint32 [n] bit k set when nbr[i][k] >= 0
    int64_t n_tiles;         // ceil(n / kMapTile)
    tsh::DevMem tile_counts; // int32  [n_tiles][27]
    tsh::DevMem tile_off;    // int32  [n_tiles][27] start of (tile, k) in the pair arrays
    tsh::DevMem pair_src;    // int32  [n_tiles][kMapTile * 27]: per tile, offsets ascending, dst ascending
    tsh::DevMem pair_dst;    // uint8  [n_tiles][kMapTile * 27]: destination row within the tile
};

struct trellis_sparse_c2s_device_map {
    int64_t n;
    int64_t n_parent;    // rows of the parent level (0 for a coordinates-only map)
    tsh::DevMem coords;  // int32 [n][4]
    tsh::DevMem parent;  // int32 [n]
    tsh::DevMem subidx;  // int32 [n]
    tsh::DevMem child;   // int32 [n_parent][8] row of each child slot or -1 (maps built by S2C)
};

namespace tsh {

// ---------------------------------------------------------------------------
// Kernel launchers (defined in the kernel translation units).  All enqueue on
// `stream` and return hipSuccess or the launch error.
// ---------------------------------------------------------------------------

// Voxel hash + kernel map (kernels_map.hip).
hipError_t launch_fill_i32(int32_t * p, int64_t count, int32_t value, hipStream_t s);
// Brick table keys to 0 and the build counters (kCounterInts) to 0, one launch.
// Also sets the pool's spare row (brick pool_empty_brick(n)) to -1.
hipError_t launch_hash_clear(uint64_t * table, int64_t slots, int32_t * counters, int32_t * pool, int64_t n,
                             hipStream_t s);
// Inserts the voxels' bricks, numbers the new ones (block b's from b * 256)
// and sets their pool rows to -1.
hipError_t launch_brick_insert(const int32_t * coords, int64_t n, uint64_t * table,
                               int64_t slots, int32_t * counters, int32_t * pool, hipStream_t s);
// Pool rows for n voxels (one per voxel slot of the insert's blocks); the
// spare row of -1 sits at index pool_empty_brick(n).
int64_t pool_empty_brick(int64_t n);

hipError_t launch_voxel_insert(const int32_t * coords, int64_t n, const uint64_t * table,
                               int64_t slots, int32_t * pool, int32_t * counters, hipStream_t s);
// Neighbour table, masks, per-(tile, offset) counts and list starts, and the
// pair lists in one pass.  Tile t's lists fill the start of its region
// [t * kMapTile * 27, (t + 1) * kMapTile * 27) of the pair arrays.
hipError_t launch_map_tiles(const int32_t * coords, int64_t n, const uint64_t * table,
                            int64_t slots, const int32_t * pool, int32_t * nbr, uint32_t * mask,
                            int32_t * tile_counts, int32_t * tile_off, int32_t * pair_src, uint8_t * pair_dst,
                            int32_t * counters, hipStream_t s);

// Convolution (kernels_conv.hip).  Weight layouts are produced by the backend.
//  generic: w32 fp32 [27][ci][co]
//  mfma:    w16 storage-type [27][ci/8][co][8]
hipError_t launch_conv_generic(int dtype, const void * x, const int32_t * nbr, const float * w32,
                               const float * bias, void * y, int64_t n, int ci, int co, hipStream_t s);
bool conv_mfma_supported(int dtype, int ci, int co);
hipError_t launch_conv_mfma_masked(int dtype, const void * x, const int32_t * nbr, const uint32_t * mask,
                                   const void * w16, const float * bias, void * y, int64_t n, int ci, int co,
                                   hipStream_t s);
// Epilogue of the 128-channel compacted conv: after bias and the rounding to
// the storage type, optionally a row norm (+ SiLU) over whole rows (co ==
// 128, one block holds every channel of its rows) or a residual add
// (rounded again), as the slot sequences conv -> row_norm(_silu) and
// conv -> add compute them.
struct ConvEpilogue {
    int mode = 0;  // kEpiNone, kEpiNorm, kEpiAdd
    int silu = 0;
    float eps = 0.0f;
    const float * gamma = nullptr;
    const float * beta = nullptr;
    const void * residual = nullptr;  // storage type [n][co]
};
enum { kEpiNone = 0, kEpiNorm = 1, kEpiAdd = 2 };

// Streamed compacted schedule over the tile-major pair lists (needs ci == 64 or ci % 128 == 0).
// Its weights use the grouped packing: [27][ci/8][co][8] whose packed column
// b*16g + nt*16 + l holds channel b*16g + l*g + nt, g = conv_stream_group(ci, co).
// Co % 256 == 0 with Ci % 128 == 0 (conv_wide_supported) runs 256-channel
// blocks over half map tiles (which need the row masks) or 128-channel
// blocks over whole tiles, as the rulebook's layout statistics
// (counters + kLayoutStats, written by the kernel map) decide on the device.
bool conv_wide_supported(int ci, int co);
int conv_stream_group(int ci, int co);
bool conv_stream_supported(int dtype, int ci, int co);
hipError_t launch_conv_mfma_stream(int dtype, const void * x, const int32_t * pair_src, const uint8_t * pair_dst,
                                   const int32_t * tile_off, const int32_t * tile_counts, const uint32_t * mask,
                                   const void * w16, const float * bias, void * y, int64_t n, int ci, int co,
                                   hipStream_t s, const ConvEpilogue & epi, const int32_t * layout_stats);

// Output-stationary MFMA conv for Ci = Co = 64 over the tile-major pair lists
// and the row masks (weights in the grouped packing of conv_stream_group(64, 64)).
bool conv_os_supported(int dtype, int ci, int co, int64_t n);
hipError_t launch_conv_os(int dtype, const void * x, const int32_t * pair_src, const int32_t * tile_off,
                          const uint32_t * mask, const void * w16, const float * bias, void * y, int64_t n, int ci,
                          int co, hipStream_t s);

// Everything else (kernels_misc.hip).
hipError_t launch_convert_from_f32(int dtype, const float * src, void * dst, int64_t count, hipStream_t s);
hipError_t launch_convert_to_f32(int dtype, const void * src, float * dst, int64_t count, hipStream_t s);
hipError_t launch_silu(int dtype, void * x, int64_t count, hipStream_t s);
hipError_t launch_add(int dtype, const void * a, const void * b, void * y, int64_t count, hipStream_t s);
hipError_t launch_row_norm(int dtype, const void * x, const float * gamma, const float * beta, void * y,
                           int64_t n, int c, float eps, int silu, hipStream_t s);
hipError_t launch_linear(int dtype, const void * x, const float * wt, const float * bias, void * y, int64_t n,
                         int ci, int co, int silu, hipStream_t s);
// MFMA linear (bf16/fp16; Ci = 64 or Ci % 128 == 0, Co % 64 == 0).  Weights
// [ci/8][co][8] in the storage type; packed column g*16j + nt*16 + l (within
// each group of 16j columns, j = linear_mfma_group(co)) holds channel
// g*16j + l*j + nt.  cus = the device's compute units (one block each).
int linear_mfma_group(int co);
bool linear_mfma_supported(int dtype, int ci, int co);
hipError_t launch_linear_mfma(int dtype, const void * x, const void * w16, const float * bias, void * y, int64_t n,
                              int ci, int co, int silu, int cus, hipStream_t s);
// The linear slots through the platform GEMM library (linear_lt.hip):
// 16-bit storage with Ci, Co >= 256 and n >= 2048; weights [co][ci] in the
// storage type.  linear_lt_run enqueues on s and returns true, or returns
// false with nothing enqueued (no plan for the shape, or the library refused).
// A non-null residual r (same layout as y, may be y) gives y = r + x W^T + b,
// added to the fp32 sums before the one rounding.
struct LinearLt;
bool linear_lt_wanted(int dtype, int64_t n, int ci, int co);
LinearLt * linear_lt_create();
void linear_lt_destroy(LinearLt * lt);
bool linear_lt_run(LinearLt * lt, int dtype, const void * x, const void * w16, const float * bias,
                   const void * residual, void * y, int64_t n, int ci, int co, int silu, void * workspace,
                   size_t workspace_bytes, hipStream_t s);
// Fused ConvNeXt MLP tail (kernels_block.hip): bf16/fp16, C = 64, 128 or 256.
// w0 [C/8][4C][8] and w2 [4C/8][C][8] in the storage type with the grouped
// column packing of the MFMA linear, groups g0 and g2 from convnext_mlp_groups.
bool convnext_mlp_supported(int dtype, int c);
void convnext_mlp_groups(int c, int * g0, int * g2);
hipError_t launch_convnext_mlp(int dtype, const void * x, const float * gamma, const float * beta, const void * w0,
                               const float * b0, const void * w2, const float * b2, const void * res, void * y,
                               int64_t n, int c, float eps, int cus, hipStream_t s);
// Spatial-to-channel downsample (kernels_s2c.hip).  flags: int32[8]; prep
// (scratch part of s2c_prep_part_bytes()) sets flags[0] to 1 or 0 (a
// negative coordinate) and flags[1..4] to the field maxima; heads sets
// flags[0] bit 1 on a repeated fine voxel.  The sort ping-pongs between buffers [0] and [1] of klo/khi/row
// (khi only when key_bits > 64) and reports which holds the result.
size_t s2c_prep_part_bytes();
hipError_t launch_s2c_prep(const int32_t * coords, int64_t n, int32_t * subidx, int32_t * part, int32_t * flags,
                           hipStream_t s);
int s2c_key_shape(const int32_t * maxima, int shifts[4]);  // returns the key width in bits
int64_t s2c_sort_tiles(int64_t n);
size_t s2c_sort_tmp_bytes(int64_t n);
hipError_t launch_s2c_sort(const int32_t * coords, int64_t n, const int shifts[4], int key_bits, uint64_t * klo[2],
                           uint64_t * khi[2], int32_t * row[2], int32_t * hist, int32_t * offs, int32_t * total,
                           void * tmp, int * out_buffer, hipStream_t s);
hipError_t launch_s2c_heads(const uint64_t * klo, const uint64_t * khi, int64_t n, int32_t * head, int32_t * flags,
                            hipStream_t s);
hipError_t launch_s2c_emit(const int32_t * coords, const int32_t * row, const int32_t * subidx, const int32_t * head,
                           const int32_t * excl, int64_t n, int32_t * parent, int32_t * coarse, int32_t * child,
                           hipStream_t s);
hipError_t launch_s2c_pack(int dtype, const void * x, const int32_t * child, void * y, int64_t m, int co,
                           hipStream_t s);
hipError_t launch_s2c_skip_mean(int dtype, const void * x, const int32_t * child, void * y, int64_t m, int ci,
                                int co, hipStream_t s);

// Narrow MFMA linear (bf16/fp16, Co <= 16, Ci a power of two in 32..1024):
// weights [co][ci] in the storage type.
bool linear_narrow_supported(int dtype, int ci, int co);
hipError_t launch_linear_narrow(int dtype, const void * x, const void * w16, const float * bias, void * y, int64_t n,
                                int ci, int co, int silu, int cus, hipStream_t s);
// FlexiDualGrid mesh extraction (kernels_mesh.hip).
hipError_t launch_fdg_check(int dtype, const int32_t * coords, const void * feats, int64_t n, int channels, int res,
                            int32_t * flags, hipStream_t s);
hipError_t launch_fdg_vertices(int dtype, const int32_t * coords, const void * feats, int64_t n, int channels, int res,
                               float * vert, float * wgt, hipStream_t s);
hipError_t launch_fdg_count(int dtype, const void * feats, const int32_t * nbr, int64_t n, int channels,
                            int32_t * counts, hipStream_t s);
hipError_t launch_fdg_faces(int dtype, const void * feats, const int32_t * nbr, const float * wgt,
                            const int32_t * first, int64_t n, int channels, int32_t * faces, hipStream_t s);
hipError_t launch_c2s_count(int dtype, const void * logits, int64_t n, int32_t * counts, hipStream_t s);
// Exclusive scan of n int32 values; total written to *total_dev.  tmp needs scan_tmp_bytes(n).
size_t scan_tmp_bytes(int64_t n);
hipError_t launch_scan_exclusive(const int32_t * in, int32_t * out, int64_t n, int32_t * total_dev, void * tmp,
                                 hipStream_t s);
hipError_t launch_c2s_fill(int dtype, const int32_t * coords, const void * logits, const int32_t * offsets,
                           int64_t n, int32_t * out_coords, int32_t * parent, int32_t * subidx, hipStream_t s);
hipError_t launch_c2s_gather(int dtype, const void * x, const int32_t * parent, const int32_t * subidx, void * y,
                             int64_t n_out, int co, hipStream_t s);
hipError_t launch_skip_repeat(int dtype, const void * x, const int32_t * parent, const int32_t * subidx, void * y,
                              int64_t n_out, int ci, int co, hipStream_t s);

}  // namespace tsh
