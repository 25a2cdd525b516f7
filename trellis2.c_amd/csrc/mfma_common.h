// mfma_common.h - device helpers shared by the MFMA kernels (conv, linear).
#pragma once
#include "tsh_internal.h"

namespace tsh {
namespace {

// Maps a linear block id onto a logical tile so that each of the 8 XCDs
// (which receive block ids round-robin) works on one contiguous range of
// tiles and its L2 sees neighbouring gathers.
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t grid) {
    constexpr int64_t kXcd = 8;
    const int64_t q = grid / kXcd, r = grid % kXcd;
    const int64_t xcd = bid % kXcd, slot = bid / kXcd;
    return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// Workgroup barrier that orders LDS only.  __syncthreads() also drains every
// outstanding global load (vmcnt(0)), which would empty the register prefetch
// ring of the streamed kernel at each barrier; its global loads only read
// data that no block writes.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt vmcnt(N) alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14;
// expcnt and lgkmcnt left at their maxima, i.e. not waited for).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Direct-to-LDS load of 16 bytes per lane: the bytes at voff + soff of the
// buffer land at LDS address lds + 16 * lane (exec-masked lanes load and
// write nothing).  Inline assembly, so that the compiler neither counts it
// nor waits for it before later LDS reads (it cannot tell LDS regions apart
// and would drain every such load at the next read); the caller waits with
// wait_vmcnt.  M0, which holds the LDS address, is saved and restored, with
// the wait state that a write of M0 needs before an LDS-DMA instruction.
__device__ __forceinline__ void dma_b128(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
    uint32_t keep;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(keep)
        : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
        : "memory");
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <int DT> struct Mfma;
template <> struct Mfma<kBF16> {
    typedef bf16x8 V;
    __device__ static f32x4 mac(V a, V b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};
template <> struct Mfma<kF16> {
    typedef f16x8 V;
    __device__ static f32x4 mac(V a, V b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};

// Lane layout of v_mfma_f32_16x16x32 (64 lanes): A fragment = row (lane%16),
// 8 consecutive K values starting at 8*(lane/16); B fragment = column
// (lane%16), the same 8 K values; D = rows 4*(lane/16)+i, column lane%16.
// Any consistent K permutation of A and B gives the same product, so only
// the row/column mapping matters for correctness.

// LDS layout of one 16-row block of A (64 granules of 16 bytes: 16 rows x 4
// chunks).  ds_read_b128 / ds_write_b128 serve 16 lanes per cycle from the 64
// banks without conflict when lanes 0-7 of each 16-lane group touch granules
// 0-7 (mod 16) and lanes 8-15 granules 8-15, each once.  Row i, chunk c sits at
//   16 * (i1 + 2 i2) + 8 i3 + 4 (c1 ^ i2) + 2 (c0 ^ i1) + i0     (bits of i, c),
// which meets that for the fragment reads (lane i + 16 c reads row i, chunk c)
// and, with quad j fetching row a_quad_row(j) (bits 1 and 3 of j exchanged),
// for the stores (lane 4 j + c stores row a_quad_row(j), chunk c).
__device__ __forceinline__ int a_granule(int i, int c) {
    const int i0 = i & 1, i1 = (i >> 1) & 1, i2 = (i >> 2) & 1, i3 = (i >> 3) & 1;
    return 16 * (i1 + 2 * i2) + 8 * i3 + 4 * (((c >> 1) & 1) ^ i2) + 2 * ((c & 1) ^ i1) + i0;
}
__device__ __forceinline__ int a_quad_row(int j) { return (j & 5) | (((j >> 1) & 1) << 3) | (((j >> 3) & 1) << 1); }

}  // namespace
}  // namespace tsh
