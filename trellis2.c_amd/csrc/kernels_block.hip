// kernels_block.hip - the ConvNeXt block's MLP in one kernel (bf16 / fp16).
//
// y = residual + W2 · SiLU(W0 · LN(x) + b0) + b2 per row, LN = row_norm with
// scale/shift and eps; the tail of the decoder's ConvNeXt block
// (src/architectures/sparse_unet_decoder/executor.c:206-241: row_norm ->
// linear_silu (C -> 4C) -> linear (4C -> C) -> add), whose 4C-wide
// intermediate otherwise makes a round trip through HBM (n * 4C * s written
// and read back).  Here it stays in LDS.  Values are rounded to the storage
// type where the slot sequence stores them: after the norm, after the SiLU,
// after the second linear and after the add.
//
// Persistent blocks of 8 wavefronts walk 64-row tiles.  At this width the
// SiLU (two transcendental instructions per hidden value) and the norm cost
// more vector-ALU time than the two GEMMs cost matrix-core time, so the work
// is arranged for the two to overlap:
//  B. GEMM 1 (64 x C times C x 4C): wavefront w owns hidden columns
//     [w * 4C/8, (w + 1) * 4C/8) for all 64 rows; its weight fragments stay in
//     registers for every tile.  Row block q's MFMAs run while the bias,
//     SiLU and rounding of row block q - 1 go through the vector ALU; the
//     hidden tile is written to LDS in the operand layout.
//  C. GEMM 2 (64 x 4C times 4C x C): 2 row groups x 4 channel groups; weight
//     fragments streamed from global memory through a 4-step register ring
//     that runs on across tiles.  Meanwhile the LayerNorm of the NEXT tile
//     (its rows loaded into registers during B) goes into the operand tile of
//     GEMM 1: C/8 lanes per row, shuffle reductions.  The GEMM 2 result, with
//     bias, is rounded into a storage-type staging tile.
//  D. residual (loaded during B) + staged value, rounded, 16-byte stores.
// Two block barriers per tile (after B and after C).  Operand tiles in LDS
// use the a_granule layout per (K step, 16-row block), conflict-free for the
// fragment reads.  fp32 accumulation throughout.
#include "tsh_internal.h"
#include "mfma_common.h"

namespace tsh {
namespace {

template <int DT, int C>
__global__ void __launch_bounds__(512) k_convnext_mlp(const typename Store<DT>::T * __restrict__ x,
                                                      const float * __restrict__ gamma,
                                                      const float * __restrict__ beta,
                                                      const typename Store<DT>::T * __restrict__ w0,
                                                      const float * __restrict__ b0,
                                                      const typename Store<DT>::T * __restrict__ w2,
                                                      const float * __restrict__ b2,
                                                      const typename Store<DT>::T * __restrict__ res,
                                                      typename Store<DT>::T * __restrict__ y, int64_t n, float eps,
                                                      int n_tiles) {
    using T = typename Store<DT>::T;
    using V = typename Mfma<DT>::V;
    constexpr int BM = 64;            // rows per tile
    constexpr int H = 4 * C;          // hidden width
    constexpr int KS1 = C / 32;       // K steps of GEMM 1
    constexpr int KS2 = H / 32;       // K steps of GEMM 2
    constexpr int WN1 = H / 8;        // hidden columns per wavefront (GEMM 1)
    constexpr int NT1 = WN1 / 16;
    constexpr int WN2 = C / 4;        // output columns per wavefront (GEMM 2: 4 channel groups)
    constexpr int NT2 = WN2 / 16;
    constexpr int LPR = C / 8;        // LayerNorm lanes per row (one 16-byte chunk each)
    constexpr int RPP = 64 / LPR;     // LayerNorm rows per wavefront pass
    constexpr int LNP = 8 / RPP;      // LayerNorm passes (8 rows per wavefront)
    constexpr int CH = C / 8;         // 16-byte chunks per row
    constexpr int DP = BM * CH / 512; // output chunks per thread
    constexpr int D2 = 4;             // GEMM 2 weight ring depth (steps)
    constexpr int OSTR = C + 8;       // staging row stride (storage elements)
    static_assert(C == 64 || C == 128, "C = 64 or 128");
    static_assert(KS2 % D2 == 0 && 8 % RPP == 0 && DP >= 1, "shapes");
    __shared__ __attribute__((aligned(16))) T s_x[KS1 * 4 * 64 * 8];
    __shared__ __attribute__((aligned(16))) T s_h[KS2 * 4 * 64 * 8];
    __shared__ __attribute__((aligned(16))) T s_o[BM * OSTR];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int l16 = lane & 15, lg = lane >> 4;
    const int G = (int) gridDim.x;
    const int lb = (int) xcd_remap(blockIdx.x, G);
    auto opnd = [](int kstep, int rb, int i, int c) { return ((kstep * 4 + rb) * 64 + a_granule(i, c)) * 8; };

    // GEMM 1 weight fragments of this wavefront, for every tile: packed
    // column wave*WN1 + nt*16 + l16 (holding hidden channel
    // wave*WN1 + l16*NT1 + nt) of K step s.
    V wf1[KS1][NT1];
#pragma unroll
    for (int s = 0; s < KS1; ++s)
#pragma unroll
        for (int nt = 0; nt < NT1; ++nt)
            wf1[s][nt] = *(const V *) (w0 + ((int64_t) (s * 4 + lg) * H + wave * WN1 + nt * 16 + l16) * 8);
    float bias1[NT1];
#pragma unroll
    for (int nt = 0; nt < NT1; ++nt) bias1[nt] = b0 != nullptr ? b0[wave * WN1 + l16 * NT1 + nt] : 0.0f;
    // GEMM 2: row group rh (row blocks rh, rh + 2), channel group ch.
    const int rh = wave & 1, ch = wave >> 1;
    float bias2[NT2];
#pragma unroll
    for (int nt = 0; nt < NT2; ++nt) bias2[nt] = b2 != nullptr ? b2[ch * WN2 + l16 * NT2 + nt] : 0.0f;
    // LayerNorm: lane handles chunk li of rows wave*8 + p*RPP + lane/LPR.
    const int li = lane % LPR;
    float gv[8], bv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        gv[e] = gamma != nullptr ? gamma[li * 8 + e] : 1.0f;
        bv[e] = beta != nullptr ? beta[li * 8 + e] : 0.0f;
    }
    const T * w2lane = w2 + ((int64_t) lg * C + ch * WN2 + l16) * 8;
    // wofs is 0, hidden from the compiler once per tile: the W2 loads are the
    // same for every tile, and hoisting them out of the tile loop would hold
    // all of W2's fragments in registers.
    int wofs = 0;
    auto load_w2 = [&](V * f, int s) {
#pragma unroll
        for (int nt = 0; nt < NT2; ++nt)
            f[nt] = *(const V *) (w2lane + wofs + (int64_t) s * 4 * C * 8 + nt * 16 * 8);
    };
    auto load_x = [&](int4 * xr, int tile) {
#pragma unroll
        for (int p = 0; p < LNP; ++p) {
            const int64_t row = (int64_t) tile * BM + wave * 8 + p * RPP + lane / LPR;
            xr[p] = row < n ? *(const int4 *) (x + row * C + li * 8) : int4{0, 0, 0, 0};
        }
    };
    // Normalised rows into s_x (rows past n normalise zeros; never stored).
    auto layer_norm = [&](const int4 * xr) {
#pragma unroll
        for (int p = 0; p < LNP; ++p) {
            const int rloc = wave * 8 + p * RPP + lane / LPR;
            float v[8];
            unpack_chunk<DT>(xr[p], v);
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) s += v[e];
#pragma unroll
            for (int d = LPR / 2; d >= 1; d >>= 1) s += __shfl_xor(s, d);
            const float mean = s / (float) C;
            float q = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[e] -= mean;
                q += v[e] * v[e];
            }
#pragma unroll
            for (int d = LPR / 2; d >= 1; d >>= 1) q += __shfl_xor(q, d);
            const float inv = 1.0f / sqrtf(q / (float) C + eps);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = v[e] * inv * gv[e] + bv[e];
            // Channels li*8 .. li*8+7 of row rloc: one operand granule.
            *(int4 *) (&s_x[opnd(li / 4, rloc / 16, rloc % 16, li % 4)]) = pack_chunk<DT>(v);
        }
    };
    // Bias, SiLU and rounding of GEMM 1 row block q: the lane's hidden
    // channels h0 .. h0 + NT1 - 1 (adjacent) of rows q*16 + lg*4 + i are NT1
    // elements of one operand granule of s_h.
    const int h0 = wave * WN1 + l16 * NT1;
    auto silu_store = [&](const f32x4 * a, int q) {
        using Hv = T __attribute__((ext_vector_type(NT1)));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            Hv o;
#pragma unroll
            for (int nt = 0; nt < NT1; ++nt) {
                float v = a[nt][i] + bias1[nt];
                v = v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
                o[nt] = round_to_store<DT>(v);
            }
            *(Hv *) (&s_h[opnd(h0 / 32, q, lg * 4 + i, (h0 % 32) / 8) + h0 % 8]) = o;
        }
    };

    // GEMM 2 weight ring: wr[r] holds K step s0 + r; the last steps of a tile
    // fetch the first steps of the next.
    V wr[D2][NT2];
#pragma unroll
    for (int s = 0; s < D2; ++s) load_w2(wr[s], s);
    {
        int4 xr[LNP];
        load_x(xr, lb);
        layer_norm(xr);
    }
    lds_barrier();

    for (int tile = lb; tile < n_tiles; tile += G) {
        const int64_t row0 = (int64_t) tile * BM;
        asm volatile("" : "+s"(wofs));
        // Loads for later phases: the next tile's rows (LayerNorm during C;
        // zeros past the last tile) and this tile's residual (D).
        int4 xr[LNP];
        load_x(xr, tile + G);
        int4 rr[DP];
#pragma unroll
        for (int p = 0; p < DP; ++p) {
            const int e = t + p * 512;
            const int64_t row = row0 + e / CH;
            rr[p] = row < n ? *(const int4 *) (res + row * C + (e % CH) * 8) : int4{0, 0, 0, 0};
        }
        // ---- B. GEMM 1 by row block; SiLU of the previous block meanwhile --
        {
            f32x4 acc[2][NT1];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
                for (int nt = 0; nt < NT1; ++nt) acc[q & 1][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < KS1; ++s) {
                    const V af = *(const V *) (&s_x[opnd(s, q, l16, lg)]);
#pragma unroll
                    for (int nt = 0; nt < NT1; ++nt) acc[q & 1][nt] = Mfma<DT>::mac(af, wf1[s][nt], acc[q & 1][nt]);
                }
                if (q > 0) silu_store(acc[(q - 1) & 1], q - 1);
            }
            silu_store(acc[1], 3);
        }
        lds_barrier();
        // ---- C. GEMM 2; the next tile's LayerNorm meanwhile -----------------
        {
            f32x4 acc[2][NT2];
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int nt = 0; nt < NT2; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s0 = 0; s0 < KS2; s0 += D2) {
#pragma unroll
                for (int r = 0; r < D2; ++r) {
                    const int s = s0 + r;
                    V af[2];
#pragma unroll
                    for (int q = 0; q < 2; ++q) af[q] = *(const V *) (&s_h[opnd(s, rh + 2 * q, l16, lg)]);
#pragma unroll
                    for (int q = 0; q < 2; ++q)
#pragma unroll
                        for (int nt = 0; nt < NT2; ++nt) acc[q][nt] = Mfma<DT>::mac(af[q], wr[r][nt], acc[q][nt]);
                    const int sn = s + D2 < KS2 ? s + D2 : s + D2 - KS2;
                    load_w2(wr[r], sn);
                }
                // s_x was last read by GEMM 1, before the barrier above.
                if (s0 == 0) layer_norm(xr);
            }
            const int c0 = ch * WN2 + l16 * NT2;
            using Ov = T __attribute__((ext_vector_type(NT2)));
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = (rh + 2 * q) * 16 + lg * 4 + i;
                    Ov o;
#pragma unroll
                    for (int nt = 0; nt < NT2; ++nt) o[nt] = round_to_store<DT>(acc[q][nt][i] + bias2[nt]);
                    *(Ov *) (&s_o[r * OSTR + c0]) = o;
                }
        }
        lds_barrier();
        // ---- D. residual add, 16-byte stores -------------------------------
        // s_o is rewritten only after the next tile's first barrier.
#pragma unroll
        for (int p = 0; p < DP; ++p) {
            const int e = t + p * 512;
            const int r = e / CH, j = e % CH;
            const int64_t row = row0 + r;
            if (row >= n) continue;
            float a[8], b[8];
            unpack_chunk<DT>(rr[p], a);
            unpack_chunk<DT>(*(const int4 *) (&s_o[r * OSTR + j * 8]), b);
#pragma unroll
            for (int k = 0; k < 8; ++k) a[k] += b[k];
            *(int4 *) (y + row * C + j * 8) = pack_chunk<DT>(a);
        }
    }
}

template <int DT, int C>
hipError_t launch_mlp_t(const void * x, const float * gamma, const float * beta, const void * w0, const float * b0,
                        const void * w2, const float * b2, const void * res, void * y, int64_t n, float eps, int cus,
                        hipStream_t s) {
    using T = typename Store<DT>::T;
    const int64_t tiles = (n + 63) / 64;
    if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
    const int64_t grid = tiles < cus ? tiles : cus;
    k_convnext_mlp<DT, C><<<(unsigned) grid, 512, 0, s>>>((const T *) x, gamma, beta, (const T *) w0, b0,
                                                         (const T *) w2, b2, (const T *) res, (T *) y, n, eps,
                                                         (int) tiles);
    return hipGetLastError();
}
}  // namespace

bool convnext_mlp_supported(int dtype, int c) { return (dtype == kF16 || dtype == kBF16) && (c == 64 || c == 128); }

void convnext_mlp_groups(int c, int * g0, int * g2) {
    *g0 = 4 * c / 8 / 16;  // hidden columns per GEMM 1 wavefront / 16
    *g2 = c / 4 / 16;      // output columns per GEMM 2 wavefront / 16
}

hipError_t launch_convnext_mlp(int dtype, const void * x, const float * gamma, const float * beta, const void * w0,
                               const float * b0, const void * w2, const float * b2, const void * res, void * y,
                               int64_t n, int c, float eps, int cus, hipStream_t s) {
    if (!convnext_mlp_supported(dtype, c) || n <= 0 || cus <= 0) return hipErrorInvalidValue;
    if (dtype == kBF16) {
        return c == 128 ? launch_mlp_t<kBF16, 128>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s)
                        : launch_mlp_t<kBF16, 64>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s);
    }
    return c == 128 ? launch_mlp_t<kF16, 128>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s)
                    : launch_mlp_t<kF16, 64>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s);
}

}  // namespace tsh
