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

// ---------------------------------------------------------------------------
// The same tail for C = 256 (H = 1024).  W0 and W2 (512 KB each in bf16) no
// longer fit in registers, and a 64-row tile would stream 16 KB of weights
// per row, so the hidden layer is taken in chunks of 128 units instead:
// persistent blocks of 8 wavefronts walk 128-row tiles, and per chunk
//   GEMM 1  (128 x 256 times 256 x 128; 2 row groups x 4 column groups, the
//           normalised rows and the chunk's W0 columns read from LDS) ->
//           bias, SiLU, rounding -> the chunk's hidden tile in LDS;
//   GEMM 2  (128 x 128 times 128 x 256; 8 column groups of 32 outputs over
//           all 128 rows) accumulates into the tile's fp32 outputs, which
//           stay in registers across the 8 chunks.
// The chunk's 64 KB of W0 are fetched once per block straight into LDS
// (direct-to-LDS loads) while the previous chunk's GEMM 2 runs: fetched per
// wavefront into registers, each W0 fragment went through the vector-memory
// path twice (once per row group) and GEMM 1 waited on that path (0.534 ms
// at 316k rows).  W2 fragments stream through a per-wavefront register ring
// 2 steps deep that runs on across chunks and tiles, each fetched once per
// tile and block.  Two barriers per chunk.  The hidden values never leave
// the CU; GEMM 2's sum over the 1024 hidden units runs in K order, chunk
// after chunk, as the linear slot's does.  Roundings as above.
// ---------------------------------------------------------------------------
template <int DT, int C>
__global__ void __launch_bounds__(512, 1) k_convnext_mlp_wide(const typename Store<DT>::T * __restrict__ x,
                                                              const float * __restrict__ gamma,
                                                              const float * __restrict__ beta,
                                                              const typename Store<DT>::T * __restrict__ w0,
                                                              const float * __restrict__ b0,
                                                              const typename Store<DT>::T * __restrict__ w2,
                                                              const float * __restrict__ b2,
                                                              const typename Store<DT>::T * __restrict__ res,
                                                              typename Store<DT>::T * __restrict__ y, int64_t n,
                                                              float eps, int n_tiles) {
    using T = typename Store<DT>::T;
    using V = typename Mfma<DT>::V;
    static_assert(C == 256, "C = 256");
    constexpr int BM = 128;             // rows per tile
    constexpr int NRB = BM / 16;        // row blocks per tile
    constexpr int H = 4 * C;            // hidden width
    constexpr int HC = 128;             // hidden units per chunk
    constexpr int NCH = H / HC;         // chunks
    constexpr int KS1 = C / 32;         // K steps of GEMM 1
    constexpr int KS2 = HC / 32;        // K steps of GEMM 2 per chunk
    constexpr int NT1 = 2;              // GEMM 1 column tiles per wavefront (32 hidden units)
    constexpr int NT2 = 2;              // GEMM 2 column tiles per wavefront (32 outputs)
    constexpr int D2 = 2;               // W2 ring depth (steps)
    constexpr int LPR = C / 8;          // LayerNorm lanes per row
    constexpr int RPP = 64 / LPR;       // LayerNorm rows per wavefront pass
    constexpr int LNP = (BM / 8) / RPP; // LayerNorm passes (BM / 8 rows per wavefront)
    constexpr int CH = C / 8;           // 16-byte chunks per row
    constexpr int DP = BM * CH / 512;   // output chunks per thread
    constexpr int OSTR = C + 8;         // staging row stride (storage elements)
    static_assert(KS2 % D2 == 0 && (BM / 8) % RPP == 0, "shapes");
    // LDS: the normalised rows (GEMM 1's A operand), the chunk's hidden tile
    // (GEMM 2's A operand), the chunk's W0 fragments (GEMM 1's B operand:
    // fragment (K step s, column group cg, column tile nt) as 64 lanes x 16
    // bytes at ((s * 4 + cg) * NT1 + nt) KB); the output staging tile reuses
    // the first two.
    constexpr int XE = KS1 * NRB * 64 * 8, HE = KS2 * NRB * 64 * 8, WE = KS1 * 4 * NT1 * 64 * 8;
    static_assert((XE + HE) >= BM * OSTR, "staging fits");
    __shared__ __attribute__((aligned(16))) T s_lds[XE + HE + WE];
    T * s_x = s_lds;
    T * s_h = s_lds + XE;
    T * s_o = s_lds;
    const T * s_w0 = s_lds + XE + HE;
    const uint32_t w0_lds = (uint32_t) (uintptr_t) (s_lds + XE + HE);

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int l16 = lane & 15, lg = lane >> 4;
    const int G = (int) gridDim.x;
    const int lb = (int) xcd_remap(blockIdx.x, G);
    auto opnd = [](int kstep, int rb, int i, int c) { return ((kstep * NRB + rb) * 64 + a_granule(i, c)) * 8; };

    // GEMM 1: row group rg (row blocks 4 rg .. 4 rg + 3), column group cg
    // (hidden units cg*32 .. cg*32+31 of each chunk; packed column
    // cg*32 + nt*16 + l16 holds unit cg*32 + 2 l16 + nt).
    const int rg = wave & 1, cg = wave >> 1;
    // GEMM 2: column group wave (outputs wave*32 .. +31, packed the same way).
    float bias2[NT2];
#pragma unroll
    for (int nt = 0; nt < NT2; ++nt) bias2[nt] = b2 != nullptr ? b2[wave * 32 + l16 * NT2 + nt] : 0.0f;
    const int li = lane % LPR;
    // Weight rings.  Step g1 of GEMM 1 (chunk g1 / KS1, K step g1 % KS1) and
    // step g2 of GEMM 2 (chunk g2 / KS2, K step g2 % KS2), both modulo a
    // tile's steps: the last steps of a tile fetch the first of the next.
    // wofs is 0, hidden from the compiler once per tile, so that it keeps
    // the loads in the rings instead of hoisting them out of the tile loop.
    int wofs = 0;
    const T * w2lane = w2 + ((int64_t) lg * C + wave * 32 + l16) * 8;
    // Chunk j's W0 fragments into s_w0: this wavefront's 8 of the 64 (K step
    // s = wave, both column tiles of the 4 column groups); lane l16 + 16 lg
    // of fragment (s, cg, nt) holds packed column j*HC + cg*32 + nt*16 + l16,
    // K values 8 (4 s + lg) .. + 7.
    const __amdgpu_buffer_rsrc_t w0res =
        __builtin_amdgcn_make_buffer_rsrc((void *) w0, 0, C * H * (int) sizeof(T), 0x00020000);
    static_assert(KS1 == 8, "one K step of W0 per wavefront");
    auto load_w0 = [&](int j) {
#pragma unroll
        for (int f = 0; f < 4 * NT1; ++f) {
            const int fcg = f / NT1, fnt = f % NT1;
            const uint32_t voff =
                (uint32_t) (((wave * 4 + lg) * H + j * HC + fcg * 32 + fnt * 16 + l16) * 16);
            dma_b128(w0res, w0_lds + (uint32_t) (((wave * 4 + fcg) * NT1 + fnt) * 1024), voff, 0u);
        }
    };
    auto load_w2 = [&](V * f, int g2) {
        const int j = g2 / KS2, s = g2 % KS2;
#pragma unroll
        for (int nt = 0; nt < NT2; ++nt)
            f[nt] = *(const V *) (w2lane + wofs + ((int64_t) (j * HC / 8 + s * 4) * C + nt * 16) * 8);
    };
    V wr2[D2][NT2];
#pragma unroll
    for (int r = 0; r < D2; ++r) load_w2(wr2[r], r);
    load_w0(0);
    wait_vmcnt<0>();
    lds_barrier();

    for (int tile = lb; tile < n_tiles; tile += G) {
        const int64_t row0 = (int64_t) tile * BM;
        asm volatile("" : "+s"(wofs));
        // ---- LayerNorm of the tile's rows into s_x (rows past n: zeros) ----
        {
            // Scale and shift per tile (wofs keeps them out of the registers
            // that the tile loop holds).
            float gv[8], bv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                gv[e] = gamma != nullptr ? gamma[wofs + li * 8 + e] : 1.0f;
                bv[e] = beta != nullptr ? beta[wofs + li * 8 + e] : 0.0f;
            }
            int4 xr[LNP];
#pragma unroll
            for (int p = 0; p < LNP; ++p) {
                const int64_t row = row0 + wave * (BM / 8) + p * RPP + lane / LPR;
                xr[p] = row < n ? *(const int4 *) (x + row * C + li * 8) : int4{0, 0, 0, 0};
            }
            // Mean, then the centred variance, each reduced over the row's
            // LPR lanes level by level for all LNP rows of the lane at once
            // (one shuffle round trip per level instead of one per row).
            float mean[LNP], inv[LNP];
#pragma unroll
            for (int p = 0; p < LNP; ++p) {
                float v[8];
                unpack_chunk<DT>(xr[p], v);
                float sm = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) sm += v[e];
                mean[p] = sm;
            }
#pragma unroll
            for (int d = LPR / 2; d >= 1; d >>= 1)
#pragma unroll
                for (int p = 0; p < LNP; ++p) mean[p] += __shfl_xor(mean[p], d);
#pragma unroll
            for (int p = 0; p < LNP; ++p) {
                mean[p] /= (float) C;
                float v[8];
                unpack_chunk<DT>(xr[p], v);
                float q = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float dv = v[e] - mean[p];
                    q += dv * dv;
                }
                inv[p] = q;
            }
#pragma unroll
            for (int d = LPR / 2; d >= 1; d >>= 1)
#pragma unroll
                for (int p = 0; p < LNP; ++p) inv[p] += __shfl_xor(inv[p], d);
#pragma unroll
            for (int p = 0; p < LNP; ++p) {
                const int rloc = wave * (BM / 8) + p * RPP + lane / LPR;
                const float iv = 1.0f / sqrtf(inv[p] / (float) C + eps);
                float v[8];
                unpack_chunk<DT>(xr[p], v);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = (v[e] - mean[p]) * iv * gv[e] + bv[e];
                *(int4 *) (&s_x[opnd(li / 4, rloc / 16, rloc % 16, li % 4)]) = pack_chunk<DT>(v);
            }
        }
        lds_barrier();
        f32x4 acc2[NRB][NT2];
#pragma unroll
        for (int q = 0; q < NRB; ++q)
#pragma unroll
            for (int nt = 0; nt < NT2; ++nt) acc2[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
        for (int j = 0; j < NCH; ++j) {
            // ---- GEMM 1 of chunk j; bias, SiLU and rounding into s_h ----------
            {
                f32x4 acc1[4][NT1];
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int nt = 0; nt < NT1; ++nt) acc1[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < KS1; ++s) {
                    V af[4], bw[NT1];
#pragma unroll
                    for (int q = 0; q < 4; ++q) af[q] = *(const V *) (&s_x[opnd(s, rg * 4 + q, l16, lg)]);
#pragma unroll
                    for (int nt = 0; nt < NT1; ++nt)
                        bw[nt] = *(const V *) (&s_w0[(((s * 4 + cg) * NT1 + nt) * 64 + lane) * 8]);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int nt = 0; nt < NT1; ++nt) acc1[q][nt] = Mfma<DT>::mac(af[q], bw[nt], acc1[q][nt]);
                }
                float bias1[NT1];
#pragma unroll
                for (int nt = 0; nt < NT1; ++nt)
                    bias1[nt] = b0 != nullptr ? b0[j * HC + cg * 32 + l16 * NT1 + nt] : 0.0f;
                using Hv = T __attribute__((ext_vector_type(NT1)));
                const int kc = cg * 32 + l16 * NT1;  // first hidden unit (in the chunk) of this lane
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        Hv o;
#pragma unroll
                        for (int nt = 0; nt < NT1; ++nt) {
                            float v = acc1[q][nt][i] + bias1[nt];
                            v = v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
                            o[nt] = round_to_store<DT>(v);
                        }
                        *(Hv *) (&s_h[opnd(kc / 32, rg * 4 + q, lg * 4 + i, (kc % 32) / 8) + kc % 8]) = o;
                    }
            }
            lds_barrier();
            // Every wavefront is done with chunk j's W0: the next chunk's (or,
            // after the last, the next tile's first) go in during GEMM 2.
            load_w0(j + 1 < NCH ? j + 1 : 0);
            // ---- GEMM 2 of chunk j into the tile's outputs --------------------
#pragma unroll
            for (int s = 0; s < KS2; ++s) {
                const int r = s % D2;
                V af[NRB];
#pragma unroll
                for (int q = 0; q < NRB; ++q) af[q] = *(const V *) (&s_h[opnd(s, q, l16, lg)]);
#pragma unroll
                for (int q = 0; q < NRB; ++q)
#pragma unroll
                    for (int nt = 0; nt < NT2; ++nt) acc2[q][nt] = Mfma<DT>::mac(af[q], wr2[r][nt], acc2[q][nt]);
                const int g2 = (j * KS2 + s + D2) % (NCH * KS2);
                load_w2(wr2[r], g2);
            }
            // The W0 loads, issued before GEMM 2's KS2 * NT2 ring loads, have
            // landed (vmcnt retires in order).  s_h (and, after the last
            // chunk, s_x) is rewritten only after this barrier.
            wait_vmcnt<KS2 * NT2>();
            lds_barrier();
        }
        // ---- bias, rounding, staging; residual add, 16-byte stores ---------
        {
            using Ov = T __attribute__((ext_vector_type(NT2)));
            const int c0 = wave * 32 + l16 * NT2;
#pragma unroll
            for (int q = 0; q < NRB; ++q)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = q * 16 + lg * 4 + i;
                    Ov o;
#pragma unroll
                    for (int nt = 0; nt < NT2; ++nt) o[nt] = round_to_store<DT>(acc2[q][nt][i] + bias2[nt]);
                    *(Ov *) (&s_o[r * OSTR + c0]) = o;
                }
        }
        lds_barrier();
#pragma unroll
        for (int p = 0; p < DP; ++p) {
            const int e = t + p * 512;
            const int r = e / CH, jc = e % CH;
            const int64_t row = row0 + r;
            if (row >= n) continue;
            float a[8], b[8];
            unpack_chunk<DT>(*(const int4 *) (res + row * C + jc * 8), a);
            unpack_chunk<DT>(*(const int4 *) (&s_o[r * OSTR + jc * 8]), b);
#pragma unroll
            for (int k = 0; k < 8; ++k) a[k] += b[k];
            *(int4 *) (y + row * C + jc * 8) = pack_chunk<DT>(a);
        }
        // The next tile's LayerNorm overwrites the staging tile.
        lds_barrier();
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

bool convnext_mlp_supported(int dtype, int c) {
    return (dtype == kF16 || dtype == kBF16) && (c == 64 || c == 128 || c == 256);
}

void convnext_mlp_groups(int c, int * g0, int * g2) {
    if (c >= 256) {  // k_convnext_mlp_wide: 32 hidden units and 32 outputs per wavefront
        *g0 = 2;
        *g2 = 2;
        return;
    }
    *g0 = 4 * c / 8 / 16;  // hidden columns per GEMM 1 wavefront / 16
    *g2 = c / 4 / 16;      // output columns per GEMM 2 wavefront / 16
}

namespace {
template <int DT>
hipError_t launch_mlp_wide_t(const void * x, const float * gamma, const float * beta, const void * w0,
                             const float * b0, const void * w2, const float * b2, const void * res, void * y,
                             int64_t n, float eps, int cus, hipStream_t s) {
    using T = typename Store<DT>::T;
    const int64_t tiles = (n + 127) / 128;
    if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
    const int64_t grid = tiles < cus ? tiles : cus;
    k_convnext_mlp_wide<DT, 256><<<(unsigned) grid, 512, 0, s>>>((const T *) x, gamma, beta, (const T *) w0, b0,
                                                                (const T *) w2, b2, (const T *) res, (T *) y, n, eps,
                                                                (int) tiles);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_convnext_mlp(int dtype, const void * x, const float * gamma, const float * beta, const void * w0,
                               const float * b0, const void * w2, const float * b2, const void * res, void * y,
                               int64_t n, int c, float eps, int cus, hipStream_t s) {
    if (!convnext_mlp_supported(dtype, c) || n <= 0 || cus <= 0) return hipErrorInvalidValue;
    if (c == 256) {
        return dtype == kBF16 ? launch_mlp_wide_t<kBF16>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s)
                              : launch_mlp_wide_t<kF16>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s);
    }
    if (dtype == kBF16) {
        return c == 128 ? launch_mlp_t<kBF16, 128>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s)
                        : launch_mlp_t<kBF16, 64>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s);
    }
    return c == 128 ? launch_mlp_t<kF16, 128>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s)
                    : launch_mlp_t<kF16, 64>(x, gamma, beta, w0, b0, w2, b2, res, y, n, eps, cus, s);
}

}  // namespace tsh
