// Block-exponent INT8 GEMM on CDNA4 i8 MFMA: C = A . B^T, A [M, K] and B [N, K] blocked along K.
//
// Arithmetic (ops.py:95-108): RA_i = max_b ea_ib, RB_j = max_b eb_jb; for every K-block b the exact product
// p_ijb = sum_{k in b} a_ik b_jk (one MFMA per 32 values of K), then acc_ij += rnd(p_ijb << 4, sa + sb) with
// sa = RA_i - ea_ib, sb = RB_j - eb_jb, round half to even; base_ij = RA_i + RB_j - 4.
//
// The rounding runs in fp32, where it is exact: |p| < 2^21, so p, p * 2^(4 - s) (a power-of-two scale) and
// its nearest-even integer (v_rndne_f32) are all representable, and for s >= 31 the scaled value is below 1/2
// and rounds to 0 exactly as rnd(., s >= 31) does. Per output and K-block this is add3 (the shift), cvt,
// ldexp, rndne, cvt, add: six VALU ops, against ~9 for the integer form. This per-block VALU epilogue, not
// the MFMA, bounds the kernel.
//
// Tiling: a workgroup of 4 waves owns a 32 x 128 output tile (one 128-column block at BLK=128, four at
// BLK=32); each wave a 32 x 32 sub-tile of 2 x 2 MFMA 16x16 tiles, with A/B fragments read straight from
// global memory (each lane 8 contiguous bytes of one row) and exponents staged once in LDS. After the K loop
// the accumulators go through LDS into a row-block layout (16 consecutive columns per lane) where the block
// quantization and the fused epilogues run:
//   MODO 0 block output | 1 raw output (split-K over gridDim.z with atomics into a zeroed buffer)
//   2 + residual add (soma) | 3 + ReLU^2 second output | 4 ReLU^2 backward with H
// The fused epilogues compute exactly the separate ops on the quantized GEMM output (jatai_cuda.cu:195-200).
#include "jt_comum.h"

typedef int v4i __attribute__((ext_vector_type(4)));

namespace gemm {
constexpr int BM = 32, BN = 128, NT = 256, PAD = 4;
}

template <int BLK, int MODO>
__global__ void __launch_bounds__(256) k_gemm(const int8_t* __restrict__ A, const int8_t* __restrict__ EA, const int8_t* __restrict__ B,
                                              const int8_t* __restrict__ EB, int8_t* __restrict__ Cm, int8_t* __restrict__ CE,
                                              int* __restrict__ C32, int16_t* __restrict__ Ce, const int8_t* __restrict__ Xm,
                                              const int8_t* __restrict__ XE, int8_t* __restrict__ Om2, int8_t* __restrict__ OE2, int M,
                                              int N, int K, int kpart, int kid) {
    using namespace gemm;
    extern __shared__ __align__(16) char smem[];
    const int nb = K / BLK;
    // LDS: ea as int32 [nb][BM], eb as int8 [nb][BN], RA [BM], RB [BN]; the accumulator tile reuses the front.
    int* ea_s = reinterpret_cast<int*>(smem);
    int8_t* eb_s = reinterpret_cast<int8_t*>(smem + (size_t)nb * BM * 4);
    int* ra_s = reinterpret_cast<int*>(smem + (size_t)nb * BM * 4 + (size_t)nb * BN);
    int* rb_s = ra_s + BM;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    for (int i = tid; i < BM * nb; i += NT) { const int r = i / nb, b = i % nb; ea_s[b * BM + r] = EA[(size_t)(row0 + r) * nb + b]; }
    for (int i = tid; i < BN * nb; i += NT) { const int r = i / nb, b = i % nb; eb_s[b * BN + r] = EB[(size_t)(col0 + r) * nb + b]; }
    __syncthreads();
    if (tid < BM) { int m = -128; for (int b = 0; b < nb; b++) m = max(m, ea_s[b * BM + tid]); ra_s[tid] = m; }
    else if (tid >= 64 && tid < 64 + BN) { const int c = tid - 64; int m = -128; for (int b = 0; b < nb; b++) m = max(m, (int)eb_s[b * BN + c]); rb_s[c] = m; }
    __syncthreads();

    // lane coordinates inside the wave's 32 x 32 sub-tile
    const int lr = lane & 15, lg = lane >> 4;                       // fragment row/col, k-group
    const int wc = wave * 32;                                       // wave's first column in the WG tile
    int k0[2][2][4];                                                // 4 - RA_i - RB_j per output
#pragma unroll
    for (int ti = 0; ti < 2; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++)
#pragma unroll
            for (int i = 0; i < 4; i++) k0[ti][tj][i] = 4 - ra_s[16 * ti + 4 * lg + i] - rb_s[wc + 16 * tj + lr];
    int acc[2][2][4] = {};
    const int8_t* pa0 = A + (size_t)(row0 + lr) * K + 8 * lg;
    const int8_t* pa1 = pa0 + (size_t)16 * K;
    const int8_t* pb0 = B + (size_t)(col0 + wc + lr) * K + 8 * lg;
    const int8_t* pb1 = pb0 + (size_t)16 * K;
    const int b_ini = blockIdx.z * kpart, b_fim = min(nb, b_ini + kpart);
    constexpr int KS = BLK / 32;                                    // MFMA k-steps per block
    long fa[2][KS], fb[2][KS];
    auto carrega = [&](int b) {
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const size_t off = (size_t)b * BLK + 32 * s;
            fa[0][s] = *reinterpret_cast<const long*>(pa0 + off);
            fa[1][s] = *reinterpret_cast<const long*>(pa1 + off);
            fb[0][s] = *reinterpret_cast<const long*>(pb0 + off);
            fb[1][s] = *reinterpret_cast<const long*>(pb1 + off);
        }
    };
    if (b_ini < b_fim) carrega(b_ini);
    for (int b = b_ini; b < b_fim; b++) {
        v4i p[2][2];
#pragma unroll
        for (int ti = 0; ti < 2; ti++)
#pragma unroll
            for (int tj = 0; tj < 2; tj++) {
                p[ti][tj] = v4i{0, 0, 0, 0};
#pragma unroll
                for (int s = 0; s < KS; s++) p[ti][tj] = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa[ti][s], fb[tj][s], p[ti][tj], 0, 0, 0);
            }
        if (b + 1 < b_fim) carrega(b + 1);                          // next block's fragments in flight
        const v4i ea0 = *reinterpret_cast<const v4i*>(ea_s + b * BM + 4 * lg);
        const v4i ea1 = *reinterpret_cast<const v4i*>(ea_s + b * BM + 16 + 4 * lg);
        const int eb0 = eb_s[b * BN + wc + lr], eb1 = eb_s[b * BN + wc + 16 + lr];
#pragma unroll
        for (int ti = 0; ti < 2; ti++)
#pragma unroll
            for (int tj = 0; tj < 2; tj++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int n = k0[ti][tj][i] + (ti ? ea1[i] : ea0[i]) + (tj ? eb1 : eb0);     // 4 - sa - sb
                    acc[ti][tj][i] += (int)rintf(ldexpf((float)p[ti][tj][i], n));
                }
    }

    // ---- output stage: accumulators to LDS, then 16 consecutive columns of one row per lane
    __syncthreads();
    int* acc_s = reinterpret_cast<int*>(smem);                     // [BM][BN + PAD]
    // RA/RB must survive: copy them to registers first
    const int orow = tid >> 3, oc = (tid & 7) * 16;
    const int ra = ra_s[orow];
    int base[16];
#pragma unroll
    for (int j = 0; j < 16; j++) base[j] = ra + rb_s[oc + j] - 4;
    __syncthreads();
#pragma unroll
    for (int ti = 0; ti < 2; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc_s[(16 * ti + 4 * lg + i) * (BN + PAD) + wc + 16 * tj + lr] = acc[ti][tj][i];
    __syncthreads();
    int v[16];
#pragma unroll
    for (int j = 0; j < 16; j += 4) {
        const v4i t = *reinterpret_cast<const v4i*>(acc_s + orow * (BN + PAD) + oc + j);
        v[j] = t[0]; v[j + 1] = t[1]; v[j + 2] = t[2]; v[j + 3] = t[3];
    }
    const int r = row0 + orow, c = col0 + oc;
    const size_t o = (size_t)r * N + c;
    if constexpr (MODO == 1) {
        if (gridDim.z > 1) {
#pragma unroll
            for (int j = 0; j < 16; j++) atomicAdd(C32 + o + j, v[j]);
        } else {
#pragma unroll
            for (int j = 0; j < 16; j += 4) *reinterpret_cast<int4*>(C32 + o + j) = make_int4(v[j], v[j + 1], v[j + 2], v[j + 3]);
        }
        if (blockIdx.z == 0) {
            int16_t eo[16];
#pragma unroll
            for (int j = 0; j < 16; j++) eo[j] = (int16_t)max(-30000, base[j]);
            grava_i16(Ce + o, eo);
        }
    } else {
        constexpr int LPB = BLK / 16;
        const bool lider = (tid & (LPB - 1)) == 0;
        const size_t oe = (size_t)r * (N / BLK) + c / BLK;
        int8_t m[16];
        const int E = quant8<16, LPB>(v, base, m, kid, o);
        if constexpr (MODO == 0 || MODO == 3) {
            grava_i8(Cm + o, m);
            if (lider) CE[oe] = (int8_t)E;
        }
        if constexpr (MODO == 3) {                                 // a = relu2(h): max(m, 0)^2, exponent 2E
            int a[16];
#pragma unroll
            for (int j = 0; j < 16; j++) { const int h = max((int)m[j], 0); a[j] = h * h; }
            int8_t q[16];
            const int Ea = quant8_comum<16, LPB>(a, 2 * E, q);
            if (Ea > 126 && lider) reporta(E_EXP, kid, (long long)o, Ea, -7);
            grava_i8(Om2 + o, q);
            if (lider) OE2[oe] = (int8_t)Ea;
        }
        if constexpr (MODO == 2) {                                 // z = soma(X, C): ec = max(xE, E) - 21
            int x[16], s[16];
            le_i8(Xm + o, x);
            const int ex = XE[oe], ec = max(ex, E) - 21;
#pragma unroll
            for (int j = 0; j < 16; j++) s[j] = desloca(x[j], ec - ex) + desloca((int)m[j], ec - E);
            int8_t q[16];
            const int Ez = quant8_comum<16, LPB>(s, ec, q);
            if (Ez > 126 && lider) reporta(E_EXP, kid, (long long)o, Ez, -6);
            grava_i8(Cm + o, q);
            if (lider) CE[oe] = (int8_t)Ez;
        }
        if constexpr (MODO == 4) {                                 // gh = C * 2 max(H, 0), exponent E + eh
            int h[16], s[16];
            le_i8(Xm + o, h);
            const int eh = XE[oe];
#pragma unroll
            for (int j = 0; j < 16; j++) s[j] = (int)m[j] * max(h[j], 0) * 2;
            int8_t q[16];
            const int Eg = quant8_comum<16, LPB>(s, E + eh, q);
            if (Eg > 126 && lider) reporta(E_EXP, kid, (long long)o, Eg, -8);
            grava_i8(Cm + o, q);
            if (lider) CE[oe] = (int8_t)Eg;
        }
    }
}

// dynamic LDS bytes for a K of nb blocks (the accumulator tile needs BM * (BN + PAD) * 4)
static inline size_t gemm_lds(int nb) {
    using namespace gemm;
    const size_t ex = (size_t)nb * BM * 4 + (size_t)nb * BN + (BM + BN) * 4;
    const size_t ac = (size_t)BM * (BN + PAD) * 4;
    return ex > ac ? ex : ac;
}
