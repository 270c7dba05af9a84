// Row kernels: rms, rms_back, softmax_ce (one row per LPR consecutive lanes, VPR values per lane), and transpoe
// (128 x 64 byte tiles through LDS). CHEIO: the row length is LPR * VPR. Otherwise it is Dr (a multiple of BLK
// below LPR * VPR, for the widths that are not powers of two): the lanes past Dr load and store nothing and join
// the row's reductions with neutral values (0 for sums, the smallest exponent for maxima).
#include "jt_comum.h"

// ---------------------------------------------------------------------------------------------- RMSNorm
// Y = quant(x * 2^k / r, e_b - k - emax + G/2), with ss = sum_b rnd(sum(m^2) << G, 2 (emax - e_b)),
// r = isqrt(ss >> log2 D), k = bitlen(r) + 10. Caches (r, emax) per row (ops.py:153-165).
template <int VPR, int LPR, int BLK, bool CHEIO = true>
__global__ void __launch_bounds__(256) k_rms(const int8_t* __restrict__ Xm, const int8_t* __restrict__ XE, int8_t* __restrict__ Ym,
                                             int8_t* __restrict__ YE, int* __restrict__ cr, int* __restrict__ cemax, int M, int log2D,
                                             int G, int kid, int Dr = 0) {
    constexpr int LPB = BLK / VPR;
    const int D = CHEIO ? VPR * LPR : Dr, nb = D / BLK;
    const int row = blockIdx.x * (256 / LPR) + threadIdx.x / LPR, lr = threadIdx.x % LPR;
    if (row >= M) return;
    const bool ativo = CHEIO || lr * VPR < D;
    const long long o = (long long)row * D + lr * VPR;
    int x[VPR];
    if (ativo) le_i8(Xm + o, x);
    else {
#pragma unroll
        for (int i = 0; i < VPR; i++) x[i] = 0;
    }
    const int b = lr / LPB, eb = ativo ? (int)XE[(long long)row * nb + b] : -128;
    const int emax = g_max<LPR>(eb);
    int sq = 0;
#pragma unroll
    for (int i = 0; i < VPR; i++) sq += x[i] * x[i];
    sq = g_sum<LPB>(sq);
    const bool lider = (lr & (LPB - 1)) == 0;
    const int ss = g_sum<LPR>(lider && ativo ? rnd(sq << G, 2 * (emax - eb), kid, (long long)row * D) : 0);
    if (ss >= LIM && lr == 0) reporta(E_ACUM, kid, (long long)row * D, ss, -1);
    // inv = 2^k / r lies in (2^10, 2^11]: the quotient bound of div_exata holds
    const int r = isqrt_i(ss >> log2D), k = bitlen(r) + 10, inv = div_exata(1 << k, r);
    int v[VPR], q[VPR];
#pragma unroll
    for (int i = 0; i < VPR; i++) v[i] = mul24(x[i], inv);      // |v| < 2^18, one exponent per block
    const int Eo = quant8_u<VPR, LPB>(v, eb - k - emax + G / 2, q, kid, o);
    if (!ativo) return;
    grava_q8(Ym + o, q);
    if (lider) YE[(long long)row * nb + b] = (int8_t)Eo;
    if (lr == 0) { cr[row] = r; cemax[row] = emax; }
}

// RMSNorm backward: dx = (g - y * mean(g y)) / rms in the spec's integer steps (ops.py:167-184). SOMA: the output
// is soma(x, dx) instead (ops.py:128-132, x given by xm, xE), as the backward's residual update uses it.
// The block-uniform alignments run through Desl: |g y| << GB < 2^21 shifts right, g shifts left by at most 21
// (ec >= eg + 7 - 28) and y S by at most 6 (|S| <= 2^15, ec >= ey + eS + 22 - 28), so every value stays below 2^28
// and the spec's left-shift checks cannot fire. Every load (x included) is issued before the first reduction.
// SOMA = 2: x is the 16-bit residual stream (int16 mantissas): om (int16), oE get z16 = soma16(x16, dx)
// (jatai_cuda.cu:514-531) and om2, oE2 its INT8 copy para8(z16) (jatai_cuda.cu:501-513), launch ids kid2, kid2 + 1.
template <int VPR, int LPR, int BLK, int SOMA = 0, bool CHEIO = true>
__global__ void __launch_bounds__(256) k_rms_back(const int8_t* __restrict__ gm, const int8_t* __restrict__ gE, const int8_t* __restrict__ ym,
                                                  const int8_t* __restrict__ yE, const int* __restrict__ cr, const int* __restrict__ cemax,
                                                  int8_t* __restrict__ om, int8_t* __restrict__ oE, int M, int log2D, int G, int GB, int kid,
                                                  const int8_t* __restrict__ xm = nullptr, const int8_t* __restrict__ xE = nullptr, int kid2 = 0,
                                                  int Dr = 0, int8_t* __restrict__ om2 = nullptr, int8_t* __restrict__ oE2 = nullptr) {
    constexpr int LPB = BLK / VPR;
    const int D = CHEIO ? VPR * LPR : Dr, nb = D / BLK;
    const int row = blockIdx.x * (256 / LPR) + threadIdx.x / LPR, lr = threadIdx.x % LPR;
    if (row >= M) return;
    const bool ativo = CHEIO || lr * VPR < D;
    const long long o = (long long)row * D + lr * VPR;
    const int b = lr / LPB;
    int g[VPR], y[VPR], a[VPR];
    int eg = -128, ey = -128, ex = 0;
    if (ativo) {
        le_i8(gm + o, g);
        le_i8(ym + o, y);
        eg = gE[(long long)row * nb + b];
        ey = yE[(long long)row * nb + b];
    } else {
#pragma unroll
        for (int i = 0; i < VPR; i++) g[i] = y[i] = 0;
    }
    const int r = cr[row], emax = cemax[row];
    if constexpr (SOMA != 0) {
        if (ativo) {
            if constexpr (SOMA == 2) le_i16(reinterpret_cast<const int16_t*>(xm) + o, a);
            else le_i8(xm + o, a);
            ex = xE[(long long)row * nb + b];
        } else {
#pragma unroll
            for (int i = 0; i < VPR; i++) a[i] = 0;
        }
    }
    const int smax = g_max<LPR>(eg + ey);
    const Desl d1(ativo ? smax - (eg + ey) : 0);
    int S = 0;
#pragma unroll
    for (int i = 0; i < VPR; i++) S += d1((g[i] * y[i]) << GB);
    S = g_sum<LPR>(S);
    if ((S >= LIM || S <= -LIM) && lr == 0) reporta(E_ACUM, kid, (long long)row * D, S, -2);
    int eS = smax - GB - log2D;
    const int sh = max(bitlen(S) - 15, 0);
    S = rnd_d(S, sh);
    eS += sh;
    const int k = bitlen(r) + 10, inv = div_exata(1 << k, r);          // 2^k / r in (2^10, 2^11]
    const int ec = max(eg + 7, ey + eS + 22) - 28;
    const Desl dg(ec - eg), dy(ec - (ey + eS));
    int v[VPR], ee[VPR];
#pragma unroll
    for (int i = 0; i < VPR; i++) {
        int dentro = dg(g[i]) - dy(mul24(y[i], S));                  // |S| <= 2^15
        const unsigned ad = (unsigned)(dentro < 0 ? -dentro : dentro);
        const int sh2 = max(32 - (int)__clz((int)ad) - 18, 0);     // bitlen(dentro) - 18
        dentro = desl_f(dentro, sh2);
        v[i] = mul24(dentro, inv);                                  // |dentro| < 2^18, inv <= 2^11
        ee[i] = ec + sh2 - k - (emax - G / 2);
    }
    int8_t q[VPR];
    const int Eo = quant8_d<VPR, LPB>(v, ee, q, kid, o);            // |ee| < 600
    if constexpr (SOMA == 2) {      // z16 = soma16(x16, dx): ec = max(xE + 15, E + 7) - 28; exponents as stored (int8)
        const int ey = (int)(int8_t)Eo, ec2 = max(ex + 15, ey + 7) - 28;
        const Desl da(ec2 - ex), dq(ec2 - ey);                       // left shifts keep |values| below 2^28
        const int ma = ex == E_ZERO ? 0 : -1, mq = ey == E_ZERO ? 0 : -1;
        int zs[VPR], qz[VPR];
#pragma unroll
        for (int i = 0; i < VPR; i++) zs[i] = (da(a[i]) & ma) + (dq((int)q[i]) & mq);
        const int Ez = quant_u<VPR, LPB, true, 15, 32767>(zs, ec2, qz, kid2, o);
        int8_t y8[VPR];
        const int Ey = quant8_u8<VPR, LPB>(qz, (int)(int8_t)Ez, y8, kid2 + 1, o);
        if (!ativo) return;
        int16_t z16[VPR];
#pragma unroll
        for (int i = 0; i < VPR; i++) z16[i] = (int16_t)qz[i];
        grava_i16(reinterpret_cast<int16_t*>(om) + o, z16);
        grava_i8(om2 + o, y8);
        if ((lr & (LPB - 1)) == 0) { oE[(long long)row * nb + b] = (int8_t)Ez; oE2[(long long)row * nb + b] = (int8_t)Ey; }
        return;
    }
    if constexpr (SOMA == 1) {                                       // z = soma(x, dx): ec = max(xE, E) - 21
        const int ec2 = max(ex, Eo) - 21;
        const Desl da(ec2 - ex), dq(ec2 - Eo);
        int zs[VPR], qz[VPR];
#pragma unroll
        for (int i = 0; i < VPR; i++) zs[i] = da(a[i]) + dq((int)q[i]);
        const int Ez = quant8_u<VPR, LPB>(zs, ec2, qz, kid2, o);
        if (!ativo) return;
        grava_q8(om + o, qz);
        if ((lr & (LPB - 1)) == 0) oE[(long long)row * nb + b] = (int8_t)Ez;
        return;
    }
    if (!ativo) return;
    grava_i8(om + o, q);
    if ((lr & (LPB - 1)) == 0) oE[(long long)row * nb + b] = (int8_t)Eo;
}

// ---------------------------------------------------------------------------------------------- softmax + CE
// raw logits -> g = (P - 1[target]) in block format with exponent -12 - log2 M; d_alvo = umax - u_target and
// soma = sum of ex per row, from which the host derives the float64 loss (ops.py:260-271; modelo.py:93).
template <int VPR, int LPR, int BLK, bool CHEIO = true>
__global__ void __launch_bounds__(256) k_softmax_ce(const int* __restrict__ acc, const int16_t* __restrict__ e, const int* __restrict__ alvo,
                                                    int8_t* __restrict__ gm, int8_t* __restrict__ gE, int* __restrict__ d_alvo,
                                                    int* __restrict__ soma_o, int M, int log2M, int kid, int Vr = 0) {
    constexpr int LPB = BLK / VPR;
    const int V = CHEIO ? VPR * LPR : Vr, nb = V / BLK;
    const int row = blockIdx.x * (256 / LPR) + threadIdx.x / LPR, lr = threadIdx.x % LPR;
    if (row >= M) return;
    const bool ativo = CHEIO || lr * VPR < V;
    const int t = alvo[row];
    if (t < 0 || t >= V) { if (lr == 0) reporta(E_ARG, kid, (long long)row * V, t, V); return; }
    const long long o = (long long)row * V + lr * VPR;
    int a[VPR], ea[VPR], u[VPR];
    if (ativo) {
        le_i32(acc + o, a);
        le_i16(e + o, ea);
    }
    int umax = U_MIN;
#pragma unroll
    for (int i = 0; i < VPR; i++) {
        u[i] = ativo ? rnd(a[i], -(ea[i] + 8), kid, o + i) : U_MIN;
        umax = max(umax, u[i]);
    }
    umax = g_max<LPR>(umax);
    int ex[VPR], s = 0;
#pragma unroll
    for (int i = 0; i < VPR; i++) { ex[i] = ativo ? exp_dif(umax, u[i]) >> 3 : 0; s += ex[i]; }
    s = g_sum<LPR>(s);
    if (s <= 0) { if (lr == 0) reporta(E_DIV, kid, (long long)row * V, s, umax); s = 1; }
    const int inv = s > 256 ? div_exata(1 << 28, s) : (1 << 28) / s;   // s >= 4095 (exp(0) >> 3 of the row maximum): 2^28 / s < 2^20
    int v[VPR];
#pragma unroll
    for (int i = 0; i < VPR; i++) {
        const int col = lr * VPR + i;
        v[i] = ((ex[i] * inv + (1 << 15)) >> 16) - (col == t ? 4096 : 0);
        if (col == t) d_alvo[row] = umax - u[i];
    }
    int8_t q[VPR];
    const int Eo = quant8_u8<VPR, LPB>(v, -12 - log2M, q, kid, o);   // one exponent per row
    if (!ativo) return;
    grava_i8(gm + o, q);
    if ((lr & (LPB - 1)) == 0) gE[(long long)row * nb + lr / LPB] = (int8_t)Eo;
    if (lr == 0) soma_o[row] = s;
}

// ---------------------------------------------------------------------------------------------- transpoe
// X [R, C] blocked along C -> Y [C, R] blocked along R: Y = quant(m^T, expand(E)^T) (ops.py:121-123).
// Tile TR rows x 64 cols (TR = 64 at BLK=32, 128 at BLK=128: a multiple of the output block), 2 TR threads.
// Lane (cg, rc) owns 4 columns (one 32-bit LDS word) x 8 rows: it reads 8 words, unpacks 32 values and runs 4
// block quantizations side by side; the LPB = BLK/8 lanes of a column block are consecutive lanes. Rows of the
// LDS tile are 18 words long and word w of row r sits at word w ^ (r / 8): the reads (a half-wave takes word cg
// of rows 8 rc + k, rc = 0 .. 15) then hit 32 distinct banks at TR = 128 (4 rows to a bank with 17-word rows and
// no swizzle); the row-pair writes stay 2-way.
// One tile's global loads (row tid / 2, half tid % 2: 32 bytes and the exponent byte of those 32 columns), kept in
// registers so a workgroup can issue the loads of several tiles before it stages the first.
struct CargaT {
    int4 v0, v1;
    int e;
};
template <int BLK, int TR>
__device__ __forceinline__ CargaT transpoe_carga(const int8_t* __restrict__ X, const int8_t* __restrict__ EX, int C, int bx, int by) {
    const int row = threadIdx.x >> 1, half = threadIdx.x & 1, r0 = by * TR, c0 = bx * 64;
    const int4* src = reinterpret_cast<const int4*>(X + (size_t)(r0 + row) * C + c0 + half * 32);
    return CargaT{src[0], src[1], (int)EX[(size_t)(r0 + row) * (C / BLK) + (c0 + half * 32) / BLK]};
}
constexpr int TLD = 18;                     // LDS row length of a transpose tile, in words
template <int BLK, int TR>
__device__ __forceinline__ void transpoe_tile(const CargaT& cg_, int (&tile)[TR][TLD], int8_t (&er)[TR][2], int8_t* __restrict__ Y,
                                              int8_t* __restrict__ EY, int R, int bx, int by, int kid) {
    constexpr int LPB = BLK / 8, RC = TR / 8;
    const int r0 = by * TR, c0 = bx * 64, tid = threadIdx.x;
    {
        const int row = tid >> 1, half = tid & 1, sw = (row >> 3) & 15;
        const int w8[8] = {cg_.v0.x, cg_.v0.y, cg_.v0.z, cg_.v0.w, cg_.v1.x, cg_.v1.y, cg_.v1.z, cg_.v1.w};
#pragma unroll
        for (int j = 0; j < 8; j++) tile[row][(8 * half + j) ^ sw] = w8[j];
        er[row][half] = (int8_t)cg_.e;
    }
    __syncthreads();
    const int cg = tid / RC, rc = tid % RC;                         // columns c0 + 4 cg .. +3, rows r0 + 8 rc .. +7
    int m[4][8], e[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int row = rc * 8 + k, word = tile[row][cg ^ (rc & 15)];     // (row / 8) % 16 = rc % 16
        e[k] = er[row][cg >> 3];
#pragma unroll
        for (int cc = 0; cc < 4; cc++) m[cc][k] = (word << (24 - 8 * cc)) >> 24;
    }
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
        const int col = c0 + 4 * cg + cc;
        const long long o = (long long)col * R + r0 + rc * 8;
        int8_t q[8];
        const int E = quant8_d<8, LPB, false>(m[cc], e, q, kid, o);    // int8 mantissas and exponents
        grava_i8(Y + o, q);
        if ((rc & (LPB - 1)) == 0) EY[(size_t)col * (R / BLK) + (r0 + rc * 8) / BLK] = (int8_t)E;
    }
}

template <int BLK, int TR>
__global__ void __launch_bounds__(2 * TR) k_transpoe(const int8_t* __restrict__ X, const int8_t* __restrict__ EX, int8_t* __restrict__ Y,
                                                     int8_t* __restrict__ EY, int R, int C, int kid) {
    __shared__ int tile[TR][TLD];
    __shared__ int8_t er[TR][2];
    transpoe_tile<BLK, TR>(transpoe_carga<BLK, TR>(X, EX, C, blockIdx.x, blockIdx.y), tile, er, Y, EY, R, blockIdx.x, blockIdx.y, kid);
}

// Many transposes in one launch. The tensor list travels by value in the kernel arguments (no device table, so
// a captured graph keeps it); tensor i owns the tiles [ini_i, ini_{i+1}) of the list, row-major over its
// (R / TR) x (C / 64) tiles, and workgroup w takes tiles TPW w .. TPW w + TPW - 1 (of any tensors): it issues
// every tile's loads first, then stages and writes them one by one, each in its own LDS buffer.
constexpr int LOTE_T = 64;
struct LoteT {
    const int8_t* X[LOTE_T];
    const int8_t* EX[LOTE_T];
    int8_t* Y[LOTE_T];
    int8_t* EY[LOTE_T];
    int R[LOTE_T], C[LOTE_T], ini[LOTE_T + 1];
    int n;
};

template <int BLK, int TR, int TPW>
__global__ void __launch_bounds__(2 * TR) k_transpoe_lote(const LoteT L, int kid) {
    __shared__ int tile[TPW][TR][TLD];
    __shared__ int8_t er[TPW][TR][2];
    int ti[TPW], bx[TPW], by[TPW];
    CargaT c[TPW];
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const int t = min(blockIdx.x * TPW + j, L.ini[L.n] - 1);   // past the list's end: a copy of the last tile, not stored
        // the last tensor whose first tile is at most t (a binary search: 6 dependent scalar loads instead of up to
        // 63 in a scan, which cost the step's three launches 140 -> 126 us at config 4); uniform, kernel arguments
        int i = 0;
        for (int s = 32; s; s >>= 1)
            if (i + s < L.n && L.ini[i + s] <= t) i += s;
        const int local = t - L.ini[i], ntx = L.C[i] / 64;
        ti[j] = i; bx[j] = local % ntx; by[j] = local / ntx;
        c[j] = transpoe_carga<BLK, TR>(L.X[i], L.EX[i], L.C[i], bx[j], by[j]);
    }
#pragma unroll
    for (int j = 0; j < TPW; j++)
        if (j == 0 || (int)blockIdx.x * TPW + j < L.ini[L.n])
            transpoe_tile<BLK, TR>(c[j], tile[j], er[j], L.Y[ti[j]], L.EY[ti[j]], L.R[ti[j]], bx[j], by[j], kid + ti[j]);
}

// The training loss from softmax_ce's per-row integers: mean over rows of d / 256 + ln(s / 4096) in float64
// (modelo.py:93). One workgroup; each term is the same float64 expression, summed in a fixed order (per thread,
// then across the wave, then the 16 wave sums in order).
__global__ void __launch_bounds__(1024) k_perda(const int* __restrict__ d, const int* __restrict__ s, double* __restrict__ out, int M) {
    __shared__ double ondas[16];
    double t = 0.0;
    for (int i = threadIdx.x; i < M; i += 1024) t += (double)d[i] / 256 + log((double)s[i] / 4096);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o);
    if ((threadIdx.x & 63) == 0) ondas[threadIdx.x >> 6] = t;
    __syncthreads();
    if (threadIdx.x == 0) {
        double u = 0.0;
#pragma unroll
        for (int w = 0; w < 16; w++) u += ondas[w];
        out[0] = u / M;
    }
}
