// Element-wise and per-block kernels: quant, soma, relu2, relu2_back, momento, peso, para16, para8, soma16,
// embed, um_quente, and the int32 fill used before split-K accumulation.
//
// Layout: 256 threads per workgroup, 8 consecutive values per lane, so a block of BLK values is LPB = BLK/8
// consecutive lanes (4 at BLK=32, 16 at BLK=128) and one workgroup covers 2048 values. Each lane moves 8 B
// (int8), 16 B (int16) or 32 B (int32) per operand with vector loads: these kernels stream HBM.
#include "jt_comum.h"

#define VPL 8
#define ELEM_PROLOGO                                                   \
    constexpr int LPB = BLK / VPL;                                     \
    const long long o = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * VPL; \
    const long long w = o / BLK;                                       \
    if (w >= nblocos) return;

// raw (acc int32, e int16) -> block (ops.py:125-126)
template <int BLK>
__global__ void __launch_bounds__(256) k_quant(const int* __restrict__ acc, const int16_t* __restrict__ e, int8_t* __restrict__ m,
                                               int8_t* __restrict__ E, long long nblocos, int kid) {
    ELEM_PROLOGO
    int v[VPL], ee[VPL];
    le_i32(acc + o, v);
    le_i16(e + o, ee);
    int8_t q[VPL];
    const int Eo = quant8_f<VPL, LPB>(v, ee, q, kid, o);
    grava_i8(m + o, q);
    if ((threadIdx.x & (LPB - 1)) == 0) E[w] = (int8_t)Eo;
}

// The ops below give every value of a block one exponent (their inputs are block tensors), so they quantize with
// quant8_u and 16 values per lane (16-byte vectors; a block is LPU = BLK/16 lanes): a few VALU operations per
// value instead of the generic quant8's per-value exponent work. One 16-value chunk per lane measured fastest on
// MI355X: several chunks per lane, with all loads issued first or with the next chunk's loads issued before the
// current chunk is computed, cost more in occupancy than they gained.
#define VPU 16
#define ELEM_PROLOGO_U                                                 \
    constexpr int LPU = BLK / VPU;                                     \
    const long long o = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * VPU; \
    const long long w = o / BLK;                                       \
    if (w >= nblocos) return;

// z = x + y: ec = max(xE, yE) - 21 (ops.py:128-132). Both alignments are exact left shifts or roundings with
// |x| <= 2^28, so no shift check is needed.
template <int BLK>
__global__ void __launch_bounds__(256) k_soma(const int8_t* __restrict__ xm, const int8_t* __restrict__ xE, const int8_t* __restrict__ ym,
                                              const int8_t* __restrict__ yE, int8_t* __restrict__ zm, int8_t* __restrict__ zE,
                                              long long nblocos, int kid) {
    ELEM_PROLOGO_U
    int a[VPU], b[VPU], v[VPU], q[VPU];
    le_i8(xm + o, a);
    le_i8(ym + o, b);
    const int ex = xE[w], ey = yE[w], ec = max(ex, ey) - 21;
    const Desl da(ec - ex), db(ec - ey);
#pragma unroll
    for (int i = 0; i < VPU; i++) v[i] = da(a[i]) + db(b[i]);
    const int Eo = quant8_u<VPU, LPU>(v, ec, q, kid, o);
    grava_q8(zm + o, q);
    if ((threadIdx.x & (LPU - 1)) == 0) zE[w] = (int8_t)Eo;
}

// a = max(h, 0)^2 with exponent 2E (ops.py:134-137)
template <int BLK>
__global__ void __launch_bounds__(256) k_relu2(const int8_t* __restrict__ hm, const int8_t* __restrict__ hE, int8_t* __restrict__ am,
                                               int8_t* __restrict__ aE, long long nblocos, int kid) {
    ELEM_PROLOGO_U
    int h[VPU], v[VPU], q[VPU];
    le_i8(hm + o, h);
#pragma unroll
    for (int i = 0; i < VPU; i++) { const int r = max(h[i], 0); v[i] = r * r; }
    const int Eo = quant8_u<VPU, LPU>(v, 2 * hE[w], q, kid, o);
    grava_q8(am + o, q);
    if ((threadIdx.x & (LPU - 1)) == 0) aE[w] = (int8_t)Eo;
}

// gh = g * 2 max(h, 0) with exponent gE + hE (ops.py:139-141)
template <int BLK>
__global__ void __launch_bounds__(256) k_relu2_back(const int8_t* __restrict__ gm, const int8_t* __restrict__ gE, const int8_t* __restrict__ hm,
                                                    const int8_t* __restrict__ hE, int8_t* __restrict__ om, int8_t* __restrict__ oE,
                                                    long long nblocos, int kid) {
    ELEM_PROLOGO_U
    int g[VPU], h[VPU], v[VPU], q[VPU];
    le_i8(gm + o, g);
    le_i8(hm + o, h);
#pragma unroll
    for (int i = 0; i < VPU; i++) v[i] = g[i] * max(h[i], 0) * 2;
    const int Eo = quant8_u<VPU, LPU>(v, gE[w] + hE[w], q, kid, o);
    grava_q8(om + o, q);
    if ((threadIdx.x & (LPU - 1)) == 0) oE[w] = (int8_t)Eo;
}

// momentum, in place: m <- 7/8 m + g with g raw (ops.py:273-278)
template <int BLK>
__global__ void __launch_bounds__(256) k_momento(const int* __restrict__ gacc, const int16_t* __restrict__ ge, int8_t* __restrict__ Mm,
                                                 int8_t* __restrict__ ME, long long nblocos, int kid) {
    ELEM_PROLOGO
    int mm[VPL], g[VPL], eg[VPL], v[VPL], ee[VPL];
    le_i8(Mm + o, mm);
    le_i32(gacc + o, g);
    le_i16(ge + o, eg);
    const int em = ME[w] - 3;
    unsigned gmax = 0;
#pragma unroll
    for (int i = 0; i < VPL; i++) {                // shifts keep |x| < 2^28 (see otim_valores): no check can fire
        const unsigned a = (unsigned)(g[i] < 0 ? -g[i] : g[i]);
        gmax = max(gmax, a);
        const int ec = max(em + 10, eg[i] + 32 - (int)__clz((int)a)) - 28;
        v[i] = desl_f(mm[i] * 7, ec - em) + desl_f(g[i], ec - eg[i]);
        ee[i] = ec;
    }
    if (gmax >= (unsigned)LIM) {
#pragma unroll
        for (int i = 0; i < VPL; i++)
            if (g[i] >= LIM || g[i] <= -LIM) reporta(E_ACUM, kid, o + i, g[i], eg[i]);
    }
    int8_t q[VPL];
    const int Eo = quant8_f<VPL, LPB>(v, ee, q, kid, o);
    grava_i8(Mm + o, q);
    if ((threadIdx.x & (LPB - 1)) == 0) ME[w] = (int8_t)Eo;
}

// weight update, in place: W <- W - 2^-k m (+ error-feedback residual R) (ops.py:280-290). ec is at least
// (largest exponent + 7) - 27, so each alignment shifts left by at most 20 (|x| < 2^27) or rounds.
template <int BLK>
__global__ void __launch_bounds__(256) k_peso(int8_t* __restrict__ Wm, int8_t* __restrict__ WE, const int8_t* __restrict__ Mm,
                                              const int8_t* __restrict__ ME, int8_t* __restrict__ Rm, int8_t* __restrict__ RE, int k_lr,
                                              int ef, long long nblocos, int kid) {
    ELEM_PROLOGO_U
    int wv[VPU], mv[VPU], rv[VPU], alvo[VPU], q[VPU];
    le_i8(Wm + o, wv);
    le_i8(Mm + o, mv);
    if (ef) le_i8(Rm + o, rv);
    else
#pragma unroll
        for (int i = 0; i < VPU; i++) rv[i] = 0;
    const int ew = WE[w], em = ME[w] - k_lr, er = ef ? (int)RE[w] : E_ZERO;
    const int ec = max(max(ew + 7, em + 7), er + 7) - 27;
    const Desl dw(ec - ew), dm(ec - em), dr(ec - er);
#pragma unroll
    for (int i = 0; i < VPU; i++) alvo[i] = dw(wv[i]) - dm(mv[i]) + dr(rv[i]);
    const int Ew = quant8_u<VPU, LPU>(alvo, ec, q, kid, o);
    grava_q8(Wm + o, q);
    const bool lider = (threadIdx.x & (LPU - 1)) == 0;
    if (lider) WE[w] = (int8_t)Ew;
    if (!ef) return;
    // the residual: what the new weight lost, alvo - q 2^(Ew - ec) (a zero mantissa contributes 0)
    const Desl dq(ec - Ew);
    int dif[VPU], r[VPU];
#pragma unroll
    for (int i = 0; i < VPU; i++) dif[i] = alvo[i] - dq(q[i]);
    const int Er = quant8_u<VPU, LPU>(dif, ec, r, kid, o);
    grava_q8(Rm + o, r);
    if (lider) RE[w] = (int8_t)Er;
}

// ---------------------------------------------------------------------------------------------- R16 residual stream
// INT8 -> R16, exact: m << 7, E - 7; zero blocks keep E = -127 (jatai_cuda.cu:491-500)
template <int BLK>
__global__ void __launch_bounds__(256) k_para16(const int8_t* __restrict__ xm, const int8_t* __restrict__ xE, int16_t* __restrict__ zm,
                                                int8_t* __restrict__ zE, long long nblocos, int kid) {
    ELEM_PROLOGO
    int a[VPL];
    le_i8(xm + o, a);
    int16_t z[VPL];
#pragma unroll
    for (int i = 0; i < VPL; i++) z[i] = (int16_t)(a[i] << 7);
    grava_i16(zm + o, z);
    if ((threadIdx.x & (LPB - 1)) == 0) zE[w] = xE[w] == E_ZERO ? (int8_t)E_ZERO : (int8_t)(xE[w] - 7);
}

// R16 -> INT8 with the INT8 quant rules (jatai_cuda.cu:501-513)
template <int BLK>
__global__ void __launch_bounds__(256) k_para8(const int16_t* __restrict__ xm, const int8_t* __restrict__ xE, int8_t* __restrict__ ym,
                                               int8_t* __restrict__ yE, long long nblocos, int kid) {
    ELEM_PROLOGO
    int v[VPL];
    le_i16(xm + o, v);
    const int ex = xE[w];
    int8_t q[VPL];
    const int Eo = quant8_u8<VPL, LPB>(v, ex, q, kid, o);            // one exponent per block
    grava_i8(ym + o, q);
    if ((threadIdx.x & (LPB - 1)) == 0) yE[w] = (int8_t)Eo;
}

// z (R16) = x (R16) + y (INT8): ec = max(ex + 15, ey + 7) - 28; zero blocks contribute 0 (jatai_cuda.cu:514-531)
template <int BLK>
__global__ void __launch_bounds__(256) k_soma16(const int16_t* __restrict__ xm, const int8_t* __restrict__ xE, const int8_t* __restrict__ ym,
                                                const int8_t* __restrict__ yE, int16_t* __restrict__ zm, int8_t* __restrict__ zE,
                                                long long nblocos, int kid) {
    ELEM_PROLOGO
    int a[VPL], b[VPL], v[VPL], q[VPL];
    le_i16(xm + o, a);
    le_i8(ym + o, b);
    const int ex = xE[w], ey = yE[w], ec = max(ex + 15, ey + 7) - 28;
    // ec - ex >= -13 and ec - ey >= -21: the left shifts keep |a|, |b| below 2^28, so the spec's checks cannot
    // fire; one exponent per block, so the alignments are block-uniform roundings and the quantization is quant_u's
    const Desl da(ec - ex), db(ec - ey);
    const int ma = ex == E_ZERO ? 0 : -1, mb = ey == E_ZERO ? 0 : -1;
#pragma unroll
    for (int i = 0; i < VPL; i++) v[i] = (da(a[i]) & ma) + (db(b[i]) & mb);
    const int Eo = quant_u<VPL, LPB, true, 15, 32767>(v, ec, q, kid, o);
    int16_t q16[VPL];
#pragma unroll
    for (int i = 0; i < VPL; i++) q16[i] = (int16_t)q[i];
    grava_i16(zm + o, q16);
    if ((threadIdx.x & (LPB - 1)) == 0) zE[w] = (int8_t)Eo;
}

// ---------------------------------------------------------------------------------------------- embedding
// X[t] = W[tok[t]] (ops.py:143-145). One lane per 16 bytes of a row; a token outside the vocabulary is
// reported (E_ARG, index = start of output row t) and its row is written as a zero block row.
template <int BLK>
__global__ void __launch_bounds__(256) k_embed(const int8_t* __restrict__ Wm, const int8_t* __restrict__ WE, const int* __restrict__ tok,
                                               int8_t* __restrict__ Xm, int8_t* __restrict__ XE, int M, int D, int V, int kid) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;      // 16-byte chunk index
    const int chunks = D / 16;
    if (i >= (long long)M * chunks) return;
    const int t = (int)(i / chunks), c = (int)(i % chunks);
    const int v = tok[t];
    const bool ok = v >= 0 && v < V;
    if (!ok && c == 0) reporta(E_ARG, kid, (long long)t * D, v, V);
    const int4 z = ok ? *reinterpret_cast<const int4*>(Wm + (size_t)v * D + c * 16) : make_int4(0, 0, 0, 0);
    *reinterpret_cast<int4*>(Xm + (size_t)t * D + c * 16) = z;
    const int nb = D / BLK;
    // exponent bytes: chunk c covers bytes [16c, 16c + 16) of the row; its blocks start there
    for (int b = c * 16 / BLK; b < nb && b * BLK < (c + 1) * 16; b++)
        if (b * BLK >= c * 16) XE[(size_t)t * nb + b] = ok ? WE[(size_t)v * nb + b] : (int8_t)E_ZERO;
}

// Training windows of a byte corpus resident in device memory (treino_int8_gpu/treino.py:41-44): sequence b is the
// T + 1 bytes from ini[b]; tok gets its first T and alvo its last T, as int32 token ids (the kernels' token type),
// so the step's inputs are written in place with no host copy and no int64 -> int32 conversion. A start outside
// [0, n - T - 1] is reported (E_ARG, index = b * T, value = the start, aux = n - T - 1) and its rows written as 0.
__global__ void __launch_bounds__(256) k_janelas(const uint8_t* __restrict__ corpus, long long n, const long long* __restrict__ ini,
                                                 int* __restrict__ tok, int* __restrict__ alvo, int Bt, int T, int kid) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)Bt * T) return;
    const int b = (int)(i / T), t = (int)(i - (long long)b * T);
    const long long s = ini[b], ult = n - T - 1;
    const bool ok = s >= 0 && s <= ult;
    if (!ok && t == 0) reporta(E_ARG, kid, (long long)b * T, s, ult);
    tok[i] = ok ? (int)corpus[s + t] : 0;
    alvo[i] = ok ? (int)corpus[s + t + 1] : 0;
}

// one-hot rows: U[t, tok[t]] = 1, exponent 0 (not -127) for every block (ops.py:147-151)
template <int BLK>
__global__ void __launch_bounds__(256) k_um_quente(const int* __restrict__ tok, int8_t* __restrict__ U, int8_t* __restrict__ UE, int M,
                                                   int V, int kid) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int chunks = V / 16;
    if (i >= (long long)M * chunks) return;
    const int t = (int)(i / chunks), c = (int)(i % chunks);
    const int v = tok[t];
    const bool ok = v >= 0 && v < V;
    if (!ok && c == 0) reporta(E_ARG, kid, (long long)t * V, v, V);
    int8_t q[16];
#pragma unroll
    for (int j = 0; j < 16; j++) q[j] = (ok && c * 16 + j == v) ? 1 : 0;
    grava_i8(U + (size_t)t * V + c * 16, q);
    const int nb = V / BLK;
    for (int b = c * 16 / BLK; b < nb && b * BLK < (c + 1) * 16; b++)
        if (b * BLK >= c * 16) UE[(size_t)t * nb + b] = 0;
}

// int32 fill (split-K accumulators are zeroed with a kernel, so graph replays need no memset node)
__global__ void __launch_bounds__(256) k_zera32(int* __restrict__ p, long long n) {
    const long long i = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i + 4 <= n) *reinterpret_cast<int4*>(p + i) = make_int4(0, 0, 0, 0);
    else
        for (long long j = i; j < n; j++) p[j] = 0;
}

// ---------------------------------------------------------------------------------------------- fused optimizer
// momento then peso for many tensors in one launch. Per block: Mom <- quant(rnd(7 m, ec - em) + rnd(g, ec - ge), ec)
// (ops.py:273-278), then W, R <- peso(W, Mom, R, k, ef) (ops.py:280-290) on the new Mom held in registers: the
// same arithmetic as k_momento followed by k_peso, with Mom read once and the second launch gone.
// The tensor list is a device table of TabOtim entries (fixed addresses: parameters, momenta, residuals and the
// persistent raw-gradient buffers of the model); entry t covers global blocks [inicio_t, inicio_t + nblocos_t).
// compacto = 1: ge holds the gradient's exponents as the vectors ge[i] = RA_i (i < M), ge[M + j] = RB_j - 4 of the
// grouped GEMM's compact output (the exponent of (i, j) is their sum); else one int16 per value. M, N: the tensor's
// shape. Tm, TE (k_otimizador_t only, may be null): the transpose of the new weight, transpoe(W) [N, M] blocked
// along M (ops.py:121-123).
struct TabOtim {
    const int* gacc;
    const int16_t* ge;
    int8_t *Mm, *ME, *Wm, *WE, *Rm, *RE, *Tm, *TE;
    long long inicio, nblocos;
    int M, N, compacto, pad;
};

// momento then peso for NV consecutive values of one block, the block held by NL consecutive lanes: g raw with
// exponents eg; o = offset of the first value in the tensor, w = its block, lider = the block's first lane. Used by
// k_otimizador and by the weight-gradient GEMM's epilogue (NV = 16 in both).
struct Otim {
    int8_t *Mm, *ME, *Wm, *WE, *Rm, *RE;
};
// the optimizer's inputs of NV values: loaded before any store (the three tensors are distinct, but the compiler
// cannot know it and would otherwise order each load after the previous tensor's store)
template <int NV>
struct OtimEnt {
    unsigned mm[NV / 4], wv[NV / 4], rv[NV / 4];                   // int8 values, 4 per register
    int me, we, re;
    __device__ int m(int i) const { return (int)(int8_t)(mm[i >> 2] >> (8 * (i & 3))); }
    __device__ int w(int i) const { return (int)(int8_t)(wv[i >> 2] >> (8 * (i & 3))); }
    __device__ int r(int i) const { return (int)(int8_t)(rv[i >> 2] >> (8 * (i & 3))); }
};
template <int NV>
__device__ __forceinline__ void le_pk(const int8_t* p, unsigned (&d)[NV / 4]) {
#pragma unroll
    for (int k = 0; k < NV / 4; k += 2) {
        const uint2 t = *reinterpret_cast<const uint2*>(p + 4 * k);
        d[k] = t.x;
        d[k + 1] = t.y;
    }
}
template <int NV>
__device__ __forceinline__ OtimEnt<NV> otim_le(const Otim& d, long long o, long long w, int ef) {
    OtimEnt<NV> x;
    le_pk<NV>(d.Mm + o, x.mm);
    le_pk<NV>(d.Wm + o, x.wv);
    if (ef) le_pk<NV>(d.Rm + o, x.rv);
    else
#pragma unroll
        for (int i = 0; i < NV / 4; i++) x.rv[i] = 0;
    x.me = d.ME[w];
    x.we = d.WE[w];
    x.re = ef ? (int)d.RE[w] : E_ZERO;
    return x;
}
// Every shift below keeps |x| < 2^28 (the momentum terms by ec >= bitlen - 28 per value, the weight terms by
// ec >= largest exponent + 7 - 27), so none of the spec's left-shift checks can fire and the shifts run without
// branches (desl_f per value, Desl per block); a gradient value out of range is still reported.
// qw, Ew: the new weight's mantissas and block exponent, for a caller that also writes its transpose
template <int NV, int NL>
__device__ __forceinline__ void otim_valores(const int (&g)[NV], const int (&eg)[NV], const OtimEnt<NV>& x, const Otim& d, long long o, long long w,
                                             bool lider, int k_lr, int ef, int kid, int (&qw)[NV], int& Ew) {
    int v[NV], ee[NV];
    const int em = x.me - 3;
    unsigned gmax = 0;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const unsigned a = (unsigned)(g[i] < 0 ? -g[i] : g[i]);
        gmax = max(gmax, a);
        const int ec = max(em + 10, eg[i] + 32 - (int)__clz((int)a)) - 28;          // eg + bitlen(g)
        v[i] = desl_f(x.m(i) * 7, ec - em) + desl_f(g[i], ec - eg[i]);
        ee[i] = ec;
    }
    if (gmax >= (unsigned)LIM) {
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (g[i] >= LIM || g[i] <= -LIM) reporta(E_ACUM, kid, o + i, g[i], eg[i]);
    }
    int8_t q[NV];
    const int Em = quant8_f<NV, NL>(v, ee, q, kid, o);
    grava_i8(d.Mm + o, q);
    if (lider) d.ME[w] = (int8_t)Em;
    // peso with the new momentum: one exponent per block from here on
    const int ew = x.we, emk = Em - k_lr, er = x.re;
    const int ec = max(max(ew + 7, emk + 7), er + 7) - 27;
    const Desl dw(ec - ew), dm(ec - emk), dr(ec - er);
    int alvo[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) alvo[i] = dw(x.w(i)) - dm(q[i]) + dr(x.r(i));
    Ew = quant8_u<NV, NL>(alvo, ec, qw, kid, o);
    grava_q8(d.Wm + o, qw);
    if (lider) d.WE[w] = (int8_t)Ew;
    if (!ef) return;
    // the residual: what the new weight lost, alvo - qw 2^(Ew - ec) (a zero mantissa contributes 0)
    const Desl dq(ec - Ew);
    int dif[NV], r[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) dif[i] = alvo[i] - dq(qw[i]);
    const int Er = quant8_u<NV, NL>(dif, ec, r, kid, o);
    grava_q8(d.Rm + o, r);
    if (lider) d.RE[w] = (int8_t)Er;
}

// 16 values per lane; each workgroup finds the table entry of each lane's block by a binary search over the
// entries' first blocks staged in LDS (the table is at most 256 entries)
template <int BLK>
__global__ void __launch_bounds__(256) k_otimizador(const TabOtim* __restrict__ tab, int ntab, long long nblocos, int k_lr, int ef, int kid) {
    constexpr int NVO = 16, LPB = BLK / NVO;
    __shared__ long long ini[256];
    for (int i = threadIdx.x; i < ntab; i += blockDim.x) ini[i] = tab[i].inicio;
    __syncthreads();
    const long long og = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * NVO;
    const long long wg = og / BLK;
    if (wg >= nblocos) return;
    int t = 0;                                                      // table entry holding global block wg (entries sorted)
    for (int s = 128; s; s >>= 1)
        if (t + s < ntab && ini[t + s] <= wg) t += s;
    const TabOtim d = tab[t];
    const long long w = wg - d.inicio, o = w * BLK + (og % BLK);
    const Otim ot{d.Mm, d.ME, d.Wm, d.WE, d.Rm, d.RE};
    const OtimEnt<NVO> x = otim_le<NVO>(ot, o, w, ef);
    int g[NVO], eg[NVO];
    le_i32(d.gacc + o, g);
    if (d.compacto) {                                               // 16 values of one row (N % 16 == 0)
        const int row = (int)(o / d.N), col = (int)(o - (long long)row * d.N);
        const int er = d.ge[row];
        le_i16(d.ge + d.M + col, eg);
#pragma unroll
        for (int j = 0; j < NVO; j++) eg[j] = max(-30000, er + eg[j]);
    } else {
        le_i16(d.ge + o, eg);
    }
    int qw[NVO], Ew;
    otim_valores<NVO, LPB>(g, eg, x, ot, o, w, (threadIdx.x & (LPB - 1)) == 0, k_lr, ef, kid, qw, Ew);
}

// The same update with each workgroup on one 32 x 128 tile of a tensor (BLK = 32; every tensor with M % 32 == 0 and
// N % 128 == 0; its blocks counted from inicio as in k_otimizador, so tile t of the launch is global blocks
// 128 t .. 128 t + 127), which also writes the transpose of the new weight when the entry's Tm is set: the tile's
// 128 columns are 128 blocks of 32 rows of transpoe(W), re-quantized from the new mantissas and block exponents
// staged in LDS (quant of the transposed values with their exponents, ops.py:121-123). The weights' transposes the
// next step's backward reads are then written here instead of by a separate launch.
// LDS: mantissa rows of 128 bytes whose 16-byte chunk j sits at chunk j ^ (row / 16), and exponent rows 5 bytes
// apart, so the column reads (two threads per column, rows 16 p .. 16 p + 15) fall in distinct banks.
__global__ void __launch_bounds__(256) k_otimizador_t(const TabOtim* __restrict__ tab, int ntab, int k_lr, int ef, int kid) {
    constexpr int NVO = 16, LPB = 2, BN = 128, ES = 5;
    __shared__ long long ini[256];
    __shared__ __align__(16) int8_t qs[32 * BN];
    __shared__ int8_t es[32 * ES];
    for (int i = threadIdx.x; i < ntab; i += blockDim.x) ini[i] = tab[i].inicio;
    __syncthreads();
    const long long b0 = (long long)blockIdx.x * 128;               // the tile's first global block (uniform)
    int t = 0;
    for (int s = 128; s; s >>= 1)
        if (t + s < ntab && ini[t + s] <= b0) t += s;
    const TabOtim d = tab[t];
    const int tid = threadIdx.x, ntc = d.N / BN;
    const long long tl = (b0 - d.inicio) / 128;                     // tile index in the tensor, row-major over tiles
    const int row0 = (int)(tl / ntc) * 32, col0 = (int)(tl % ntc) * BN;
    const int orow = tid >> 3, oc = 16 * (tid & 7);
    const long long o = (long long)(row0 + orow) * d.N + col0 + oc, w = o / 32;
    const Otim ot{d.Mm, d.ME, d.Wm, d.WE, d.Rm, d.RE};
    const OtimEnt<NVO> x = otim_le<NVO>(ot, o, w, ef);
    int g[NVO], eg[NVO];
    le_i32(d.gacc + o, g);
    if (d.compacto) {
        const int er = d.ge[row0 + orow];
        le_i16(d.ge + d.M + col0 + oc, eg);
#pragma unroll
        for (int j = 0; j < NVO; j++) eg[j] = max(-30000, er + eg[j]);
    } else {
        le_i16(d.ge + o, eg);
    }
    int qw[NVO], Ew;
    otim_valores<NVO, LPB>(g, eg, x, ot, o, w, (tid & (LPB - 1)) == 0, k_lr, ef, kid, qw, Ew);
    if (d.Tm == nullptr) return;                                     // uniform: one tensor per workgroup
    int8_t q8[NVO];
#pragma unroll
    for (int i = 0; i < NVO; i++) q8[i] = (int8_t)qw[i];
    grava_i8<NVO, false>(qs + orow * BN + 16 * ((oc >> 4) ^ ((orow >> 4) & 7)), q8);
    if ((tid & (LPB - 1)) == 0) es[orow * ES + oc / 32] = (int8_t)Ew;
    __syncthreads();
    const int c = tid >> 1, pt = tid & 1;                            // column c, rows 16 pt .. 16 pt + 15
    const int8_t* qc = qs + 16 * ((c >> 4) ^ pt) + (c & 15);
    int tv[16], te[16];
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int r = 16 * pt + k;
        tv[k] = qc[r * BN];
        te[k] = es[r * ES + (c >> 5)];
    }
    int8_t t8[16];
    const long long ot2 = (long long)(col0 + c) * d.M + row0 + 16 * pt;
    const int Et = quant8_d<16, 2>(tv, te, t8, kid, ot2);
    grava_i8(d.Tm + ot2, t8);
    if (pt == 0) d.TE[(size_t)(col0 + c) * (d.M / 32) + row0 / 32] = (int8_t)Et;
}
