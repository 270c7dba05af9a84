// Jatai INT8 training kernels for MI355X (gfx950): shared formats, primitives and the device error record.
//
// Formats (same storage contract as the reference, jatai_cuda/jatai_cuda.cu:3-6 and ops.py:9):
//   block tensor  m int8 [R, C] + E int8 [R, C / BLK]; value m * 2^E; an all-zero block has E = -127.
//   raw tensor    acc int32 [R, C] + e int16 [R, C] (one exponent per element).
//   R16 tensor    m int16 [R, C] + E int8 [R, C / BLK] (16-bit residual stream).
// BLK is a template parameter of every kernel (32 or 128); the reference fixes 128 (ops.py:17).
//
// Every intermediate is an int32 kept below 2^30; the kernels check the bound where a proof does not cover it
// and record the first violation in `g_erro` (the reference's sentinel contract, jatai_cuda.cu:22-36,
// decoded by the host registry). Rounding is always half-to-even.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

#define E_ZERO (-127)
#define LIM (1 << 30)
#define SEM_TOPO (-100000)
#define U_MIN (-2147483647)

enum { E_ACUM = 1, E_EXP = 2, E_SAT = 3, E_DIV = 4, E_SHL = 5, E_ARG = 6 };

struct Erro {
    int n, codigo, kid, pad;
    long long idx, valor, aux;
};
extern __device__ Erro g_erro;

// Cold path, kept out of line so it does not inflate hot loops. First event wins.
__device__ __noinline__ void reporta(int codigo, int kid, long long idx, long long valor, long long aux);

// ---------------------------------------------------------------------------------------------- primitives
__device__ __forceinline__ int bitlen(int x) { return x == 0 ? 0 : 32 - __clz(x < 0 ? -x : x); }

// x * 2^-s rounded half to even (ops.py:42-51). s <= 0 is a left shift, checked against 2^30.
__device__ __forceinline__ int rnd(int x, int s, int kid, long long idx) {
    if (s <= 0) {
        if (s == 0 || x == 0) return x;
        s = -s;
        if (s > 30 || bitlen(x) + s > 30) { reporta(E_SHL, kid, idx, x, -s); return 0; }
        return x << s;
    }
    if (s > 30) return 0;                        // |x| < 2^30 < 2^(s-1): rounds to 0
    return (x + ((1 << (s - 1)) - 1) + ((x >> s) & 1)) >> s;
}

// rnd for a known s >= 0 with |x| < 2^30 (s >= 31 gives 0 through the same formula once s is clamped to 31)
__device__ __forceinline__ int rnd_d(int x, int s) {
    s = min(s, 31);
    if (s == 0) return x;
    return (x + ((1 << (s - 1)) - 1) + ((x >> s) & 1)) >> s;
}

// left shift of a possibly negative int as two's-complement bits (a signed left shift of a negative value is
// undefined in C++17)
__device__ __forceinline__ int shl(int x, int s) { return (int)((unsigned)x << s); }

// x * 2^-s for either sign of s where a left shift provably keeps every bit (no check)
__device__ __forceinline__ int desloca(int x, int s) { return s >= 0 ? rnd_d(x, s) : shl(x, min(-s, 31)); }

// a * b for -2^23 <= a, b < 2^23: the low 32 bits of the product, which is what a * b gives, from the full-rate
// 24-bit multiply (v_mul_i32_i24, and v_mad_i32_i24 when added) instead of the quarter-rate 32-bit one the
// compiler emits when it cannot bound the operands. Each use states why its operands lie in that range.
__device__ __forceinline__ int mul24(int a, int b) { return __mul24(a, b); }

// exp(-d/256) in Q15 for d >= 0: shift plus a cubic (ops.py:75-81). Every product is a 24-bit one: min(d, 6000)
// and 23637 are below 2^15, f < 2^15, and p stays within (-2^15, 2^15) through the three steps.
__device__ __forceinline__ int exp_int(int d) {
    int t = mul24(min(d, 6000), 23637);
    int n = t >> 22, f = (t & ((1 << 22) - 1)) >> 7;
    int p = -1295;
    p = (mul24(p, f) >> 15) + 7556;
    p = (mul24(p, f) >> 15) - 22645;
    p = (mul24(p, f) >> 15) + 32765;
    return n > 30 ? 0 : p >> n;
}
// exp(-(mx - u)/256) with the difference clamped before subtracting (mx - u may exceed 2^31)
__device__ __forceinline__ int exp_dif(int mx, int u) { return exp_int(u <= mx - 6000 ? 6000 : mx - u); }

// The softmax numerator exp_int(d) >> 3 (ops.py:203) as a table: d takes at most 6001 values, and from EXP_D0 on
// the numerator is 0, so EXP_D0 + 1 entries (the last 0) hold it exactly. Built at compile time by the same integer
// arithmetic; the compiler checks that every d in [EXP_D0, 6000] gives 0 and that EXP_D0 is the first such d.
// A kernel copies it into LDS (exp_tab_lds) and reads one 16-bit entry per score instead of the cubic's ~16
// instructions.
namespace tabexp {
constexpr int exp_int_c(int d) {
    const int t = (d < 6000 ? d : 6000) * 23637;
    const int n = t >> 22, f = (t & ((1 << 22) - 1)) >> 7;
    int p = -1295;
    p = ((p * f) >> 15) + 7556;
    p = ((p * f) >> 15) - 22645;
    p = ((p * f) >> 15) + 32765;
    return n > 30 ? 0 : p >> n;
}
constexpr int primeiro_zero() {
    int d = 6000;
    while (d > 0 && (exp_int_c(d - 1) >> 3) == 0) d--;
    return d;
}
}  // namespace tabexp
constexpr int EXP_D0 = tabexp::primeiro_zero();
constexpr int EXP_N = (EXP_D0 + 1 + 7) & ~7;                        // entries, padded to whole 16-byte chunks
static_assert(EXP_D0 > 0 && (tabexp::exp_int_c(EXP_D0 - 1) >> 3) != 0, "exp table: EXP_D0 is the first zero");
struct TabExp { unsigned short v[EXP_N]; };
constexpr TabExp faz_tab_exp() {
    TabExp t{};
    for (int d = 0; d < EXP_N; d++) t.v[d] = (unsigned short)(d < EXP_D0 ? tabexp::exp_int_c(d) >> 3 : 0);
    return t;
}
constexpr bool tab_exp_zero_depois() {
    for (int d = EXP_D0; d <= 6000; d++)
        if ((tabexp::exp_int_c(d) >> 3) != 0) return false;
    return true;
}
static_assert(tab_exp_zero_depois(), "exp table: the numerator is 0 for every d >= EXP_D0");
__constant__ const TabExp TAB_EXP = faz_tab_exp();
// copy the table into a workgroup's LDS (EXP_N / 8 chunks of 16 bytes); the caller's barrier publishes it
__device__ __forceinline__ void exp_tab_lds(unsigned short* t) {
    for (int c = threadIdx.x; c < EXP_N / 8; c += blockDim.x)
        reinterpret_cast<int4*>(t)[c] = reinterpret_cast<const int4*>(TAB_EXP.v)[c];
}
// The same copy in two halves: exp_tab_le loads a thread's chunks into registers, exp_tab_grava stores them, so
// the kernel's other loads can be issued in between (a store right after its load waits for it first). NCH chunks
// per thread: blockDim.x * NCH >= EXP_N / 8.
template <int NCH>
__device__ __forceinline__ void exp_tab_le(int4 (&r)[NCH]) {
#pragma unroll
    for (int k = 0; k < NCH; k++) {                                  // unconditional: past the table a thread re-reads
        const int c0 = threadIdx.x + k * blockDim.x;                  // its first chunk (blockDim.x <= EXP_N / 8)
        r[k] = reinterpret_cast<const int4*>(TAB_EXP.v)[c0 < EXP_N / 8 ? c0 : threadIdx.x];
    }
}
template <int NCH>
__device__ __forceinline__ void exp_tab_grava(unsigned short* t, const int4 (&r)[NCH]) {
#pragma unroll
    for (int k = 0; k < NCH; k++) {                                  // unconditional, as the loads (a thread writes its
        const int c0 = threadIdx.x + k * blockDim.x;                  // first chunk again: no other thread's)
        reinterpret_cast<int4*>(t)[c0 < EXP_N / 8 ? c0 : threadIdx.x] = r[k];
    }
}
// exp_dif(mx, u) >> 3 from the table for u <= mx: the difference, taken in unsigned arithmetic (no signed
// overflow), is exact (below 2^32) however far apart mx and u are, and every difference from EXP_D0 on reads the final 0 (an index never leaves the table)
__device__ __forceinline__ int exp_tab(const unsigned short* t, int mx, int u) { return t[min((unsigned)mx - (unsigned)u, (unsigned)EXP_D0)]; }

// The spec's isqrt (ops.py:84-89: 10 Newton steps from 2^ceil(bitlen(n)/2)) is floor(sqrt(n)) for every
// 1 <= n < 2^31 (checked over all of them) and 1 for n <= 0. Here: a float square root, within 0.01 of sqrt(n) for
// these n, whose floor is off by at most one and is corrected by one exact integer step either way.
__device__ __forceinline__ int isqrt_i(int n) {
    if (n <= 0) return 1;
    unsigned r = (unsigned)__builtin_sqrtf((float)n);
    r -= (unsigned)(r * r > (unsigned)n);
    r += (unsigned)((r + 1) * (r + 1) <= (unsigned)n);
    return (int)r;
}

// floor(a / b) for 0 <= a < 2^30, b >= 1 and a quotient below 2^20: a float estimate (relative error a few
// 2^-24, so within 1 of the quotient) corrected by one exact integer step either way -- in place of a 32-bit
// integer division, which costs about 40 VALU instructions.
__device__ __forceinline__ int div_exata(int a, int b) {
    int q = (int)((float)a * __builtin_amdgcn_rcpf((float)b));
    q -= (int)(q * b > a);
    q += (int)((q + 1) * b <= a);
    return q;
}

// largest of the four signed bytes of w
__device__ __forceinline__ int max_i8x4(int w) {
    return max(max((int)(int8_t)w, (int)(int8_t)(w >> 8)), max((int)(int8_t)(w >> 16), w >> 24));
}

__host__ __device__ constexpr int ilog2_c(int n) { return n <= 1 ? 0 : 1 + ilog2_c(n >> 1); }

// ---------------------------------------------------------------------------------------------- lane groups
// A block of BLK values is held by LPB consecutive lanes (a power of two <= 64), VPL values each.
// Reductions over the group run on DPP lane permutations (quad permutes, then the half-row and row mirrors: each
// an involution that pairs the two halves of the next larger group, so every lane ends with the group's result),
// a lane swap across rows for 32, and the whole-wave reduction of the device library for 64 -- no LDS
// round trip, except the one ds_bpermute of the 32-lane step. Every lane of a group is active where these run.
template <int LPB, class OP>
__device__ __forceinline__ int g_red(int v, OP op) {
    static_assert(LPB >= 1 && LPB <= 32 && (LPB & (LPB - 1)) == 0, "");
    if constexpr (LPB >= 2) v = op(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));    // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (LPB >= 4) v = op(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));    // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (LPB >= 8) v = op(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false));   // row_half_mirror
    if constexpr (LPB >= 16) v = op(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false));  // row_mirror
    if constexpr (LPB >= 32) v = op(v, __shfl_xor(v, 16));
    return v;
}
template <int LPB>
__device__ __forceinline__ int g_max(int v) {
    if constexpr (LPB == 64) return __ockl_wfred_max_i32(v);
    else return g_red<LPB>(v, [](int a, int b) { return max(a, b); });
}
template <int LPB>
__device__ __forceinline__ int g_sum(int v) {
    if constexpr (LPB == 64) return __ockl_wfred_add_i32(v);
    else return g_red<LPB>(v, [](int a, int b) { return a + b; });
}

// x * 2^-s rounded half to even for any int32 x and any s >= -20, in double precision: the conversion and the
// power-of-two scaling are exact (53-bit significand); adding 1.5 * 2^52 puts the value where doubles are spaced
// by 1, so that addition's round-to-nearest-even is rnd's, and its low word is the result in two's complement. A
// scale so small that the value leaves the normal range leaves it below 1/2, where the rounding gives 0 as rnd
// does. Three VALU instructions, against about twelve for the same rounding in integer form with a per-value
// shift; MI355X runs vector FP64 at the unpacked FP32 rate.
__device__ __forceinline__ int desl_f(int x, int s) {
    return __double2loint(__builtin_ldexp((double)x, -s) + 0x1.8p52);
}

// Quantize one block (LPB lanes x VPL values, per-element exponent e) into mantissas of MBITS bits plus one
// exponent (ops.py:58-72; 16-bit variant jatai_cuda.cu:451-483): topo = max(e + bitlen(v)) over nonzeros,
// E = topo - MBITS, q = rnd(v, E - e), E += 1 if any |q| > LIMQ, all-zero or E < -126 -> zero block.
// Returns E (E_ZERO for a zero block). idx0 is the flat index of this lane's first value (for sentinels).
// Written without per-value branches: e + bitlen(v) <= topo for every nonzero v bounds |v 2^(e - E)| below
// 2^MBITS, so after the +1 no |q| exceeds LIMQ and the spec's saturation check and clamp never act; a value out
// of range (|v| >= 2^30) is found from the block's largest |v| and reported, value by value, off the hot path.
template <int VPL, int LPB, typename MT, int MBITS, int LIMQ>
__device__ __forceinline__ int quant_grupo(const int (&v)[VPL], const int (&e)[VPL], MT (&m)[VPL], int kid, long long idx0) {
    int topo = SEM_TOPO;
    unsigned amax = 0;
#pragma unroll
    for (int i = 0; i < VPL; i++) {
        const unsigned a = (unsigned)(v[i] < 0 ? -v[i] : v[i]);
        amax = max(amax, a);
        topo = max(topo, a ? e[i] + 32 - (int)__clz((int)a) : SEM_TOPO);
    }
    if (amax >= (unsigned)LIM) {
#pragma unroll
        for (int i = 0; i < VPL; i++)
            if (v[i] >= LIM || v[i] <= -LIM) reporta(E_ACUM, kid, idx0 + i, v[i], e[i]);
    }
    topo = g_max<LPB>(topo);
    int E = topo - MBITS, q[VPL], qmax = 0;
#pragma unroll
    for (int i = 0; i < VPL; i++) { q[i] = desl_f(v[i], E - e[i]); qmax = max(qmax, q[i] < 0 ? -q[i] : q[i]); }
    if (g_max<LPB>(qmax) > LIMQ) {
        E += 1;
#pragma unroll
        for (int i = 0; i < VPL; i++) q[i] = desl_f(v[i], E - e[i]);
    }
    const bool zero = topo == SEM_TOPO || E < -126;
    const int manter = zero ? 0 : -1;
#pragma unroll
    for (int i = 0; i < VPL; i++) m[i] = (MT)(q[i] & manter);
    if (!zero && E > 126) reporta(E_EXP, kid, idx0, E, topo);
    return zero ? E_ZERO : E;
}
template <int VPL, int LPB>
__device__ __forceinline__ int quant8(const int (&v)[VPL], const int (&e)[VPL], int8_t (&m)[VPL], int kid, long long idx0) {
    return quant_grupo<VPL, LPB, int8_t, 7, 127>(v, e, m, kid, idx0);
}

// quant8 of values whose per-value exponents satisfy |e| <= 990 (the GEMM epilogue: e = RA + RB - 4), through
// d = v 2^e in double precision, exact, normal and finite for every nonzero int32 v. bitlen(|v|) + e is the binary
// exponent of d, so topo is read from the exponent field of the block's largest |d|. q = rnd(d 2^-E) is the low
// word of fma(d, 2^-E, 1.5 * 2^52) (the sum lies where doubles are spaced by 1, so the FMA's rounding is the
// half-to-even rounding), and that rounding is monotone: max |q| = rnd(max |d| 2^-E), so the bump test takes one
// FMA per lane instead of a pass over the values. Same results and sentinels as quant8. CHECA = false drops the
// accumulator-range sentinel for callers whose values are int8 mantissas (|v| <= 128 < LIM: it cannot fire).
template <int VPL, int LPB, bool CHECA = true>
__device__ __forceinline__ int quant8_d(const int (&v)[VPL], const int (&e)[VPL], int8_t (&m)[VPL], int kid, long long idx0) {
    double d[VPL], dmax = 0.0;
    unsigned fora = 0;                                              // max of v + LIM - 1 as unsigned: >= 2 LIM - 1 iff |v| >= LIM
#pragma unroll
    for (int i = 0; i < VPL; i++) {
        d[i] = __builtin_ldexp((double)v[i], e[i]);
        dmax = __builtin_fmax(dmax, __builtin_fabs(d[i]));
        if constexpr (CHECA) fora = max(fora, (unsigned)v[i] + (unsigned)(LIM - 1));
    }
    if (CHECA && fora >= 2u * LIM - 1) {
#pragma unroll
        for (int i = 0; i < VPL; i++)
            if (v[i] >= LIM || v[i] <= -LIM) reporta(E_ACUM, kid, idx0 + i, v[i], e[i]);
    }
    // exponent field - 1022 = floor(log2 dmax) + 1; a lane of zeros gives -1022, below every real topo
    const int topo = g_max<LPB>((__double2hiint(dmax) >> 20) - 1022);
    const int E0 = topo - 7;
    const double k0 = __hiloint2double((1023 - E0) << 20, 0);
    const int bump = g_max<LPB>(__double2loint(__builtin_fma(dmax, k0, 0x1.8p52))) > 127;
    const int E = E0 + bump;
    const double k = bump ? k0 * 0.5 : k0;                          // 2^-E
    const bool zero = E < -126;                                     // also the all-zero block (topo = -1022)
    const int manter = zero ? 0 : -1;
#pragma unroll
    for (int i = 0; i < VPL; i++) m[i] = (int8_t)(__double2loint(__builtin_fma(d[i], k, 0x1.8p52)) & manter);
    if (!zero && E > 126) reporta(E_EXP, kid, idx0, E, topo);
    return zero ? E_ZERO : E;
}


// quant8 through quant8_d when every exponent of the group lies in [-990, 990] (the momentum's, whose exponents
// are at least -148; the raw inputs of quant, produced by GEMMs as RA + RB - 4), else through the generic quant8.
template <int VPL, int LPB>
__device__ __forceinline__ int quant8_f(const int (&v)[VPL], const int (&e)[VPL], int8_t (&m)[VPL], int kid, long long idx0) {
    unsigned fora = 0;                                              // e + 990 as unsigned: above 1980 iff |e| > 990
#pragma unroll
    for (int i = 0; i < VPL; i++) fora = max(fora, (unsigned)(e[i] + 990));
    if (g_max<LPB>((int)(fora > 1980u)) != 0) return quant8<VPL, LPB>(v, e, m, kid, idx0);
    return quant8_d<VPL, LPB>(v, e, m, kid, idx0);
}

// x * 2^-s rounded half to even for one s shared by a group of values (|x| < 2^31; s < 0 is a left shift the
// caller knows to be exact): the scale 2^-s is built once, then each value is fma(x, 2^-s, 1.5 * 2^52), whose
// low word is the rounded result (the rounding of desl_f): a conversion and an FMA, with no branch. A large s
// gives 0, as rnd does for s > 30.
struct Desl {
    double k;
    __device__ __forceinline__ explicit Desl(int s) { k = __hiloint2double((1023 - min(max(s, -40), 1000)) << 20, 0); }
    __device__ __forceinline__ int operator()(int x) const { return __double2loint(__builtin_fma((double)x, k, 0x1.8p52)); }
};

// quant8 for a block whose values all share exponent e and satisfy |v| < 2^30 (the element-wise ops whose
// inputs are block tensors): the spec's rules (ops.py:58-72) with the per-element work reduced by two facts.
// topo = e + bitlen(max |v|), because bitlen is monotone in |v|; and half-to-even rounding is monotone and odd,
// so max |q| = rnd(max |v|, E - e) and the overflow test (any |q| > 127 -> E + 1) is decided on the block
// maximum before any value is rounded. Each value is then rounded once, and no |q| exceeds 127 (so the
// saturation clamp of the spec never acts). Returns E (E_ZERO for a zero block; those mantissas are 0).
template <int VPL, int LPB, bool REPORTA = true, int MBITS = 7, int LIMQ = 127>
__device__ __forceinline__ int quant_u(const int (&v)[VPL], int e, int (&q)[VPL], int kid, long long idx0) {
    // in double precision: bitlen(max |v|) is the exponent field of max |(double)v| (exact for int32), and each
    // value is rounded by one FMA with 1.5 * 2^52 (exact left shifts for s <= 0); the bump test is the rounding
    // of the largest |v|
    double d[VPL], dmax = 0.0;
#pragma unroll
    for (int i = 0; i < VPL; i++) {
        d[i] = (double)v[i];
        dmax = __builtin_fmax(dmax, __builtin_fabs(d[i]));
    }
    if (REPORTA && dmax >= (double)LIM) {
#pragma unroll
        for (int i = 0; i < VPL; i++)
            if (v[i] >= LIM || v[i] <= -LIM) reporta(E_ACUM, kid, idx0 + i, v[i], e);
    }
    const int bl = g_max<LPB>((__double2hiint(dmax) >> 20) - 1022);      // bitlen(max |v|); -1022 for all zeros
    const int s0 = bl - MBITS;
    const double k0 = __hiloint2double((1023 - s0) << 20, 0);            // 2^-s0
    const int bump = g_max<LPB>(__double2loint(__builtin_fma(dmax, k0, 0x1.8p52))) > LIMQ;
    const int E = e + s0 + bump;
    const double k = bump ? k0 * 0.5 : k0;
    const bool zero = bl <= 0 || E < -126;
    // every value is rounded, then masked: a select per value here makes the compiler branch around the rounding
    const int manter = zero ? 0 : -1;
#pragma unroll
    for (int i = 0; i < VPL; i++) q[i] = __double2loint(__builtin_fma(d[i], k, 0x1.8p52)) & manter;
    if (REPORTA && !zero && E > 126) reporta(E_EXP, kid, idx0, E, e + bl);
    return zero ? E_ZERO : E;
}
template <int VPL, int LPB, bool REPORTA = true>
__device__ __forceinline__ int quant8_u(const int (&v)[VPL], int e, int (&q)[VPL], int kid, long long idx0) {
    return quant_u<VPL, LPB, REPORTA, 7, 127>(v, e, q, kid, idx0);
}

// quant8_u with int8 mantissas out (sentinels reported)
template <int VPL, int LPB>
__device__ __forceinline__ int quant8_u8(const int (&v)[VPL], int e, int8_t (&m)[VPL], int kid, long long idx0) {
    int q[VPL];
    const int E = quant8_u<VPL, LPB>(v, e, q, kid, idx0);
#pragma unroll
    for (int i = 0; i < VPL; i++) m[i] = (int8_t)q[i];
    return E;
}

// Quantize a block whose values all share exponent e and are built from int8 mantissas (|v| far below 2^30): the
// fused GEMM epilogues, as jatai_cuda.cu:161-188 does; quant8_u without its sentinel reports (the callers report
// an out-of-range exponent themselves, naming their epilogue).
template <int VPL, int LPB>
__device__ __forceinline__ int quant8_comum(const int (&v)[VPL], int e, int8_t (&m)[VPL]) {
    int q[VPL];
    const int E = quant8_u<VPL, LPB, false>(v, e, q, 0, 0);
#pragma unroll
    for (int i = 0; i < VPL; i++) m[i] = (int8_t)q[i];
    return E;
}

// ---------------------------------------------------------------------------------------------- stochastic rounding
// The residual add of gemm_soma under jt_res_estocastico (no spec; restated from the reference kernel text,
// jatai_cuda.cu:146-159 and :375): x * 2^-s rounded up with probability equal to the discarded fraction, the
// coin being a 32-bit integer hash of a per-value seed mixed with the value itself.
__device__ __forceinline__ uint32_t hash32(uint32_t x) {
    x ^= x >> 16; x *= 0x7feb352dU;
    x ^= x >> 15; x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}
__device__ __forceinline__ int desloca_est(int x, int s, uint32_t h) {
    if (s <= 0) return (int)((unsigned)x << min(-s, 31));
    s = min(s, 31);
    const long long piso = (long long)x >> s, resto = (long long)x - (piso << s);     // 0 <= resto < 2^s
    const long long u = (long long)(hash32(h ^ (uint32_t)x * 0x9E3779B1u) & (uint32_t)((1ull << s) - 1));
    return (int)(piso + (u < resto ? 1 : 0));
}
// quant8 of a block with one exponent e, every value rounded by desloca_est with its seed h[i] (the reference's
// quant_grupo16<true>: bl = bitlen of the largest |v|, E = e + bl - 7, again one up if a mantissa passes 127,
// zero block below 2^-126)
template <int VPL, int LPB>
__device__ __forceinline__ int quant8_est(const int (&v)[VPL], int e, int8_t (&m)[VPL], const uint32_t (&h)[VPL]) {
    int bl = 0;
#pragma unroll
    for (int i = 0; i < VPL; i++) bl = max(bl, bitlen(v[i]));
    bl = g_max<LPB>(bl);
    int E = e + bl - 7, q[VPL], qmax = 0;
#pragma unroll
    for (int i = 0; i < VPL; i++) { q[i] = desloca_est(v[i], bl - 7, h[i]); qmax = max(qmax, q[i] < 0 ? -q[i] : q[i]); }
    if (g_max<LPB>(qmax) > 127) {
        E += 1;
#pragma unroll
        for (int i = 0; i < VPL; i++) q[i] = desloca_est(v[i], bl - 6, h[i]);
    }
    const bool zero = bl == 0 || E < -126;
#pragma unroll
    for (int i = 0; i < VPL; i++) m[i] = zero ? 0 : (int8_t)q[i];
    return zero ? E_ZERO : E;
}

// ---------------------------------------------------------------------------------------------- vector I/O
template <int N>
__device__ __forceinline__ void le_i8(const int8_t* p, int (&v)[N]) {
    static_assert(N == 4 || N == 8 || N == 16, "");
    if constexpr (N == 4) {
        const int w = *reinterpret_cast<const int*>(p);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = (int)(int8_t)(w >> (8 * i));
    } else if constexpr (N == 8) {
        const int2 w = *reinterpret_cast<const int2*>(p);
#pragma unroll
        for (int i = 0; i < 4; i++) { v[i] = (int)(int8_t)(w.x >> (8 * i)); v[4 + i] = (int)(int8_t)(w.y >> (8 * i)); }
    } else {
        const int4 w = *reinterpret_cast<const int4*>(p);
        const int ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) v[4 * j + i] = (int)(int8_t)(ws[j] >> (8 * i));
    }
}
// N int8 values packed into one store. NT (the default): a non-temporal store (global_store ... nt), which
// leaves fewer lines of the step's large outputs for the kernel's end-of-launch L2 write-back to other XCDs'
// readers (config-4 step 2.918 -> 2.909 ms); the attention forward's output keeps plain stores (its reader, the
// next GEMM, measured faster so).
template <int N, bool NT = true>
__device__ __forceinline__ void grava_i8(int8_t* p, const int8_t (&m)[N]) {
    typedef int nt2 __attribute__((ext_vector_type(2)));
    typedef int nt4 __attribute__((ext_vector_type(4)));
    int ws[(N + 3) / 4];
#pragma unroll
    for (int j = 0; j < N / 4; j++)
        ws[j] = (int)(uint8_t)m[4 * j] | ((int)(uint8_t)m[4 * j + 1] << 8) | ((int)(uint8_t)m[4 * j + 2] << 16) |
                ((int)(uint8_t)m[4 * j + 3] << 24);
    if constexpr (!NT) {
        if constexpr (N == 4) *reinterpret_cast<int*>(p) = ws[0];
        else if constexpr (N == 8) *reinterpret_cast<int2*>(p) = make_int2(ws[0], ws[1]);
        else *reinterpret_cast<int4*>(p) = make_int4(ws[0], ws[1], ws[2], ws[3]);
    } else if constexpr (N == 4) {
        __builtin_nontemporal_store(ws[0], reinterpret_cast<int*>(p));
    } else if constexpr (N == 8) {
        __builtin_nontemporal_store(nt2{ws[0], ws[1]}, reinterpret_cast<nt2*>(p));
    } else {
        __builtin_nontemporal_store(nt4{ws[0], ws[1], ws[2], ws[3]}, reinterpret_cast<nt4*>(p));
    }
}
// 16 int8 values: one 16-byte load, and its unpacking to ints (split so that loads can be issued early)
__device__ __forceinline__ int4 ld16(const int8_t* p) { return *reinterpret_cast<const int4*>(p); }
__device__ __forceinline__ void abre_i8(const int4 x, int (&v)[16]) {
    const int ws[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) v[4 * j + i] = (int)(int8_t)(ws[j] >> (8 * i));
}

// store N int mantissas known to lie in [-127, 127] as int8
template <int N>
__device__ __forceinline__ void grava_q8(int8_t* p, const int (&q)[N]) {
    static_assert(N == 4 || N == 8 || N == 16, "");
    unsigned ws[N / 4];
#pragma unroll
    for (int j = 0; j < N / 4; j++)
        ws[j] = ((unsigned)q[4 * j] & 255u) | (((unsigned)q[4 * j + 1] & 255u) << 8) | (((unsigned)q[4 * j + 2] & 255u) << 16) |
                ((unsigned)q[4 * j + 3] << 24);
    if constexpr (N == 4) *reinterpret_cast<unsigned*>(p) = ws[0];
    else if constexpr (N == 8) *reinterpret_cast<uint2*>(p) = make_uint2(ws[0], ws[1]);
    else *reinterpret_cast<uint4*>(p) = make_uint4(ws[0], ws[1], ws[2], ws[3]);
}
template <int N>
__device__ __forceinline__ void le_i32(const int* p, int (&v)[N]) {
#pragma unroll
    for (int j = 0; j < N; j += 4) {
        const int4 w = *reinterpret_cast<const int4*>(p + j);
        v[j] = w.x; v[j + 1] = w.y; v[j + 2] = w.z; v[j + 3] = w.w;
    }
}
template <int N>
__device__ __forceinline__ void le_i16(const int16_t* p, int (&v)[N]) {
    static_assert(N % 4 == 0, "");
#pragma unroll
    for (int j = 0; j < N; j += 4) {
        const int2 w = *reinterpret_cast<const int2*>(p + j);
        v[j] = (int)(int16_t)(w.x & 0xffff); v[j + 1] = w.x >> 16;
        v[j + 2] = (int)(int16_t)(w.y & 0xffff); v[j + 3] = w.y >> 16;
    }
}
template <int N>
__device__ __forceinline__ void grava_i16(int16_t* p, const int16_t (&m)[N]) {
#pragma unroll
    for (int j = 0; j < N; j += 4) {
        const int a = (int)(uint16_t)m[j] | ((int)(uint16_t)m[j + 1] << 16);
        const int b = (int)(uint16_t)m[j + 2] | ((int)(uint16_t)m[j + 3] << 16);
        *reinterpret_cast<int2*>(p + j) = make_int2(a, b);
    }
}
