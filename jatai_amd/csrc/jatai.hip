// libjatai.so for MI355X (gfx950): the C ABI of the Jatai INT8 training hot path.
//
// Entry points keep the reference's names, argument order, pointer/size conventions and return codes
// (jatai_cuda/jatai_cuda.cu:1061-1201; declared in include/jatai.h): the caller allocates every output, pointers
// are raw device addresses (NULL for an absent operand), element counts are long long, every launch carries a
// trailing launch id `kid`, and the return value is the runtime's error code (0 = success). All launches go to
// the stream set with jt_stream (torch's current, possibly capturing, stream). Like the reference, the module
// state (stream, block size, tuning knobs) is global and not thread-safe.
//
// One translation unit: the kernels and the device error record `g_erro` live in the same code object.
#include <algorithm>
#include <type_traits>

#include "jt_comum.h"
#include "jt_elem.hip"
#include "jt_linhas.hip"
#include "jt_gemm.hip"
#include "jt_atencao.hip"
#include "jt_atencao_hd.hip"
#include "jt_atencao_ws.hip"

__device__ Erro g_erro;
// A host-pinned flag beside the record (set up by the first jt_erro_le): 1 once an event is recorded, 0 after each
// clear. A read of the record that finds it 0 needs no device-to-host copy: the record is then all zeros.
__device__ int* g_erro_flag = nullptr;
__device__ __noinline__ void reporta(int codigo, int kid, long long idx, long long valor, long long aux) {
    if (atomicAdd(&g_erro.n, 1) == 0) {
        g_erro.codigo = codigo;
        g_erro.kid = kid;
        g_erro.idx = idx;
        g_erro.valor = valor;
        g_erro.aux = aux;
        __threadfence();
        if (int* f = g_erro_flag) { *f = 1; __threadfence_system(); }
    }
}

__global__ void k_erro_limpa() {
    if (threadIdx.x < sizeof(Erro) / sizeof(int)) reinterpret_cast<int*>(&g_erro)[threadIdx.x] = 0;
    if (threadIdx.x == 0)
        if (int* f = g_erro_flag) *f = 0;
}

static hipStream_t g_stream = 0;
static int g_blk = 128;                 // block size of every tensor: 32 or 128
static int g_alvo_wg = 1024;            // GEMM K-split target: tiles x K-splits per launch
static int g_gemm_bm = 0;               // GEMM tile rows: 0 = automatic, or 32, 64, 128 forced (jt_gemm_bm)
static int g_linhas = 0;                // head-width-4 attention layout (jt_atencao_linhas): 1 or 2 query rows per thread, 0 automatic
static int g_atencao_mfma = 1;          // head width 64: matrix-core attention (1) or the dot2 kernels (0)

static int fim() { return (int)hipGetLastError(); }
// Every kernel moves 8- or 16-byte vectors: operands must be 16-byte aligned (torch allocations are 256-byte
// aligned). A misaligned pointer is rejected on the host with hipErrorInvalidValue.
static bool alinhado(const void* p) { return ((uintptr_t)p & 15) == 0; }
template <typename... P>
static bool alinhados(P... p) { return (alinhado(p) && ...); }
static unsigned grade_elem(long long nblocos) { return (unsigned)((nblocos * g_blk + 2047) / 2048); }
// kernels with 16 values per lane (soma, relu2, relu2_back, peso, otimizador)
static unsigned grade_u(long long nblocos) { return (unsigned)((nblocos * g_blk + 4095) / 4096); }
static int ilog2(long long n) { int l = 0; while ((2LL << l) <= n) l++; return l; }
// attention backward's dS width: 12 bits up to T = 128, one bit less per doubling of T beyond it, rounded up, so
// that T (2^dsb - 1) (127 << 4) < 2^30 at every T
static int ds_bits(int T) { return 12 - std::max(0, ilog2(2LL * T - 1) - 7); }

// Dynamic LDS above 64 KiB must be allowed per kernel (gfx950 has 160 KiB per CU): raised once per kernel and
// size, remembered by kernel address (every k_gemm instantiation has the same function type).
template <typename K>
static void lds_max(K* k, size_t lds) {
    static const void* chave[64];
    static size_t feito[64];
    static int n = 0;
    if (lds <= 65536) return;
    const void* f = reinterpret_cast<const void*>(k);
    int i = 0;
    while (i < n && chave[i] != f) i++;
    if (i < n && feito[i] >= lds) return;
    (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);   // a refusal surfaces at the launch
    if (i == n && n < 64) { chave[n] = f; feito[n] = lds; n++; }
    else if (i < n) feito[i] = lds;
}

#define POR_BLK(CHAMADA) (g_blk == 32 ? (CHAMADA(32)) : (CHAMADA(128)))

// K-splits inside a workgroup: doubled (up to 4) while tiles x splits stays within g_alvo_wg and each split
// keeps at least four K-blocks. A split adds a group of 4 waves to the workgroup: more resident waves per SIMD to
// hide LDS and MFMA latency under the VALU rounding work, as long as the grid does not already fill the chip
// (1024 = 256 CUs x 4 SIMDs). (Each K-split holds two stage buffers in LDS -- 10 KiB each at BLK=32, 21 KiB at
// BLK=128, 160 KiB per workgroup.) Up to 4 splits for modes 0-2 at BLK=32 (mode 2 at 1024 threads: 60 VGPRs, no
// spills; config 4's residual-add GEMMs 14.2 -> 13.4 us on average), 2 for the fused ReLU^2 epilogues.
// K up to 65536; past 4096 (one chunk of shift tables) the exponent rows are read with 16-byte loads, so the
// number of K-blocks must be a multiple of 16
static bool k_ok(int K) { return K <= 4096 || (K <= 65536 && (K / g_blk) % 16 == 0); }

// Tile of 32 R rows. Forced by jt_gemm_bm: 64 (R = 2) or 128 (R = 4), falling back to the tallest tile that
// divides M (every M here is a multiple of 32). Automatic: R = 1, except the fused ReLU^2 GEMMs (modes 3 and 4)
// when 128-row tiles make one or two workgroups per CU -- measured on MI355X at M = N = 2048, K = 512 (config 4):
// 20.4 / 19.7 us against 21.5 / 21.2 at 32 rows; with many more tiles (config 5, M = 16384) and at every other
// step shape 32 rows are fastest.
static int gemm_r(int M, int N = 0, int modo = 0) {
    int r = g_gemm_bm >= 128 ? 4 : g_gemm_bm >= 64 ? 2 : 1;
    const long long t128 = (long long)(M / 128) * (N / 128);
    if (g_gemm_bm == 0 && (modo == 3 || modo == 4) && t128 >= 256 && t128 <= 512) r = 4;
    while (r > 1 && M % (32 * r)) r /= 2;
    return r;
}
static int gemm_divisoes_r(int M, int N, int K, int modo, int r) {
    const long long tiles = (long long)(M / (32 * r)) * (N / gemm::BN);
    const int nb = K / g_blk, ksmax = std::min((g_blk == 32 && modo < 3) ? 4 : 2, 4 / r);   // 256 R KS <= 1024 threads
    int ks = 1;
    while (ks < ksmax && tiles * 2 * ks <= g_alvo_wg && nb >= 8 * ks) ks *= 2;
    return ks;
}
static int gemm_divisoes(int M, int N, int K, int modo) { return gemm_divisoes_r(M, N, K, modo, gemm_r(M, N, modo)); }

extern "C" {

// ---------------------------------------------------------------------------------------------- state
// jatai_cuda.cu:1062: reads the record after every launch so far, on any stream, has finished.
// The flag of each device (host-pinned, allocated at that device's first read and kept to the process's end).
static volatile int* g_flag_h[64] = {};
int jt_erro_le(long long* out) {
    hipError_t c = hipDeviceSynchronize();
    int dev = 0;
    if (c == hipSuccess) c = hipGetDevice(&dev);
    if (c != hipSuccess) return -(int)c;
    volatile int* f = dev >= 0 && dev < 64 ? g_flag_h[dev] : nullptr;
    if (f != nullptr && *f == 0) {                  // no event since the last clear: the record is all zeros
        for (int i = 0; i < 6; i++) out[i] = 0;
        return 0;
    }
    Erro e;
    c = hipMemcpyFromSymbol(&e, HIP_SYMBOL(g_erro), sizeof(Erro), 0, hipMemcpyDeviceToHost);
    if (c != hipSuccess) return -(int)c;
    out[0] = e.n; out[1] = e.codigo; out[2] = e.kid; out[3] = e.idx; out[4] = e.valor; out[5] = e.aux;
    if (f == nullptr && dev >= 0 && dev < 64) {     // first read on this device (idle: synchronized above)
        void* h = nullptr;
        int* hd = nullptr;
        if (hipHostMalloc(&h, sizeof(int), hipHostMallocCoherent) == hipSuccess) {
            *static_cast<volatile int*>(h) = e.n > 0 ? 1 : 0;
            if (hipHostGetDevicePointer(reinterpret_cast<void**>(&hd), h, 0) == hipSuccess &&
                hipMemcpyToSymbol(HIP_SYMBOL(g_erro_flag), &hd, sizeof(hd)) == hipSuccess)
                g_flag_h[dev] = static_cast<volatile int*>(h);
        }
        (void)hipGetLastError();                    // a failed set-up leaves the copy path, and no error behind
    }
    return e.n;
}
// jatai_cuda.cu:1069: clears the record. A kernel on the library's stream rather than a synchronous copy: the
// launches before it cannot write into the cleared record, and the host does not wait for the GPU to drain.
int jt_erro_limpa() {
    k_erro_limpa<<<1, 64, 0, g_stream>>>();
    return fim();
}
int jt_sincroniza() { return (int)hipDeviceSynchronize(); }
void jt_stream(void* st) { g_stream = (hipStream_t)st; }
void jt_gemm_split(int alvo) { g_alvo_wg = alvo > 0 ? alvo : 1024; }
// jatai_cuda.cu:1090: GEMM tile rows, 0 automatic (32), or 64 / 128 forced (32 forces the default); same bits.
void jt_gemm_bm(int bm) { g_gemm_bm = bm; }
// jatai_cuda.cu:1091: query rows per thread of the head-width-4 attention, 1 (default) or 2 (rows i and T - 1 - i,
// which balances the causal work); same bits.
void jt_atencao_linhas(int n) { g_linhas = n == 1 || n == 2 ? n : 0; }
// No reference counterpart: selects the matrix-core (1, default) or dot2 (0) attention kernels at head width 64.
void jt_atencao_mfma(int ligado) { g_atencao_mfma = ligado ? 1 : 0; }
// jatai_cuda.cu:1087: stochastic rounding of gemm_soma's residual add. A synchronous copy into the device global
// g_res_est of the current device; gemm_soma kernels read it when they run.
int jt_res_estocastico(int ligado) {
    const int v = ligado ? 1 : 0;
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_res_est), &v, sizeof(int));
}
// No reference counterpart: the reference fixes BLK = 128 (jatai_cuda.cu:16).
int jt_bloco(int blk) {
    if (blk != 32 && blk != 128) return (int)hipErrorInvalidValue;
    g_blk = blk;
    return 0;
}
int jt_bloco_atual() { return g_blk; }

// ---------------------------------------------------------------------------------------------- GEMM
// No reference counterpart: the K-split count jt_gemm_f uses for a shape (workgroup = 256 x splits threads).
int jt_gemm_divisoes(int M, int N, int K, int modo) { return gemm_divisoes(M, N, K, modo); }
// No reference counterpart: the tile rows (32, 64 or 128) jt_gemm_f uses for a shape and mode.
int jt_gemm_tile(int M, int N, int modo) { return 32 * gemm_r(M, N, modo); }
}  // extern "C"
// modes 0-4 (jt_gemm_f) and 6 (jt_gemm_soma16)
static int gemm_f(const void* A, const void* EA, const void* B, const void* EB, void* Cm, void* CE, void* C32, void* Ce, const void* Xm,
                  const void* XE, void* Om2, void* OE2, int M, int N, int K, int modo, int kid) {
    using namespace gemm;
    if (M <= 0 || N <= 0 || K <= 0 || M % BM || N % BN || K % g_blk || !k_ok(K)) return (int)hipErrorInvalidValue;
    if (!alinhados(A, EA, B, EB, Cm, CE, C32, Ce, Xm, XE, Om2, OE2)) return (int)hipErrorInvalidValue;
    const int nb = K / g_blk, r = gemm_r(M, N, modo);
    // mode 4 with Om2 (T(gh)) and mode 3 with C32, Ce (T(a)): the transposed copy needs a single K-split (BLK = 32 only)
    if (modo == 4 && (Om2 || OE2) && (g_blk != 32 || !Om2 || !OE2)) return (int)hipErrorInvalidValue;
    if (modo == 3 && (C32 || Ce) && (g_blk != 32 || !C32 || !Ce)) return (int)hipErrorInvalidValue;
    const int ks = ((modo == 4 && Om2) || (modo == 3 && C32)) ? 1 : gemm_divisoes_r(M, N, K, modo, r);
    const dim3 grade(N / BN, M / (32 * r));
    const size_t lds = gemm_lds(nb, ks, g_blk, r);
#define ARGS (const int8_t*)A, (const int8_t*)EA, (const int8_t*)B, (const int8_t*)EB, (int8_t*)Cm, (int8_t*)CE, (int*)C32, (int16_t*)Ce, \
             (const int8_t*)Xm, (const int8_t*)XE, (int8_t*)Om2, (int8_t*)OE2, M, N, K, kid
#define L(BL, MD, S, RR) (lds_max(k_gemm<BL, MD, S, RR>, lds), k_gemm<BL, MD, S, RR><<<grade, 256 * RR * S, lds, g_stream>>>(ARGS))
#define LS2(BL, MD, RR) (ks == 1 ? L(BL, MD, 1, RR) : L(BL, MD, 2, RR))
#define LS4(BL, MD) (ks == 1 ? L(BL, MD, 1, 1) : ks == 2 ? L(BL, MD, 2, 1) : L(BL, MD, 4, 1))
#define LR(BL, MD, LS1) (r == 1 ? LS1 : r == 2 ? LS2(BL, MD, 2) : L(BL, MD, 1, 4))
#define LB2(MD) (g_blk == 32 ? LR(32, MD, LS2(32, MD, 1)) : LR(128, MD, LS2(128, MD, 1)))
#define LB4(MD) (g_blk == 32 ? LR(32, MD, LS4(32, MD)) : LR(128, MD, LS2(128, MD, 1)))
    switch (modo) {
        case 0: LB4(0); break;
        case 1: LB4(1); break;
        case 2: LB4(2); break;
        case 3: LB2(3); break;
        case 4: LB2(4); break;
        case 6: LB2(6); break;
    }
#undef LB2
#undef LB4
#undef LR
#undef LS2
#undef LS4
#undef L
#undef ARGS
    return fim();
}
extern "C" {
int jt_gemm_f(const void* A, const void* EA, const void* B, const void* EB, void* Cm, void* CE, void* C32, void* Ce, const void* Xm,
              const void* XE, void* Om2, void* OE2, int M, int N, int K, int modo, int kid) {
    if (modo < 0 || modo > 4) return (int)hipErrorInvalidValue;
    return gemm_f(A, EA, B, EB, Cm, CE, C32, Ce, Xm, XE, Om2, OE2, M, N, K, modo, kid);
}
// No reference counterpart: Z16 = soma16(X16, gemm(A, B)) and Y8 = para8(Z16) in one launch -- the 16-bit residual
// stream's add (modelo.py:67-72, 78-84) and the INT8 copy the next RMSNorm reads -- with the bits of jt_gemm
// (mode 0), jt_soma16 and jt_para8 in turn. X16, Z16 int16 [M, N]; XE, ZE, YE8 int8 [M, N / BLK]; Y8 int8 [M, N].
int jt_gemm_soma16(const void* A, const void* EA, const void* B, const void* EB, const void* X16, const void* XE, void* Z16, void* ZE,
                   void* Y8, void* YE8, int M, int N, int K, int kid) {
    if (!X16 || !XE || !Z16 || !ZE || !Y8 || !YE8) return (int)hipErrorInvalidValue;
    return gemm_f(A, EA, B, EB, Z16, ZE, nullptr, nullptr, X16, XE, Y8, YE8, M, N, K, 6, kid);
}
int jt_gemm(const void* A, const void* EA, const void* B, const void* EB, void* Cm, void* CE, void* C32, void* Ce, int M, int N, int K,
            int modo, int kid) {
    return jt_gemm_f(A, EA, B, EB, Cm, CE, C32, Ce, nullptr, nullptr, nullptr, nullptr, M, N, K, modo, kid);
}

// No reference counterpart: n raw-output GEMMs sharing K in launches of up to 64 (host array of EntradaG, device
// pointers inside); entry i equals jt_gemm(A, EA, B, EB, NULL, NULL, C32, Ce, M, N, K, 1, kid + i).
// compacto = 1: Ce holds the exponents as the vectors Ce[i] = RA_i (i < M), Ce[M + j] = RB_j - 4 (M + N int16); the
// raw exponent of (i, j) is their sum. All entries of a launch (64 at a time) share the setting.
struct EntradaG { const void *A, *EA, *B, *EB; void *C32, *Ce; int M, N, K, compacto; };
int jt_gemm_lote(const void* entradas, int n, int kid) {
    using namespace gemm;
    if (n < 0 || (n > 0 && !entradas)) return (int)hipErrorInvalidValue;
    const EntradaG* e = (const EntradaG*)entradas;
    for (int base = 0; base < n; base += LOTE_G) {
        LoteG L;
        L.n = std::min(LOTE_G, n - base);
        L.K = e[base].K;
        L.compacto = e[base].compacto;
        int r = 4;                                                   // the tallest forced tile every M of the group allows
        for (int i = 0; i < L.n; i++) r = std::min(r, gemm_r(e[base + i].M > 0 ? e[base + i].M : 32));
        long long tot = 0;
        for (int i = 0; i < L.n; i++) {
            const EntradaG& x = e[base + i];
            if (x.M <= 0 || x.N <= 0 || x.K != L.K || x.M % BM || x.N % BN || x.K % g_blk || !k_ok(x.K) || x.K <= 0) return (int)hipErrorInvalidValue;
            if (x.compacto != L.compacto || (x.compacto != 0 && x.compacto != 1)) return (int)hipErrorInvalidValue;
            if (!alinhados(x.A, x.EA, x.B, x.EB, x.C32, x.Ce)) return (int)hipErrorInvalidValue;
            L.A[i] = (const int8_t*)x.A; L.EA[i] = (const int8_t*)x.EA; L.B[i] = (const int8_t*)x.B; L.EB[i] = (const int8_t*)x.EB;
            L.C32[i] = (int*)x.C32; L.Ce[i] = (int16_t*)x.Ce; L.M[i] = x.M; L.N[i] = x.N; L.ini[i] = (int)tot;
            tot += (long long)(x.M / (32 * r)) * (x.N / BN);
        }
        if (tot > 0x7fffffff) return (int)hipErrorInvalidValue;
        L.ini[L.n] = (int)tot;
        if (tot == 0) continue;
        // K-splits for the whole group, by the rule of jt_gemm_f with the group's tile count
        const int nb = L.K / g_blk, ksmax = std::min(g_blk == 32 ? 4 : 2, 4 / r);
        int ks = 1;
        while (ks < ksmax && tot * 2 * ks <= g_alvo_wg && nb >= 8 * ks) ks *= 2;
        const size_t lds = gemm_lds(nb, ks, g_blk, r, gemm::CTAB_LOTE);
#define L_(BL, S, RR) (lds_max(k_gemm_lote<BL, S, RR>, lds), k_gemm_lote<BL, S, RR><<<(unsigned)tot, 256 * RR * S, lds, g_stream>>>(L, kid + base))
        if (r == 4) { if (g_blk == 32) L_(32, 1, 4); else L_(128, 1, 4); }
        else if (r == 2) { if (g_blk == 32) { if (ks == 1) L_(32, 1, 2); else L_(32, 2, 2); } else { if (ks == 1) L_(128, 1, 2); else L_(128, 2, 2); } }
        else if (g_blk == 32) { if (ks == 1) L_(32, 1, 1); else if (ks == 2) L_(32, 2, 1); else L_(32, 4, 1); }
        else { if (ks == 1) L_(128, 1, 1); else L_(128, 2, 1); }
#undef L_
        const int rc = fim();
        if (rc) return rc;
    }
    return 0;
}
int jt_entrada_g_bytes() { return (int)sizeof(EntradaG); }

// No reference counterpart: n weight-gradient GEMMs sharing K with the optimizer applied in the epilogue, in launches
// of up to 32 (host array of EntradaGO). Entry i equals jt_gemm(A, EA, B, EB, NULL, NULL, G32, Ge, M, N, K, 1,
// kid + i) followed by jt_momento(G32, Ge, Mm, ME, ...) and jt_peso(Wm, WE, Mm, ME, Rm, RE, k_lr, ef, ...) on the
// [M, N] weight, without storing the gradient.
struct EntradaGO { const void *A, *EA, *B, *EB; void *Mm, *ME, *Wm, *WE, *Rm, *RE; int M, N, K, pad; };
int jt_gemm_otim_lote(const void* entradas, int n, int k_lr, int ef, int kid) {
    using namespace gemm;
    if (n < 0 || (n > 0 && !entradas)) return (int)hipErrorInvalidValue;
    const EntradaGO* e = (const EntradaGO*)entradas;
    for (int base = 0; base < n; base += LOTE_GO) {
        LoteGO L;
        L.n = std::min(LOTE_GO, n - base);
        L.K = e[base].K;
        long long tot = 0;
        for (int i = 0; i < L.n; i++) {
            const EntradaGO& x = e[base + i];
            if (x.M <= 0 || x.N <= 0 || x.K != L.K || x.M % BM || x.N % BN || x.K % g_blk || !k_ok(x.K) || x.K <= 0) return (int)hipErrorInvalidValue;
            if (!alinhados(x.A, x.EA, x.B, x.EB, x.Mm, x.ME, x.Wm, x.WE) || !alinhados(x.Rm, x.RE)) return (int)hipErrorInvalidValue;
            L.A[i] = (const int8_t*)x.A; L.EA[i] = (const int8_t*)x.EA; L.B[i] = (const int8_t*)x.B; L.EB[i] = (const int8_t*)x.EB;
            L.ot[i] = Otim{(int8_t*)x.Mm, (int8_t*)x.ME, (int8_t*)x.Wm, (int8_t*)x.WE, (int8_t*)x.Rm, (int8_t*)x.RE};
            L.M[i] = x.M; L.N[i] = x.N; L.ini[i] = (int)tot;
            tot += (long long)(x.M / BM) * (x.N / BN);
        }
        if (tot > 0x7fffffff) return (int)hipErrorInvalidValue;
        L.ini[L.n] = (int)tot;
        if (tot == 0) continue;
        const int nb = L.K / g_blk;
        int ks = 1;                                                  // mode 5: the epilogue is a fused one, at most 2 splits
        while (ks < 2 && tot * 2 * ks <= g_alvo_wg && nb >= 8 * ks) ks *= 2;
        const size_t lds = gemm_lds(nb, ks, g_blk);
#define L_(BL, S) (lds_max(k_gemm_otim_lote<BL, S>, lds), k_gemm_otim_lote<BL, S><<<(unsigned)tot, 256 * S, lds, g_stream>>>(L, k_lr, ef, kid + base))
        if (g_blk == 32) { if (ks == 1) L_(32, 1); else L_(32, 2); }
        else { if (ks == 1) L_(128, 1); else L_(128, 2); }
#undef L_
        const int r = fim();
        if (r) return r;
    }
    return 0;
}
int jt_entrada_go_bytes() { return (int)sizeof(EntradaGO); }

// ---------------------------------------------------------------------------------------------- element-wise
int jt_quant(const void* acc, const void* e, void* m, void* E, long long nblocos, int kid) {
    if (nblocos <= 0) return 0;
    if (!alinhados(acc, e, m, E)) return (int)hipErrorInvalidValue;
#define C(BL) (k_quant<BL><<<grade_elem(nblocos), 256, 0, g_stream>>>((const int*)acc, (const int16_t*)e, (int8_t*)m, (int8_t*)E, nblocos, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
int jt_soma(const void* xm, const void* xE, const void* ym, const void* yE, void* zm, void* zE, long long nblocos, int kid) {
    if (nblocos <= 0) return 0;
    if (!alinhados(xm, xE, ym, yE, zm, zE)) return (int)hipErrorInvalidValue;
#define C(BL) (k_soma<BL><<<grade_u(nblocos), 256, 0, g_stream>>>((const int8_t*)xm, (const int8_t*)xE, (const int8_t*)ym, (const int8_t*)yE, \
                                                                      (int8_t*)zm, (int8_t*)zE, nblocos, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
int jt_relu2(const void* hm, const void* hE, void* am, void* aE, long long nblocos, int kid) {
    if (nblocos <= 0) return 0;
    if (!alinhados(hm, hE, am, aE)) return (int)hipErrorInvalidValue;
#define C(BL) (k_relu2<BL><<<grade_u(nblocos), 256, 0, g_stream>>>((const int8_t*)hm, (const int8_t*)hE, (int8_t*)am, (int8_t*)aE, nblocos, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
int jt_relu2_back(const void* gm, const void* gE, const void* hm, const void* hE, void* om, void* oE, long long nblocos, int kid) {
    if (nblocos <= 0) return 0;
    if (!alinhados(gm, gE, hm, hE, om, oE)) return (int)hipErrorInvalidValue;
#define C(BL) (k_relu2_back<BL><<<grade_u(nblocos), 256, 0, g_stream>>>((const int8_t*)gm, (const int8_t*)gE, (const int8_t*)hm, \
                                                                            (const int8_t*)hE, (int8_t*)om, (int8_t*)oE, nblocos, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
int jt_momento(const void* gacc, const void* ge, void* Mm, void* ME, long long nblocos, int kid) {
    if (nblocos <= 0) return 0;
    if (!alinhados(gacc, ge, Mm, ME)) return (int)hipErrorInvalidValue;
#define C(BL) (k_momento<BL><<<grade_elem(nblocos), 256, 0, g_stream>>>((const int*)gacc, (const int16_t*)ge, (int8_t*)Mm, (int8_t*)ME, nblocos, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
int jt_peso(void* Wm, void* WE, const void* Mm, const void* ME, void* Rm, void* RE, int k_lr, int ef, long long nblocos, int kid) {
    if (nblocos <= 0) return 0;
    if (!alinhados(Wm, WE, Mm, ME, Rm, RE)) return (int)hipErrorInvalidValue;
#define C(BL) (k_peso<BL><<<grade_u(nblocos), 256, 0, g_stream>>>((int8_t*)Wm, (int8_t*)WE, (const int8_t*)Mm, (const int8_t*)ME, (int8_t*)Rm, \
                                                                      (int8_t*)RE, k_lr, ef, nblocos, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
// No reference counterpart: momento + peso of ntab tensors in one launch (table of TabOtim entries in device
// memory, sorted by `inicio`, nblocos = total blocks). Same results as jt_momento then jt_peso per tensor.
int jt_otimizador(const void* tabela, int ntab, long long nblocos, int k_lr, int ef, int kid) {
    if (nblocos <= 0 || ntab <= 0 || ntab > 256) return nblocos == 0 ? 0 : (int)hipErrorInvalidValue;
    if (!alinhados(tabela)) return (int)hipErrorInvalidValue;
#define C(BL) (k_otimizador<BL><<<grade_u(nblocos), 256, 0, g_stream>>>((const TabOtim*)tabela, ntab, nblocos, k_lr, ef, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
int jt_tab_otim_bytes() { return (int)sizeof(TabOtim); }
// No reference counterpart: jt_otimizador with one workgroup per 32 x 128 tile, which also writes the transposes of
// the new weights (entries with Tm, TE set). BLK 32; every entry M % 32 == 0, N % 128 == 0 (so nblocos % 128 == 0).
int jt_otimizador_t(const void* tabela, int ntab, long long nblocos, int k_lr, int ef, int kid) {
    if (nblocos <= 0 || ntab <= 0 || ntab > 256) return nblocos == 0 ? 0 : (int)hipErrorInvalidValue;
    if (g_blk != 32 || nblocos % 128 || !alinhados(tabela)) return (int)hipErrorInvalidValue;
    k_otimizador_t<<<(unsigned)(nblocos / 128), 256, 0, g_stream>>>((const TabOtim*)tabela, ntab, k_lr, ef, kid);
    return fim();
}
int jt_para16(const void* xm, const void* xE, void* zm, void* zE, long long nblocos, int kid) {
    if (nblocos <= 0) return 0;
    if (!alinhados(xm, xE, zm, zE)) return (int)hipErrorInvalidValue;
#define C(BL) (k_para16<BL><<<grade_elem(nblocos), 256, 0, g_stream>>>((const int8_t*)xm, (const int8_t*)xE, (int16_t*)zm, (int8_t*)zE, nblocos, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
int jt_para8(const void* xm, const void* xE, void* ym, void* yE, long long nblocos, int kid) {
    if (nblocos <= 0) return 0;
    if (!alinhados(xm, xE, ym, yE)) return (int)hipErrorInvalidValue;
#define C(BL) (k_para8<BL><<<grade_elem(nblocos), 256, 0, g_stream>>>((const int16_t*)xm, (const int8_t*)xE, (int8_t*)ym, (int8_t*)yE, nblocos, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
int jt_soma16(const void* xm, const void* xE, const void* ym, const void* yE, void* zm, void* zE, long long nblocos, int kid) {
    if (nblocos <= 0) return 0;
    if (!alinhados(xm, xE, ym, yE, zm, zE)) return (int)hipErrorInvalidValue;
#define C(BL) (k_soma16<BL><<<grade_elem(nblocos), 256, 0, g_stream>>>((const int16_t*)xm, (const int8_t*)xE, (const int8_t*)ym, (const int8_t*)yE, \
                                                                        (int16_t*)zm, (int8_t*)zE, nblocos, kid), 0)
    POR_BLK(C);
#undef C
    return fim();
}
int jt_transpoe(const void* X, const void* EX, void* Y, void* EY, int R, int C, int kid) {
    const int TR = g_blk == 32 ? 64 : 128;
    if (R <= 0 || C <= 0 || R % TR || C % 64 || C % g_blk) return (int)hipErrorInvalidValue;
    if (!alinhados(X, EX, Y, EY)) return (int)hipErrorInvalidValue;
#define L(BL) (k_transpoe<BL, BL == 32 ? 64 : 128><<<dim3(C / 64, R / (BL == 32 ? 64 : 128)), BL == 32 ? 128 : 256, 0, g_stream>>>( \
    (const int8_t*)X, (const int8_t*)EX, (int8_t*)Y, (int8_t*)EY, R, C, kid), 0)
    POR_BLK(L);
#undef L
    return fim();
}
// No reference counterpart: n transposes in launches of up to 64 (host array of EntradaT, device pointers inside).
// Each entry equals jt_transpoe(X, EX, Y, EY, R, C, kid + i).
struct EntradaT { const void* X; const void* EX; void* Y; void* EY; int R; int C; };
// Tiles per workgroup of the batched transpose: 4 from 8192 tiles up (at config 4, 10880 tiles: 48.0 -> 45.4 us;
// each workgroup's later tiles are loaded while the first is converted), else 2, which keeps a smaller launch's
// workgroups at several per CU (4624 tiles: 21.4 us at 2, 24.8 at 4).
constexpr int TPW_T = 2, TPW_T4 = 4, TPW_T4_MIN = 8192;
int jt_transpoe_lote(const void* entradas, int n, int kid) {
    if (n < 0 || (n > 0 && !entradas)) return (int)hipErrorInvalidValue;
    const EntradaT* e = (const EntradaT*)entradas;
    const int TR = 128;                          // 128-row tiles at both BLK: each column's output is a 128-byte line
    for (int base = 0; base < n; base += LOTE_T) {
        LoteT L;
        L.n = std::min(LOTE_T, n - base);
        long long tot = 0;
        for (int i = 0; i < L.n; i++) {
            const EntradaT& x = e[base + i];
            if (x.R <= 0 || x.C <= 0 || x.R % 128 || x.C % 64) return (int)hipErrorInvalidValue;
            if (!alinhados(x.X, x.EX, x.Y, x.EY)) return (int)hipErrorInvalidValue;
            L.X[i] = (const int8_t*)x.X; L.EX[i] = (const int8_t*)x.EX; L.Y[i] = (int8_t*)x.Y; L.EY[i] = (int8_t*)x.EY;
            L.R[i] = x.R; L.C[i] = x.C; L.ini[i] = (int)tot;
            tot += (long long)(x.R / TR) * (x.C / 64);
        }
        if (tot > 0x7fffffff) return (int)hipErrorInvalidValue;
        L.ini[L.n] = (int)tot;
        if (tot == 0) continue;
        if (tot >= TPW_T4_MIN) {
            const unsigned wg = (unsigned)((tot + TPW_T4 - 1) / TPW_T4);
            if (g_blk == 32) k_transpoe_lote<32, 128, TPW_T4><<<wg, 256, 0, g_stream>>>(L, kid + base);
            else k_transpoe_lote<128, 128, TPW_T4><<<wg, 256, 0, g_stream>>>(L, kid + base);
        } else {
            const unsigned wg = (unsigned)((tot + TPW_T - 1) / TPW_T);
            if (g_blk == 32) k_transpoe_lote<32, 128, TPW_T><<<wg, 256, 0, g_stream>>>(L, kid + base);
            else k_transpoe_lote<128, 128, TPW_T><<<wg, 256, 0, g_stream>>>(L, kid + base);
        }
        const int r = fim();
        if (r) return r;
    }
    return 0;
}
int jt_entrada_t_bytes() { return (int)sizeof(EntradaT); }
int jt_embed(const void* Wm, const void* WE, const void* tok, void* Xm, void* XE, int M, int D, int V, int kid) {
    if (M <= 0 || D % g_blk || D % 16) return (int)hipErrorInvalidValue;
    if (!alinhados(Wm, WE, tok, Xm, XE)) return (int)hipErrorInvalidValue;
    const unsigned g = (unsigned)(((long long)M * (D / 16) + 255) / 256);
#define L(BL) (k_embed<BL><<<g, 256, 0, g_stream>>>((const int8_t*)Wm, (const int8_t*)WE, (const int*)tok, (int8_t*)Xm, (int8_t*)XE, M, D, V, kid), 0)
    POR_BLK(L);
#undef L
    return fim();
}
int jt_janelas(const void* corpus, long long n, const void* ini, void* tok, void* alvo, int Bt, int T, int kid) {
    if (Bt <= 0 || T <= 0 || n < (long long)T + 1 || !corpus || !ini || !tok || !alvo) return (int)hipErrorInvalidValue;
    if (((uintptr_t)ini & 7) || ((uintptr_t)tok & 3) || ((uintptr_t)alvo & 3)) return (int)hipErrorInvalidValue;
    const unsigned g = (unsigned)(((long long)Bt * T + 255) / 256);
    k_janelas<<<g, 256, 0, g_stream>>>((const uint8_t*)corpus, n, (const long long*)ini, (int*)tok, (int*)alvo, Bt, T, kid);
    return fim();
}
int jt_um_quente(const void* tok, void* U, void* UE, int M, int V, int kid) {
    if (M <= 0 || V % g_blk || V % 16) return (int)hipErrorInvalidValue;
    if (!alinhados(tok, U, UE)) return (int)hipErrorInvalidValue;
    const unsigned g = (unsigned)(((long long)M * (V / 16) + 255) / 256);
#define L(BL) (k_um_quente<BL><<<g, 256, 0, g_stream>>>((const int*)tok, (int8_t*)U, (int8_t*)UE, M, V, kid), 0)
    POR_BLK(L);
#undef L
    return fim();
}

// ---------------------------------------------------------------------------------------------- rows
// One row per LP lanes with VP values each. The widths 128, 256, 512 and 1024 have layouts of their own; any other
// multiple of BLK up to 1024 (the reference's domain: ops.py:453 for rms, ops.py:496 for softmax_ce) runs with 16
// values per lane on the next power of two of lanes, the lanes past the row idle (CH = false).
}  // extern "C"
template <int VP_, int LP_, bool CH_>
struct FormaLinha { static constexpr int VP = VP_, LP = LP_; static constexpr bool CH = CH_; };
// Calls f(FormaLinha<...>{}, integral_constant BLK) for the layout of a row of `len` values; false if len is not
// a multiple of BLK in (0, 1024].
template <class F>
static bool por_linha(int len, F&& f) {
    if (len <= 0 || len > 1024 || len % g_blk) return false;
    auto blk = [&](auto fm) {
        using FM = decltype(fm);
        if (g_blk == 32) f(fm, std::integral_constant<int, 32>{});
        else if constexpr (128 / FM::VP <= FM::LP) f(fm, std::integral_constant<int, 128>{});   // a block in LP lanes
    };
    switch (len) {
        case 128: blk(FormaLinha<4, 32, true>{}); return true;
        case 256: blk(FormaLinha<4, 64, true>{}); return true;
        case 512: blk(FormaLinha<16, 32, true>{}); return true;
        case 1024: blk(FormaLinha<16, 64, true>{}); return true;
    }
    int l = std::max(2, g_blk / 16);
    while (l * 16 < len) l *= 2;
    switch (l) {
        case 2: blk(FormaLinha<16, 2, false>{}); break;
        case 4: blk(FormaLinha<16, 4, false>{}); break;
        case 8: blk(FormaLinha<16, 8, false>{}); break;
        case 16: blk(FormaLinha<16, 16, false>{}); break;
        case 32: blk(FormaLinha<16, 32, false>{}); break;
        default: blk(FormaLinha<16, 64, false>{}); break;
    }
    return true;
}
static unsigned grade_linhas(int M, int LP) { return (unsigned)((M + 256 / LP - 1) / (256 / LP)); }
extern "C" {

int jt_rms(const void* Xm, const void* XE, void* Ym, void* YE, void* cr, void* cemax, int M, int D, int log2D, int G, int kid) {
    if (M <= 0) return (int)hipErrorInvalidValue;
    if (!alinhados(Xm, XE, Ym, YE, cr, cemax)) return (int)hipErrorInvalidValue;
    const bool ok = por_linha(D, [&](auto fm, auto bl) {
        using FM = decltype(fm);
        k_rms<FM::VP, FM::LP, decltype(bl)::value, FM::CH><<<grade_linhas(M, FM::LP), 256, 0, g_stream>>>(
            (const int8_t*)Xm, (const int8_t*)XE, (int8_t*)Ym, (int8_t*)YE, (int*)cr, (int*)cemax, M, log2D, G, kid, D);
    });
    return ok ? fim() : (int)hipErrorInvalidValue;
}
int jt_rms_back(const void* gm, const void* gE, const void* ym, const void* yE, const void* cr, const void* cemax, void* om, void* oE, int M,
                int D, int log2D, int G, int GB, int kid) {
    if (M <= 0) return (int)hipErrorInvalidValue;
    if (!alinhados(gm, gE, ym, yE, cr, cemax, om, oE)) return (int)hipErrorInvalidValue;
    const bool ok = por_linha(D, [&](auto fm, auto bl) {
        using FM = decltype(fm);
        k_rms_back<FM::VP, FM::LP, decltype(bl)::value, 0, FM::CH><<<grade_linhas(M, FM::LP), 256, 0, g_stream>>>(
            (const int8_t*)gm, (const int8_t*)gE, (const int8_t*)ym, (const int8_t*)yE, (const int*)cr, (const int*)cemax, (int8_t*)om,
            (int8_t*)oE, M, log2D, G, GB, kid, nullptr, nullptr, 0, D);
    });
    return ok ? fim() : (int)hipErrorInvalidValue;
}
// No reference counterpart: soma(x, rms_back(g, y, cache)) in one launch (the backward's residual update); equals
// jt_rms_back into a temporary then jt_soma(x, temporary). Launch ids: kid for the rms_back part, kid + 1 for soma.
int jt_rms_back_soma(const void* gm, const void* gE, const void* ym, const void* yE, const void* cr, const void* cemax, const void* xm,
                     const void* xE, void* om, void* oE, int M, int D, int log2D, int G, int GB, int kid) {
    if (M <= 0) return (int)hipErrorInvalidValue;
    if (!alinhados(gm, gE, ym, yE, cr, cemax, om, oE) || !alinhados(xm, xE)) return (int)hipErrorInvalidValue;
    const bool ok = por_linha(D, [&](auto fm, auto bl) {
        using FM = decltype(fm);
        k_rms_back<FM::VP, FM::LP, decltype(bl)::value, 1, FM::CH><<<grade_linhas(M, FM::LP), 256, 0, g_stream>>>(
            (const int8_t*)gm, (const int8_t*)gE, (const int8_t*)ym, (const int8_t*)yE, (const int*)cr, (const int*)cemax, (int8_t*)om,
            (int8_t*)oE, M, log2D, G, GB, kid, (const int8_t*)xm, (const int8_t*)xE, kid + 1, D);
    });
    return ok ? fim() : (int)hipErrorInvalidValue;
}
// No reference counterpart: z16 = soma16(x16, rms_back(g, y, cache)) and y8 = para8(z16) in one launch (the
// backward's update of the 16-bit residual stream, modelo.py:114-130, and the INT8 copy the next GEMMs read);
// equals jt_rms_back, jt_soma16 and jt_para8 in turn (launch ids kid, kid + 1, kid + 2). x16, z16 int16 [M, D];
// xE, zE, yE8 int8 [M, D / BLK]; y8 int8 [M, D].
int jt_rms_back_soma16(const void* gm, const void* gE, const void* ym, const void* yE, const void* cr, const void* cemax, const void* x16,
                       const void* xE, void* z16, void* zE, void* y8, void* yE8, int M, int D, int log2D, int G, int GB, int kid) {
    if (M <= 0 || !x16 || !xE || !z16 || !zE || !y8 || !yE8) return (int)hipErrorInvalidValue;
    if (!alinhados(gm, gE, ym, yE, cr, cemax, z16, zE) || !alinhados(x16, xE, y8, yE8)) return (int)hipErrorInvalidValue;
    const bool ok = por_linha(D, [&](auto fm, auto bl) {
        using FM = decltype(fm);
        k_rms_back<FM::VP, FM::LP, decltype(bl)::value, 2, FM::CH><<<grade_linhas(M, FM::LP), 256, 0, g_stream>>>(
            (const int8_t*)gm, (const int8_t*)gE, (const int8_t*)ym, (const int8_t*)yE, (const int*)cr, (const int*)cemax, (int8_t*)z16,
            (int8_t*)zE, M, log2D, G, GB, kid, (const int8_t*)x16, (const int8_t*)xE, kid + 1, D, (int8_t*)y8, (int8_t*)yE8);
    });
    return ok ? fim() : (int)hipErrorInvalidValue;
}
int jt_softmax_ce(const void* acc, const void* e, const void* alvo, void* gm, void* gE, void* d_alvo, void* soma, int M, int V, int log2M,
                  int kid) {
    if (M <= 0 || V % 128) return (int)hipErrorInvalidValue;
    if (!alinhados(acc, e, alvo, gm, gE, d_alvo, soma)) return (int)hipErrorInvalidValue;
    const bool ok = por_linha(V, [&](auto fm, auto bl) {
        using FM = decltype(fm);
        k_softmax_ce<FM::VP, FM::LP, decltype(bl)::value, FM::CH><<<grade_linhas(M, FM::LP), 256, 0, g_stream>>>(
            (const int*)acc, (const int16_t*)e, (const int*)alvo, (int8_t*)gm, (int8_t*)gE, (int*)d_alvo, (int*)soma, M, log2M, kid, V);
    });
    return ok ? fim() : (int)hipErrorInvalidValue;
}

// No reference counterpart: the loss mean(d / 256 + ln(s / 4096)) (modelo.py:93) into one float64, one launch.
int jt_perda(const void* d_alvo, const void* soma, void* out, int M, int kid) {
    (void)kid;
    if (M <= 0 || !d_alvo || !soma || !out || !alinhados(d_alvo, soma, out)) return (int)hipErrorInvalidValue;
    k_perda<<<1, 1024, 0, g_stream>>>((const int*)d_alvo, (const int*)soma, (double*)out, M);
    return fim();
}

// ---------------------------------------------------------------------------------------------- attention
// Shapes: head width 4 (the reference's, jatai_cuda.cu:1176-1187 with ops.py:475) takes T a multiple of 32 up to
// 256 and H <= 64 (the ALiBi schedule 8 - h // 8 of ops.py:208); head widths 16, 32, 64 (no reference
// counterpart) take T a multiple of 64 up to 512. GA, the guard bits of the aligned values, is the spec's 4
// (ops.py:20) or less: every bound the kernels rest on assumes |aligned value| <= 127 << 4 = 2032 (int32 sums,
// exact f16 values, the 24-bit products, the dS width), as the reference's own int32 bounds do at T <= 128.
static bool atencao_forma(int Bt, int T, int H, int D, int GA) {
    if (Bt <= 0 || H <= 0 || T <= 0 || D % H || GA < 0 || GA > 4) return false;
    if (D / H == 4) return T % 32 == 0 && T <= 256 && H <= 64;
    return T % 64 == 0 && T <= 512;
}
int jt_atencao(const void* qm, const void* qE, void* Oacc, void* Oe, void* P, int Bt, int T, int H, int D, int GA, int kid) {
    if (!atencao_forma(Bt, T, H, D, GA)) return (int)hipErrorInvalidValue;
    if (!alinhados(qm, qE, Oacc, Oe, P)) return (int)hipErrorInvalidValue;
    const int hd = D / H;
    if (hd == 4) {
        if (g_linhas == 0 && T <= 128) {                 // automatic: 8 lanes per query row
            k_atencao4l<128, 8><<<Bt * H, 1024, 0, g_stream>>>((const int8_t*)qm, (const int8_t*)qE, (int*)Oacc, (int16_t*)Oe, (uint8_t*)P,
                                                              T, H, D, g_blk, GA, kid);
            return fim();
        }
        const int nl = g_linhas == 2 ? 2 : 1;
        const int nt = (T / nl + 63) & ~63;              // whole waves; threads without a row only join the reductions
#define A4(TM, NR) k_atencao4<TM, NR><<<Bt * H, nt, 0, g_stream>>>((const int8_t*)qm, (const int8_t*)qE, (int*)Oacc, (int16_t*)Oe, \
                                                                    (uint8_t*)P, T, H, D, g_blk, GA, kid)
        if (T <= 128) { if (nl == 2) A4(128, 2); else A4(128, 1); }
        else { if (nl == 2) A4(256, 2); else A4(256, 1); }
#undef A4
        return fim();
    }
    if ((hd != 16 && hd != 32 && hd != 64) || hd % g_blk && g_blk % hd) return (int)hipErrorInvalidValue;
    const unsigned g = (unsigned)(Bt * H * (T / hd::QB));
    if (hd == 64 && g_atencao_mfma) {                // matrix-core forward (scores kept in registers: T <= 256)
        const size_t Tk = (size_t)T, lds_mf = Tk * 64 + ((Tk * 2 + 15) & ~(size_t)15) + 64 * Tk * 2 + 4 * 16 * Tk * 2;
        if (T <= 256) {
            lds_max(k_atencao_mf<256>, lds_mf);
            k_atencao_mf<256><<<g, 256, lds_mf, g_stream>>>((const int8_t*)qm, (const int8_t*)qE, (int*)Oacc, (int16_t*)Oe, (uint8_t*)P,
                                                            T, H, D, g_blk, GA, kid);
            return fim();
        }
    }
    const size_t lds = (size_t)T * hd * 4;
#define L(HD) (lds_max(k_atencao_hd<HD>, lds), k_atencao_hd<HD><<<g, hd::NT, lds, g_stream>>>((const int8_t*)qm, (const int8_t*)qE, \
              (int*)Oacc, (int16_t*)Oe, (uint8_t*)P, T, H, D, g_blk, GA, kid))
    if (hd == 16) L(16); else if (hd == 32) L(32); else L(64);
#undef L
    return fim();
}
// No reference counterpart: jt_atencao with a caller workspace of jt_atencao_ws_bytes(Bt, T, H, D) bytes
// (16-byte aligned). Same outputs as jt_atencao. At head width 64 on matrix cores (T % 64 == 0, T <= 512) it
// converts k and v once per (sequence, head) into the workspace and splits each 16-row query tile's keys over
// four waves; otherwise it runs jt_atencao and leaves the workspace untouched.
long long jt_atencao_ws_bytes(int Bt, int T, int H, int D) {
    if (Bt <= 0 || H <= 0 || T <= 0 || D % H) return 0;
    return (long long)atw::bytes_fwd((long long)Bt * H, T);
}
// salvo (optional): the backward's conversions of q, k, v are written there too (atw::Salvo)
static int atencao_ws(const void* qm, const void* qE, void* O1, void* O2, void* P, int Bt, int T, int H, int D, int GA, void* ws, long long ws_bytes,
                      bool bloco, int kid, void* salvo = nullptr) {
    if (!alinhados(qm, qE, O1, O2, P, ws, salvo) || !ws || ws_bytes < jt_atencao_ws_bytes(Bt, T, H, D) || 64 % g_blk && g_blk % 64)
        return (int)hipErrorInvalidValue;
    const long long BH = (long long)Bt * H;
    const atw::Ws w = atw::parte(ws, BH, T);
    if (salvo) k_atf_prep<true><<<(unsigned)(BH * (T / 64)), 256, 0, g_stream>>>((const int8_t*)qm, (const int8_t*)qE, w, atw::parte_s(salvo, BH, T),
                                                                                  T, H, D, g_blk, GA);
    else k_atf_prep<false><<<(unsigned)(BH * (T / 64)), 256, 0, g_stream>>>((const int8_t*)qm, (const int8_t*)qE, w, atw::Salvo{}, T, H, D, g_blk, GA);
    const unsigned g = (unsigned)(BH * (T / 16));
#define L(NTW, B) k_atf<NTW, B><<<g, 256, 0, g_stream>>>((const int8_t*)qm, (const int8_t*)qE, w, O1, O2, (uint8_t*)P, T, H, D, g_blk, GA, kid)
    if (bloco) { if (T <= 256) L(4, true); else L(8, true); }
    else { if (T <= 256) L(4, false); else L(8, false); }
#undef L
    return fim();
}
int jt_atencao_ws(const void* qm, const void* qE, void* Oacc, void* Oe, void* P, int Bt, int T, int H, int D, int GA, void* ws,
                  long long ws_bytes, int kid) {
    if (!atencao_forma(Bt, T, H, D, GA)) return (int)hipErrorInvalidValue;
    if (D / H != 64 || !g_atencao_mfma || T > 512) return jt_atencao(qm, qE, Oacc, Oe, P, Bt, T, H, D, GA, kid);
    return atencao_ws(qm, qE, Oacc, Oe, P, Bt, T, H, D, GA, ws, ws_bytes, false, kid);
}
// No reference counterpart: jt_atencao_ws writing the output quantized to block format (Om int8 [M, D], OE int8
// [M, D/32]), equal to jt_quant of the raw output. Head width 64 on matrix cores at BLK = 32 only (a block is then
// half a head); hipErrorNotSupported otherwise.
int jt_atencao_ws_q(const void* qm, const void* qE, void* Om, void* OE, void* P, int Bt, int T, int H, int D, int GA, void* ws,
                    long long ws_bytes, int kid) {
    if (!atencao_forma(Bt, T, H, D, GA) || T % 64) return (int)hipErrorInvalidValue;
    if (D / H != 64 || !g_atencao_mfma || T > 512 || g_blk != 32) return (int)hipErrorNotSupported;
    return atencao_ws(qm, qE, Om, OE, P, Bt, T, H, D, GA, ws, ws_bytes, true, kid);
}
// No reference counterpart: bytes of the buffer in which jt_atencao_ws_qs saves the backward's conversions of q, k, v
// for jt_atencao_back_ws_qs (0 for an invalid shape).
long long jt_atencao_salvo_bytes(int Bt, int T, int H, int D) {
    if (Bt <= 0 || H <= 0 || T <= 0 || D % H) return 0;
    return (long long)atw::bytes_salvo((long long)Bt * H, T);
}
// No reference counterpart: jt_atencao_ws_q that also writes into salvo (jt_atencao_salvo_bytes bytes, 16-byte
// aligned) the conversions of q, k, v that the backward of the same qkv reads (jt_atencao_back_ws_qs), from the pass
// that converts k and v for the forward anyway. Same outputs as jt_atencao_ws_q.
int jt_atencao_ws_qs(const void* qm, const void* qE, void* Om, void* OE, void* P, int Bt, int T, int H, int D, int GA, void* ws,
                     long long ws_bytes, void* salvo, long long salvo_bytes, int kid) {
    if (!atencao_forma(Bt, T, H, D, GA) || T % 64) return (int)hipErrorInvalidValue;
    if (D / H != 64 || !g_atencao_mfma || T > 512 || g_blk != 32) return (int)hipErrorNotSupported;
    if (!salvo || salvo_bytes < jt_atencao_salvo_bytes(Bt, T, H, D)) return (int)hipErrorInvalidValue;
    return atencao_ws(qm, qE, Om, OE, P, Bt, T, H, D, GA, ws, ws_bytes, true, kid, salvo);
}
int jt_atencao_back(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gacc, void* Ge, int Bt, int T, int H,
                    int D, int GA, int limite, int kid) {
    if (!atencao_forma(Bt, T, H, D, GA)) return (int)hipErrorInvalidValue;
    if (!alinhados(gom, goE, qm, qE, P, Gacc, Ge)) return (int)hipErrorInvalidValue;
    const int hd = D / H;
    const int dsb = ds_bits(T);
    if (hd == 4) {
#define ARGS (const int8_t*)gom, (const int8_t*)goE, (const int8_t*)qm, (const int8_t*)qE, (const uint8_t*)P, (int*)Gacc, (int16_t*)Ge, T, H, D, g_blk, GA, dsb, kid
        if (g_linhas == 0 && T <= 128) {                 // automatic: 8 lanes per query row
            if (limite) k_atencao4l_back<128, 1, 8><<<Bt * H, 1024, 0, g_stream>>>(ARGS);
            else k_atencao4l_back<128, 0, 8><<<Bt * H, 1024, 0, g_stream>>>(ARGS);
            return fim();
        }
        const int nl = g_linhas == 2 ? 2 : 1;
        const int nt = (T / nl + 63) & ~63;
#define B4(TM, LM) { if (nl == 2) k_atencao4_back<TM, LM, 2><<<Bt * H, nt, 0, g_stream>>>(ARGS); \
                     else k_atencao4_back<TM, LM, 1><<<Bt * H, nt, 0, g_stream>>>(ARGS); }
        if (T <= 128) { if (limite) B4(128, 1) else B4(128, 0) }
        else { if (limite) B4(256, 1) else B4(256, 0) }
#undef B4
#undef ARGS
        return fim();
    }
    if ((hd != 16 && hd != 32 && hd != 64) || hd % g_blk && g_blk % hd) return (int)hipErrorInvalidValue;
    const unsigned g = (unsigned)(Bt * H * (T / hd::QB));
    if (hd == 64 && g_atencao_mfma && T <= 256) {        // matrix-core backward: 5 launches
        const int8_t *go8 = (const int8_t*)gom, *goE8 = (const int8_t*)goE, *q8 = (const int8_t*)qm, *qE8 = (const int8_t*)qE;
        const uint8_t* P8 = (const uint8_t*)P;
        int16_t* Ge16 = (int16_t*)Ge;
        int* G32 = (int*)Gacc;
        const size_t n = (size_t)T, pad = (n * 2 + 15) & ~(size_t)15;
        const size_t l_lin = n * 64 + pad, l_gq = n * 64 + pad + 64 * n * 2 + 4 * 16 * n * 2;
        const size_t l_gkv = n * 64 + pad + 2 * 64 * n * 2 + 4 * 16 * n * 2 + 4 * 16 * n + n * 4;
        const size_t lds1 = (size_t)T * hd * 2;
#define MF(LM)                                                                                                              \
        {                                                                                                                   \
            if (LM) k_atb_max1<64, 1><<<g, hd::NT, lds1, g_stream>>>(go8, goE8, q8, qE8, Ge16, T, H, D, g_blk, GA);         \
            else k_atb_mf_linhas<256, 1, 0><<<g, 256, l_lin, g_stream>>>(go8, goE8, q8, qE8, P8, Ge16, T, H, D, g_blk, GA, kid); \
            k_atb_mf_linhas<256, 2, LM><<<g, 256, l_lin, g_stream>>>(go8, goE8, q8, qE8, P8, Ge16, T, H, D, g_blk, GA, kid);  \
            lds_max(k_atb_mf_gq<256, LM>, l_gq);                                                                            \
            k_atb_mf_gq<256, LM><<<g, 256, l_gq, g_stream>>>(go8, goE8, q8, qE8, P8, G32, Ge16, T, H, D, g_blk, GA, dsb, kid); \
            lds_max(k_atb_mf_gkv<256, LM>, l_gkv);                                                                          \
            k_atb_mf_gkv<256, LM><<<g, 256, l_gkv, g_stream>>>(go8, goE8, q8, qE8, P8, G32, Ge16, T, H, D, g_blk, GA, dsb, kid); \
            k_atb_exp<64, LM><<<Bt * H, hd::NT, 0, g_stream>>>(goE8, qE8, Ge16, T, H, D, g_blk, GA, dsb);                  \
        }
        if (limite) MF(1) else MF(0)
#undef MF
        return fim();
    }
    const size_t lds1 = (size_t)T * hd * 2, lds3 = (size_t)(2 * T + 2 * hd::QB) * hd * 2 + (size_t)T * 4;
    const int8_t *go8 = (const int8_t*)gom, *goE8 = (const int8_t*)goE, *q8 = (const int8_t*)qm, *qE8 = (const int8_t*)qE;
    const uint8_t* P8 = (const uint8_t*)P;
    int16_t* Ge16 = (int16_t*)Ge;
#define FASES(HD, LM)                                                                                                      \
    {                                                                                                                      \
        k_atb_max1<HD, LM><<<g, hd::NT, lds1, g_stream>>>(go8, goE8, q8, qE8, Ge16, T, H, D, g_blk, GA);                   \
        k_atb_slin<HD, LM><<<g, hd::NT, lds1, g_stream>>>(go8, goE8, q8, qE8, P8, Ge16, T, H, D, g_blk, GA, kid);          \
        lds_max(k_atb_grad<HD, LM>, lds3);                                                                                 \
        k_atb_grad<HD, LM><<<g, hd::NT, lds3, g_stream>>>(go8, goE8, q8, qE8, P8, (int*)Gacc, Ge16, T, H, D, g_blk, GA, dsb, kid); \
        k_atb_exp<HD, LM><<<Bt * H, hd::NT, 0, g_stream>>>(goE8, qE8, Ge16, T, H, D, g_blk, GA, dsb);                       \
    }
#define LIM_(HD) { if (limite) FASES(HD, 1) else FASES(HD, 0) }
    if (hd == 16) LIM_(16) else if (hd == 32) LIM_(32) else LIM_(64)
#undef LIM_
#undef FASES
    return fim();
}

// No reference counterpart: jt_atencao_back with a caller workspace of jt_atencao_back_ws_bytes(Bt, T, H, D)
// bytes (16-byte aligned). Same outputs as jt_atencao_back. At head width 64 on matrix cores (T % 64 == 0,
// T <= 512) it converts dO, q, k, v once per (sequence, head) into the workspace and splits each 16-row tile's
// partner tiles over four waves (4 launches; the exact variant's per-tile max |gP| in the conversion launch at
// T <= 256, a launch of its own past that or when the forward saved the q, k, v conversions); otherwise it runs
// jt_atencao_back.
long long jt_atencao_back_ws_bytes(int Bt, int T, int H, int D) {
    if (Bt <= 0 || H <= 0 || T <= 0 || D % H) return 0;
    return (long long)atw::bytes_back((long long)Bt * H, T);
}
// salvo (optional, exact variant): the conversions of q, k, v saved by jt_atencao_ws_qs for the same qkv
static int atencao_back_ws(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* G1, void* G2, int Bt, int T,
                           int H, int D, int GA, int limite, void* ws, long long ws_bytes, bool bloco, int kid, const void* salvo = nullptr) {
    if (!alinhados(gom, goE, qm, qE, P, G1, G2, ws, salvo) || !ws || ws_bytes < jt_atencao_back_ws_bytes(Bt, T, H, D) || 64 % g_blk && g_blk % 64)
        return (int)hipErrorInvalidValue;
    const long long BH = (long long)Bt * H;
    atw::WsB w = atw::parte_b(ws, BH, T);
    const int* smx = nullptr;
    if (salvo && !limite) {                              // q, k, v read from the saved conversions
        const atw::Salvo s = atw::parte_s(const_cast<void*>(salvo), BH, T);
        w.vm8 = s.vm8; w.vL = s.vL; w.kt = s.kt; w.qt = s.qt;
        smx = s.mx;
    }
    const int dsb = ds_bits(T);
    const int8_t *go8 = (const int8_t*)gom, *goE8 = (const int8_t*)goE, *q8 = (const int8_t*)qm, *qE8 = (const int8_t*)qE;
    const uint8_t* P8 = (const uint8_t*)P;
    const unsigned gp = (unsigned)(BH * (T / 64)), gt = (unsigned)(BH * (T / 16));
#define FASES(NTW, LM, B)                                                                                                 \
    {                                                                                                                     \
        if (!LM && smx) k_atb_prep_s<<<gp, 256, 0, g_stream>>>(go8, goE8, w, smx, T, H, D, g_blk, GA);                     \
        else if (!LM && T <= 256) k_atb_prep<0, true><<<2 * gp, 256, 0, g_stream>>>(go8, goE8, q8, qE8, w, T, H, D, g_blk, GA); \
        else k_atb_prep<LM><<<gp, 256, 0, g_stream>>>(go8, goE8, q8, qE8, w, T, H, D, g_blk, GA);                         \
        if (!LM && (smx || T > 256)) k_atb1<NTW><<<gt, 256, 0, g_stream>>>(w, T, H);                                      \
        k_atb2<NTW, LM><<<gt, 256, 0, g_stream>>>(w, P8, T, H, D, kid);                                                    \
        k_atbqkv<NTW, LM, B><<<2 * gt, 256, 0, g_stream>>>(w, P8, (int*)G1, (int16_t*)G2, T, H, D, dsb, kid);              \
    }
#define VAR(B) { if (T <= 256) { if (limite) FASES(4, 1, B) else FASES(4, 0, B) } else { if (limite) FASES(8, 1, B) else FASES(8, 0, B) } }
    if (bloco) VAR(true) else VAR(false)
#undef VAR
#undef FASES
    return fim();
}
int jt_atencao_back_ws(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gacc, void* Ge, int Bt, int T,
                       int H, int D, int GA, int limite, void* ws, long long ws_bytes, int kid) {
    if (!atencao_forma(Bt, T, H, D, GA)) return (int)hipErrorInvalidValue;
    if (D / H != 64 || !g_atencao_mfma || T > 512) return jt_atencao_back(gom, goE, qm, qE, P, Gacc, Ge, Bt, T, H, D, GA, limite, kid);
    return atencao_back_ws(gom, goE, qm, qE, P, Gacc, Ge, Bt, T, H, D, GA, limite, ws, ws_bytes, false, kid);
}
// No reference counterpart: jt_atencao_back_ws without a workspace argument and without any allocation, for callers
// that cannot allocate (code under graph capture, serving loops, harnesses that forbid hipMalloc). The workspace is
// the file-scope device array `scratch` (SCRATCH_BYTES, held by every GPU the library runs on until the process
// ends); a call needing more (jt_atencao_back_ws_bytes > SCRATCH_BYTES) returns hipErrorOutOfMemory and launches
// nothing. Nothing in the workspace has to start at zero (every slot a kernel reads was written earlier in the
// same call), so the array needs no clearing. Calls that overlap on one GPU (two streams, two host threads) share
// the array and race.
constexpr size_t SCRATCH_BYTES = (size_t)32 << 20;       // config 4's backward needs 25 MB
static __device__ __align__(256) char scratch[SCRATCH_BYTES];
}  // extern "C"
// the device address of `scratch` on each device, looked up once per device with that device current (each GPU
// holds its own copy of the array; the array's name in host code is not a device address)
static void* scratch_por_device[64];
static hipError_t scratch_do_device(void** p) {
    int dev = 0;
    hipError_t c = hipGetDevice(&dev);
    if (c != hipSuccess) return c;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!scratch_por_device[dev]) {
        void* q = nullptr;
        c = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
        if (c != hipSuccess) return c;
        scratch_por_device[dev] = q;
    }
    *p = scratch_por_device[dev];
    return hipSuccess;
}
extern "C" {
long long jt_scratch_bytes() { return (long long)SCRATCH_BYTES; }
int jt_atencao_back_sem_alocar(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gacc, void* Ge, int Bt,
                               int T, int H, int D, int GA, int limite, int kid) {
    if (!atencao_forma(Bt, T, H, D, GA)) return (int)hipErrorInvalidValue;
    if (D / H != 64 || !g_atencao_mfma) return jt_atencao_back(gom, goE, qm, qE, P, Gacc, Ge, Bt, T, H, D, GA, limite, kid);
    const long long n = jt_atencao_back_ws_bytes(Bt, T, H, D);
    if (n <= 0 || n > (long long)SCRATCH_BYTES) return (int)hipErrorOutOfMemory;
    void* ws = nullptr;
    const hipError_t c = scratch_do_device(&ws);
    if (c != hipSuccess) return (int)c;
    return atencao_back_ws(gom, goE, qm, qE, P, Gacc, Ge, Bt, T, H, D, GA, limite, ws, n, false, kid);
}
// No reference counterpart: jt_atencao_back_ws writing the gradient quantized to block format (Gm int8 [M, 3D],
// GE int8 [M, 3D/32]), equal to jt_quant of the raw gradient. Head width 64 on matrix cores at BLK = 32 only;
// hipErrorNotSupported otherwise.
int jt_atencao_back_ws_q(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gm, void* GE, int Bt, int T,
                         int H, int D, int GA, int limite, void* ws, long long ws_bytes, int kid) {
    if (!atencao_forma(Bt, T, H, D, GA) || T % 64) return (int)hipErrorInvalidValue;
    if (D / H != 64 || !g_atencao_mfma || T > 512 || g_blk != 32) return (int)hipErrorNotSupported;
    return atencao_back_ws(gom, goE, qm, qE, P, Gm, GE, Bt, T, H, D, GA, limite, ws, ws_bytes, true, kid);
}
// No reference counterpart: jt_atencao_back_ws_q reading the conversions of q, k, v that jt_atencao_ws_qs saved in
// salvo for this qkv (the caller keeps salvo and qkv unchanged in between), so that only dO is converted. The bound
// variant (limite = 1) also needs per-64-token norms of v, which the forward does not save: it converts q, k, v
// itself and leaves salvo unread. Same outputs as jt_atencao_back_ws_q.
int jt_atencao_back_ws_qs(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gm, void* GE, int Bt, int T,
                          int H, int D, int GA, int limite, void* ws, long long ws_bytes, const void* salvo, long long salvo_bytes, int kid) {
    if (!atencao_forma(Bt, T, H, D, GA) || T % 64) return (int)hipErrorInvalidValue;
    if (D / H != 64 || !g_atencao_mfma || T > 512 || g_blk != 32) return (int)hipErrorNotSupported;
    if (!salvo || salvo_bytes < jt_atencao_salvo_bytes(Bt, T, H, D)) return (int)hipErrorInvalidValue;
    return atencao_back_ws(gom, goE, qm, qE, P, Gm, GE, Bt, T, H, D, GA, limite, ws, ws_bytes, true, kid, salvo);
}

}  // extern "C"
