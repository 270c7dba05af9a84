/* libjatai.so -- C ABI of the Jatai INT8 training hot path on MI355X (gfx950).
 *
 * Drop-in for the reference library's C interface (jatai_cuda/jatai_cuda.cu:1061-1201), bound from Python by
 * ctypes exactly as the reference binds libjatai.so (jatai_cuda/ops.py:297-310). Conventions, as in the reference:
 *   - the caller allocates every output; the library never allocates device memory;
 *   - pointers are raw device addresses; an absent operand is NULL;
 *   - block tensors are (int8 mantissas [R, C], int8 exponents [R, C/BLK]); raw tensors (int32 acc [R, C],
 *     int16 exponents [R, C]); R16 tensors (int16 mantissas [R, C], int8 exponents [R, C/BLK]);
 *   - element counts are long long; every launch takes a trailing launch id `kid`, recorded by device sentinels;
 *   - the return value is a hipError_t code (0 = success); launches are asynchronous on the stream set by
 *     jt_stream (NULL = default stream);
 *   - module state (stream, block size, knobs) is global: not thread-safe, one host thread drives the library.
 * BLK (32 or 128) is chosen with jt_bloco; the reference fixes BLK = 128 (jatai_cuda.cu:16).
 */
#ifndef JATAI_H
#define JATAI_H
#ifdef __cplusplus
extern "C" {
#endif

/* ---- device error record and stream (jatai_cuda.cu:1062-1073, 1088) */
int jt_erro_le(long long* out);        /* jatai_cuda.cu:1062: out[6] = {n, code, kid, idx, value, aux}; returns n, or -hipError; synchronizes the device first (the first call on a device also allocates a 4-byte host-pinned event flag, kept to the process's end) */
int jt_erro_limpa(void);               /* jatai_cuda.cu:1069: clears the record, ordered on the library's stream (no host wait) */
int jt_sincroniza(void);               /* hipDeviceSynchronize */
void jt_stream(void* stream);          /* every later launch goes to this hipStream_t (graph capture) */

/* ---- tuning knobs (jatai_cuda.cu:1087-1091) */
void jt_gemm_split(int alvo_wg);       /* split-K target workgroup count for raw GEMM outputs */
void jt_gemm_bm(int bm);               /* jatai_cuda.cu:1090: GEMM tile rows: 0 automatic (32), 64 or 128 forced (32 forces the
                                        * default); a forced tile that does not divide M falls back to one that does; same bits */
void jt_atencao_linhas(int n);         /* jatai_cuda.cu:1091: query rows per thread of the head-width-4 attention: 1 or 2 (rows
                                        * i and T - 1 - i); any other value (0, the default) is automatic: 8 lanes per query row
                                        * up to T = 128, one row per thread beyond; same bits */
int jt_res_estocastico(int ligado);    /* jatai_cuda.cu:1087: 1 = gemm_soma's residual add rounds stochastically (0 = off, the default) */

/* ---- no reference counterpart: attention kernel family at head width 64, matrix cores (1, default) or dot2 (0) */
void jt_atencao_mfma(int ligado);

/* ---- block size: no reference counterpart (the reference fixes 128) */
int jt_bloco(int blk);                 /* 32 or 128; hipErrorInvalidValue otherwise */
int jt_bloco_atual(void);

/* ---- GEMM C = A . B^T, A [M,K], B [N,K] blocked along K (jatai_cuda.cu:1093-1127)
 * modo 0: block C (Cm, CE) | 1: raw C (C32, Ce), split-K over K-blocks | 2: Cm = soma(X, A.B^T)
 * 3: Cm = h = A.B^T and Om2 = relu2(h), and when C32/Ce are given (no reference counterpart; BLK = 32 only) also
 * transpoe(Om2) [N, M] into them, as int8 mantissas (C32) and int8 exponents [N, M/BLK] (Ce)
 * | 4: Cm = relu2_back(A.B^T, X), and when Om2/OE2 are given (no reference counterpart; BLK = 32 only) also
 * Om2 = transpoe(Cm) [N, M]
 * Requires M % 32 == 0, N % 128 == 0, K % BLK == 0, K <= 4096 (the reference: M % 64, N % 128, K % 128). */
int jt_gemm_f(const void* A, const void* EA, const void* B, const void* EB, void* Cm, void* CE, void* C32, void* Ce,
              const void* Xm, const void* XE, void* Om2, void* OE2, int M, int N, int K, int modo, int kid);
int jt_gemm_divisoes(int M, int N, int K, int modo);   /* no reference counterpart: K-splits jt_gemm_f uses
                                                        * for a shape (workgroup = 256 x tile rows / 32 x splits threads) */
int jt_gemm_tile(int M, int N, int modo);              /* no reference counterpart: tile rows (32, 64, 128) jt_gemm_f
                                                        * uses for a shape and mode */
int jt_gemm(const void* A, const void* EA, const void* B, const void* EB, void* Cm, void* CE, void* C32, void* Ce,
            int M, int N, int K, int modo, int kid);
/* no reference counterpart: Z16 = soma16(X16, A.B^T) (R16, int16 mantissas) and Y8 = para8(Z16) in one launch, the
 * bits of jt_gemm (modo 0), jt_soma16 and jt_para8 in turn (the R16 step's residual add, modelo.py:67-72, 78-84).
 * X16, Z16 int16 [M,N]; XE, ZE, YE8 int8 [M,N/BLK]; Y8 int8 [M,N]. Shapes as jt_gemm_f. Launch ids: kid for the GEMM,
 * kid + 1 for the soma16 stage, kid + 2 for the para8 stage. */
int jt_gemm_soma16(const void* A, const void* EA, const void* B, const void* EB, const void* X16, const void* XE, void* Z16,
                   void* ZE, void* Y8, void* YE8, int M, int N, int K, int kid);

/* ---- no reference counterpart: n raw-output GEMMs sharing K, in launches of up to 64. `entradas` is a HOST array of
 * n entries {const void *A, *EA, *B, *EB; void *C32, *Ce; int M, N, K, compacto;} (device pointers inside); entry i
 * equals jt_gemm(A, EA, B, EB, NULL, NULL, C32, Ce, M, N, K, 1, kid + i). For the weight gradients of a step.
 * compacto = 1 (the same in every entry): Ce is an int16 vector of M + N, Ce[i] = RA_i and Ce[M + j] = RB_j - 4,
 * whose sum is the exponent jt_gemm writes at (i, j) (2 bytes per value fewer written, and read by jt_otimizador). */
int jt_gemm_lote(const void* entradas, int n, int kid);
int jt_entrada_g_bytes(void);          /* sizeof of one entry (64) */
/* ---- no reference counterpart: n weight-gradient GEMMs sharing K with momento + peso in the epilogue, in launches of
 * up to 32. `entradas` is a HOST array of n entries {const void *A, *EA, *B, *EB; void *Mm, *ME, *Wm, *WE, *Rm, *RE;
 * int M, N, K, pad;}; entry i equals jt_gemm(A, EA, B, EB, NULL, NULL, G32, Ge, M, N, K, 1, kid + i), then
 * jt_momento(G32, Ge, Mm, ME) and jt_peso(Wm, WE, Mm, ME, Rm, RE, k_lr, ef) on the [M, N] weight (ops.py:273-290),
 * without storing the gradient. */
int jt_gemm_otim_lote(const void* entradas, int n, int k_lr, int ef, int kid);
int jt_entrada_go_bytes(void);         /* sizeof of one entry (96) */

/* ---- element-wise, nblocos = elements / BLK (jatai_cuda.cu:1128-1154, 1074-1086) */
int jt_quant(const void* acc, const void* e, void* m, void* E, long long nblocos, int kid);
int jt_soma(const void* xm, const void* xE, const void* ym, const void* yE, void* zm, void* zE, long long nblocos, int kid);
int jt_relu2(const void* hm, const void* hE, void* am, void* aE, long long nblocos, int kid);
int jt_relu2_back(const void* gm, const void* gE, const void* hm, const void* hE, void* om, void* oE, long long nblocos, int kid);
int jt_momento(const void* gacc, const void* ge, void* Mm, void* ME, long long nblocos, int kid);                 /* in place */
int jt_peso(void* Wm, void* WE, const void* Mm, const void* ME, void* Rm, void* RE, int k_lr, int ef, long long nblocos,
            int kid);                                                                                          /* in place */
int jt_para16(const void* xm, const void* xE, void* zm, void* zE, long long nblocos, int kid);
int jt_para8(const void* xm, const void* xE, void* ym, void* yE, long long nblocos, int kid);
int jt_soma16(const void* xm, const void* xE, const void* ym, const void* yE, void* zm, void* zE, long long nblocos, int kid);

/* ---- no reference counterpart: momento then peso for ntab tensors in one launch. `tabela` is a device array of
 * ntab entries {const int* gacc; const int16_t* ge; int8_t *Mm, *ME, *Wm, *WE, *Rm, *RE, *Tm, *TE; long long inicio,
 * nblocos; int M, N, compacto, pad;} sorted by inicio (the tensor's first block in a global numbering), ntab <= 256,
 * nblocos = the total; [M, N] the tensor's shape; compacto = 1: ge is jt_gemm_lote's compact exponent vector of the
 * gradient (N % 16 == 0), else one exponent per value. Results equal jt_momento followed by jt_peso on each tensor
 * (ops.py:273-290). jt_otimizador ignores Tm, TE. */
int jt_otimizador(const void* tabela, int ntab, long long nblocos, int k_lr, int ef, int kid);
int jt_tab_otim_bytes(void);           /* sizeof of one table entry (112) */
/* The same with one workgroup per 32 x 128 tile (BLK 32; every entry with M % 32 == 0 and N % 128 == 0), also
 * writing transpoe(W) of the new weight into Tm [N, M], TE [N, M / 32] where an entry sets them (null: not written):
 * the weights' transposes of the next step's backward (ops.py:121-123) without a transpose launch. */
int jt_otimizador_t(const void* tabela, int ntab, long long nblocos, int k_lr, int ef, int kid);

/* ---- re-blocking, gathers (jatai_cuda.cu:1155-1166). transpoe: R % 128 == 0, C % 64 == 0. */
int jt_transpoe(const void* X, const void* EX, void* Y, void* EY, int R, int C, int kid);
/* no reference counterpart: n transposes in launches of up to 64 tensors. `entradas` is a HOST array of n entries
 * {const void* X; const void* EX; void* Y; void* EY; int R; int C;} (device pointers inside); entry i equals
 * jt_transpoe(X, EX, Y, EY, R, C, kid + i). */
int jt_transpoe_lote(const void* entradas, int n, int kid);
int jt_entrada_t_bytes(void);          /* sizeof of one entry (40) */
int jt_embed(const void* Wm, const void* WE, const void* tok, void* Xm, void* XE, int M, int D, int V, int kid);
int jt_um_quente(const void* tok, void* U, void* UE, int M, int V, int kid);
/* Training windows of a byte corpus in device memory (no reference entry point: the reference draws them on the
 * host, treino_int8_gpu/treino.py:41-44, and copies int64 tokens in). corpus: uint8 [n]; ini: int64 [Bt] window
 * starts; tok, alvo: int32 [Bt, T] get corpus[ini[b] + t] and corpus[ini[b] + t + 1]. A start outside
 * [0, n - T - 1] raises E_ARG (index b*T, value the start) and zeroes that row. */
int jt_janelas(const void* corpus, long long n, const void* ini, void* tok, void* alvo, int Bt, int T, int kid);

/* ---- rows (jatai_cuda.cu:1167-1176, 1195-1200): rms / rms_back take any D <= 1024 that is a multiple of BLK
 * (ops.py:453), softmax_ce any V <= 1024 that is a multiple of 128 (ops.py:496) */
int jt_rms(const void* Xm, const void* XE, void* Ym, void* YE, void* cr, void* cemax, int M, int D, int log2D, int G, int kid);
int jt_rms_back(const void* gm, const void* gE, const void* ym, const void* yE, const void* cr, const void* cemax, void* om,
                void* oE, int M, int D, int log2D, int G, int GB, int kid);
/* no reference counterpart: om = soma(x, rms_back(g, y, cache)) in one launch (kid: rms_back part, kid + 1: soma) */
int jt_rms_back_soma(const void* gm, const void* gE, const void* ym, const void* yE, const void* cr, const void* cemax, const void* xm,
                     const void* xE, void* om, void* oE, int M, int D, int log2D, int G, int GB, int kid);
/* no reference counterpart: z16 = soma16(x16, rms_back(g, y, cache)) and y8 = para8(z16) in one launch (the R16
 * backward's residual update, modelo.py:114-130), the bits of jt_rms_back, jt_soma16 and jt_para8 in turn (launch
 * ids kid, kid + 1, kid + 2). x16, z16 int16 [M,D]; xE, zE, yE8 int8 [M,D/BLK]; y8 int8 [M,D]. */
int jt_rms_back_soma16(const void* gm, const void* gE, const void* ym, const void* yE, const void* cr, const void* cemax,
                       const void* x16, const void* xE, void* z16, void* zE, void* y8, void* yE8, int M, int D, int log2D, int G,
                       int GB, int kid);
int jt_softmax_ce(const void* acc, const void* e, const void* alvo, void* gm, void* gE, void* d_alvo, void* soma, int M, int V,
                  int log2M, int kid);
/* no reference counterpart: the loss of modelo.py:93, mean over M rows of d_alvo / 256 + ln(soma / 4096) (int32 rows from
 * jt_softmax_ce), as one float64 written to out, in one launch on the library's stream */
int jt_perda(const void* d_alvo, const void* soma, void* out, int M, int kid);

/* ---- causal ALiBi attention (jatai_cuda.cu:1177-1194). Head width D / H = 4, the reference's: T % 32 == 0,
 * T <= 256 (the reference: T <= 128), H <= 64, ALiBi slope 8 - h / 8 (ops.py:208, 475). No reference counterpart:
 * head widths 16, 32, 64 with T % 64 == 0, T <= 512 and slope 8 - 8h / H. Every attention entry point takes GA, the
 * guard bits of the aligned values, from 0 to 4 (the spec's is 4, ops.py:20), else hipErrorInvalidValue. */
int jt_atencao(const void* qm, const void* qE, void* Oacc, void* Oe, void* P, int Bt, int T, int H, int D, int GA, int kid);
/* no reference counterpart: jt_atencao with a caller workspace of jt_atencao_ws_bytes(Bt, T, H, D) bytes (16-byte
 * aligned); same outputs. At head width 64 on matrix cores (T <= 512) k and v are converted once per (sequence,
 * head) into the workspace and each 16-row query tile's keys are split over four waves; otherwise it runs
 * jt_atencao. */
long long jt_atencao_ws_bytes(int Bt, int T, int H, int D);
int jt_atencao_ws(const void* qm, const void* qE, void* Oacc, void* Oe, void* P, int Bt, int T, int H, int D, int GA, void* ws,
                  long long ws_bytes, int kid);
int jt_atencao_back(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gacc, void* Ge,
                    int Bt, int T, int H, int D, int GA, int limite, int kid);
/* no reference counterpart: jt_atencao_ws writing the output already quantized (Om int8 [M, D], OE int8 [M, D/32]),
 * equal to jt_quant of the raw output; head width 64 on matrix cores at BLK = 32 only, else hipErrorNotSupported. */
int jt_atencao_ws_q(const void* qm, const void* qE, void* Om, void* OE, void* P, int Bt, int T, int H, int D, int GA, void* ws,
                    long long ws_bytes, int kid);
/* no reference counterpart: jt_atencao_back with a caller workspace of jt_atencao_back_ws_bytes(Bt, T, H, D) bytes
 * (16-byte aligned); same outputs. At head width 64 on matrix cores (T <= 512) dO, q, k, v are converted once per
 * (sequence, head) into the workspace and each 16-row tile's partner tiles are split over four waves; otherwise
 * it runs jt_atencao_back. */
long long jt_atencao_back_ws_bytes(int Bt, int T, int H, int D);
int jt_atencao_back_ws(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gacc, void* Ge, int Bt, int T,
                       int H, int D, int GA, int limite, void* ws, long long ws_bytes, int kid);
/* no reference counterpart; for callers that cannot allocate (code under graph capture, tight serving loops, harnesses
 * that forbid hipMalloc): jt_atencao_back_ws with its workspace in the library's own fixed device array of
 * jt_scratch_bytes() = 32 MiB per GPU (held until the process ends), no workspace argument, and no allocation of
 * any kind. A shape whose jt_atencao_back_ws_bytes exceeds the array returns hipErrorOutOfMemory and launches
 * nothing (config 4's backward needs about 25 MB; config 5's, about 200 MB, is refused). Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams or host threads) race. */
int jt_atencao_back_sem_alocar(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gacc, void* Ge,
                               int Bt, int T, int H, int D, int GA, int limite, int kid);
long long jt_scratch_bytes(void);
/* no reference counterpart: jt_atencao_back_ws writing the gradient already quantized (Gm int8 [M, 3D], GE int8
 * [M, 3D/32]), equal to jt_quant of the raw gradient; same support as jt_atencao_ws_q. */
int jt_atencao_back_ws_q(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gm, void* GE, int Bt, int T,
                         int H, int D, int GA, int limite, void* ws, long long ws_bytes, int kid);
/* no reference counterpart: the forward/backward pair that converts q, k, v once for both. jt_atencao_ws_qs is
 * jt_atencao_ws_q that also saves, in salvo (jt_atencao_salvo_bytes(Bt, T, H, D) bytes, 16-byte aligned), the
 * backward's conversions of q, k, v; jt_atencao_back_ws_qs is jt_atencao_back_ws_q reading them from salvo, so it
 * converts only dO. The caller keeps salvo and qkv unchanged from the one call to the other. The bound variant
 * (limite = 1) converts q, k, v itself and leaves salvo unread. Same outputs as jt_atencao_ws_q and
 * jt_atencao_back_ws_q. */
long long jt_atencao_salvo_bytes(int Bt, int T, int H, int D);
int jt_atencao_ws_qs(const void* qm, const void* qE, void* Om, void* OE, void* P, int Bt, int T, int H, int D, int GA, void* ws,
                     long long ws_bytes, void* salvo, long long salvo_bytes, int kid);
int jt_atencao_back_ws_qs(const void* gom, const void* goE, const void* qm, const void* qE, const void* P, void* Gm, void* GE, int Bt, int T,
                          int H, int D, int GA, int limite, void* ws, long long ws_bytes, const void* salvo, long long salvo_bytes, int kid);

#ifdef __cplusplus
}
#endif
#endif
