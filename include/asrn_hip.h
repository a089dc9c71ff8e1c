/* ASRN layer hot path on MI355X (gfx950): C ABI of libasrn_hip.so.
 *
 * Conventions for every entry point:
 *   - device pointers are plain pointers; sizes are int64_t; `stream` is a hipStream_t passed as void*;
 *   - the return value is 0 on success, nonzero on a rejected argument or a failed launch, with the message in
 *     asrn_hip_last_error() (per calling thread);
 *   - the caller owns every buffer (outputs and workspaces); the library never allocates, frees or synchronizes;
 *   - work is stream-ordered and deterministic: no floating-point atomics, the same inputs give the same bits.
 *
 * Layout names: B batch rows, L positions, d width, T hash tables, nb bits per table, P = T*nb hash outputs,
 * C candidates per table, cf confirmation width, K suffix length, n n-gram orders. A "row" of a per-table array
 * is r = b*T + tau, as in the reference (estable:282).
 */
#ifndef ASRN_HIP_H
#define ASRN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Last error message of the calling thread ("" if none). */
const char* asrn_hip_last_error(void);

/* ABI version of this library (increments on any signature change). */
int32_t asrn_hip_abi_version(void);

/* ---- a1 + a2: sign hash and stable bucket sort ------------------------------------------------------------------
 * Replaces CapaASRN._ids (asrn/nucleo.py:661-664), `ids.argsort(dim=-1, stable=True)` and `torch.gather(ids, 1,
 * orden)` (asrn/estable.py:282-283, 288-291).
 *   phi        (B, L, phi_stride) fp32; table tau reads columns [tau*nb, tau*nb + nb); or null, and then ids is
 *              an input: the bucket ids asrn_hash_fwd wrote with its phi (the sign hash already done)
 *   ids        (B*T, L) int32 out (in when phi is null): bucket id of each position, text order
 *   order      (B*T, L) int32 out: sorted rank -> text position (stable: ties keep text order)
 *   ids_sorted (B*T, L) int32 out: ids[order]
 *   rank       (B, L, T) int32 out: text position -> sorted rank, per table
 *   win        (B, L, T) int32 out: the recent-mates index, min(C, earlier positions in the bucket) |
 *              min(C, later positions in the bucket) << 8: the query window is the last `win & 255` sorted ranks
 *              before `rank`, the key window the first `win >> 8` after it
 *   workspace  asrn_bucket_sort_workspace(B, L, T) bytes (0, and workspace may be null, unless 1024 < L <= 4096)
 * Requires 1 <= nb <= 14, 1 <= C <= 255. */
int64_t asrn_bucket_sort_workspace(int64_t B, int64_t L, int32_t T);
int asrn_bucket_sort(const float* phi, int64_t B, int64_t L, int32_t T, int32_t nb, int64_t phi_stride, int32_t C,
                     int32_t* ids, int32_t* order, int32_t* ids_sorted, int32_t* rank, int32_t* win, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* ---- a3 - a7: candidate attention, forward ---------------------------------------------------------------------
 * Replaces _CasillerosTriton.forward / _casilleros_ida in ESTABLE mode (asrn/nucleo.py:359-382, 465-488) as called
 * from CapaASRNEstable._acumular_triton (asrn/estable.py:274-292), with the table sum and the gate signals of
 * _senales (asrn/estable.py:294-300) done in the kernel.
 * For query t and table tau the candidates are the last (win & 255) sorted ranks before s = rank of t (both from
 * asrn_bucket_sort): its <= C most recent earlier bucket mates. Score = <phi_q, phi_k> * scale_phi + <Qc_q, Kc_k> * scale_c
 * + w_suf[suffix match] + log_alfa_k + (gamma_tau / C) * fp32(Bt_k - Bt_q); exact masked softmax.
 *   sig (B, L) fp32 token signatures; Bt (B, L) fp64 clock; log_alfa (B, L); w_suf (K+1); gamma (T)
 *   salida  (B, L, d) out: sum over tables of sum_k att * V_k (bf16, rounded to nearest even, when rows_bf16 > 0)
 *   signals (B, L, 4) out: peso_total, mejor, pico, peso_ctx
 *   entries (B, L, T, C, 2) out: [..., 0] the weight of each candidate, at [query][tau][distance - 1] (distance
 *           in sorted ranks, 1..n; slots beyond the table's n candidates are not written); [..., 1] is filled by the
 *           backward. Kept for the backward.
 *   lists   (B*L, asrn_candidates_record_bytes(T, C)) bytes out, or null: each query's deduplicated candidate list,
 *           which the backward's query pass then reads instead of gathering and deduplicating again.
 *   V rows: position p of batch row b is read at V + (b*L + p + v_shift) * ldv (ldv >= d, a multiple of 4, V 16-byte
 *           aligned). v_shift = 0: V as the reference passes it (V[p] = W_v E[p+1], nucleo:659, the last row 0);
 *           v_shift = 1: V is the projection W_v E of every position (e.g. a column block of a wider GEMM output,
 *           ldv its row stride), and the kernels read the next position's row themselves.
 *   rows_bf16: 0 fp32 rows; 1 V holds bf16 values (the same layout in 2-byte elements; the reference's V under
 *           bf16 autocast); 2 phi, Qc and Kc are bf16 too. The kernels widen each element exactly, so the results
 *           equal those from fp32 copies.
 *   Qc, Kc rows: row t at Qc + t * ldq (and Kc + t * ldq): ldq = cf for dense rows, or the row stride when both are
 *           column blocks of one projection (ldq >= cf, a multiple of 4, rows 16-byte aligned).
 *   clock_mode: 0 the protected layer's clock term above (fp64 clock, difference taken before the product); 1 the
 *           unprotected core layer's (asrn.ASRNCoreLayer = nucleo.CapaASRN, nucleo:330-332, 815-817): Bt holds the
 *           fp32 clock (fp32 values in fp64), and the term is (log_alfa_k + rate * B_k) - rate * B_q in fp32, each
 *           product and sum rounded on its own, added to base + w_suf.
 *   leak: null, or a device int32 to which the kernel adds the number of (query, table) pairs whose best valid score
 *           is within 256 of -1e9. There the core layer's -1e9 fill (nucleo:337-339, 813) gives the invalid keys of
 *           its block window weight (the leak estable:20-24 describes), which the exact candidate set here never
 *           sees; everywhere else the fill and the exact mask give the same weights. The caller clears it.
 * Requires d % 4 == 0 (widths past 1024 run the value phases over column slabs of 1024), 1 <= C <= 64,
 * P + cf <= 256, K <= 16, T <= 32, L * ldv < 2^31. */
int asrn_candidates_fwd(const float* phi, const float* V, const float* Qc, const float* Kc, const float* sig,
                        const double* Bt, const float* log_alfa, const float* w_suf, const float* gamma,
                        const int32_t* order, const int32_t* win, const int32_t* rank, int64_t B, int64_t L,
                        int32_t d, int32_t P, int32_t cf, int32_t K, int32_t T, int32_t Tc, int32_t C,
                        float scale_phi, float scale_c, int64_t ldv, int32_t v_shift, int64_t ldq, int32_t rows_bf16,
                        float* salida, float* signals, float* entries, uint8_t* lists, int32_t clock_mode,
                        int32_t* leak, void* stream);

/* Bytes of one token's record in the `lists` buffer (B*L records, 16-byte aligned): the query's deduplicated candidate
 * list (table offsets, each entry's distinct candidate, the candidates' positions, clock differences and suffix
 * lengths) as the forward builds it. */
int64_t asrn_candidates_record_bytes(int32_t T, int32_t C);

/* The candidate lists the forward and backward walk, materialized for checking (a3, a4): for each (b, t, tau) the
 * text positions of the <= C most recent earlier bucket mates in the C-slot window [s - C, s) of the sorted row
 * (oldest first; the empty slots come first and hold -1), and their suffix-match lengths (asrn/nucleo.py:98-108,
 * 313-320).
 *   pos, ell (B, L, T, C) int32 out (-1 where the window slot holds no candidate). */
int asrn_candidate_lists(const float* sig, const int32_t* order, const int32_t* win, const int32_t* rank,
                         int64_t B, int64_t L, int32_t T, int32_t C, int32_t K, int32_t* pos, int32_t* ell,
                         void* stream);

/* ---- a8: candidate attention, backward -------------------------------------------------------------------------
 * Replaces _CasillerosTriton.backward / _casilleros_vuelta (asrn/nucleo.py:384-451, 490-515). Two passes with one
 * owner per output row, so no atomics, and neither recomputes a score: a query pass (from the forward's att:
 * ds = att (dp - D) with D = sum att*dp per (query, table), query-side gradients, per-query partials of d gamma and
 * d w_suf) and a key pass (key-side gradients from att and ds at the slots of the queries that see the key: the
 * next <= C same-bucket sorted ranks).
 *   dsalida (B, L, d), 16-byte aligned: bf16 with V when rows_bf16 > 0; entries from asrn_candidates_fwd (its
 *   [..., 1] receives ds, read back by the key pass)
 *   lists   the forward's candidate lists (same inputs), or null to gather and deduplicate again
 *   dphi (B, L, P) dense, dBt (B, L) fp64, dlog_alfa (B, L) out (overwritten); dV (bf16 when rows_bf16 > 0), dQc
 *   and dKc (fp32) have the layout of
 *   V, Qc and Kc (row strides ldv and ldq, 16-byte aligned): their d (cf) columns of every row are written, the rest
 *   of a row is left alone; with v_shift = 1, dV is the gradient of the per-position rows (row 0 of each batch row
 *   is 0)
 *   partials (B*L, T + K + 1) fp32 out: per query, d gamma_tau then d w_suf[0..K]; the caller sums over rows. */
int asrn_candidates_bwd(const float* phi, const float* V, const float* Qc, const float* Kc, const float* sig,
                        const double* Bt, const float* log_alfa, const float* w_suf, const float* gamma,
                        const int32_t* order, const int32_t* win, const int32_t* rank, int64_t B, int64_t L,
                        int32_t d, int32_t P, int32_t cf, int32_t K, int32_t T, int32_t Tc, int32_t C,
                        float scale_phi, float scale_c, int64_t ldv, int32_t v_shift, int64_t ldq, int32_t rows_bf16,
                        const float* dsalida, float* entries, const uint8_t* lists, float* dphi, float* dV,
                        float* dQc, float* dKc, double* dBt, float* dlog_alfa, float* partials, void* stream);

/* ---- scan workspace -------------------------------------------------------------------------------------------
 * No counterpart in the reference (PyTorch allocates for it). Every scan below cuts its rows into chunks spread over
 * the CUs; rows longer than 1024 elements need a device workspace of asrn_scan_workspace(rows, N) bytes for the chunk
 * totals (0 for shorter rows, where the workspace pointer may be null; -1 when rows x chunks would reach 2^31). The
 * contents need no clearing and are dead after the call. */
int64_t asrn_scan_workspace(int64_t rows, int64_t N);

/* ---- a0 (part): the context producer's LayerNorm and clock projection (asrn/estable.py:153-194) ----------------
 * Replaces ln_ctx, the fp32 clock projection and its softplus / logsigmoid / clamps of _contexto. Per token of h
 * (BL, d) fp32: hh = LayerNorm(h) (biased variance, eps) * ln_w + ln_b (BL, d) fp32 out, the input of the Qc/Kc GEMM;
 * u_k = hh . w_reloj[k] + b_reloj[k] (w_reloj (2, d)); beta = min(softplus(u_0), beta_max) (BL) fp64 out (beta_max < 0:
 * no clamp); log_alfa = max(logsigmoid(u_1) + log 2, log_alfa_min) (BL) fp32 out (-inf: no clamp); stats (BL, 4) =
 * (mean, rstd, u_0, u_1) kept for the backward. d % 4 == 0, d <= 1024.
 * context_bwd: from dhh (BL, d) (the Qc/Kc GEMM's input gradient), or instead from that GEMM's output gradient dy
 * (BL rows of ny <= 32, row stride ldy) and its weight wq (ny, d) with d <= 512, as dhh = dy wq formed in the kernel
 * (replacing the GEMM `grad @ weight` of the Linear's backward), and from dbeta (BL) fp64 and dlog_alfa (BL): gives
 * dh (BL, d) (overwritten; plus dh_add (BL, d) when not null: the gradient of h through the gate) and dparams
 * (4 d + 2) = the gradients of [ln_w | ln_b | w_reloj (2 d) | b_reloj (2)], summed over tokens in a fixed order.
 * Exactly one of dhh and dy is given. workspace: asrn_context_bwd_workspace(BL, d) bytes. */
int asrn_context_fwd(const float* h, const float* ln_w, const float* ln_b, const float* w_reloj, const float* b_reloj,
                     int64_t BL, int32_t d, float eps, float beta_max, float log_alfa_min, float* hh, float* stats,
                     double* beta, float* log_alfa, void* stream);
int64_t asrn_context_bwd_workspace(int64_t BL, int32_t d);
int asrn_context_bwd(const float* h, const float* ln_w, const float* ln_b, const float* w_reloj, const float* stats,
                     int64_t BL, int32_t d, float beta_max, float log_alfa_min, const float* dhh, const float* dy,
                     int64_t ldy, int32_t ny, const float* wq, const double* dbeta, const float* dlog_alfa,
                     const float* dh_add, float* dh, float* dparams, void* workspace, int64_t workspace_bytes,
                     void* stream);

/* ---- a0 (part): the hash MLPs' hidden layer (asrn/nucleo.py:644-659) -------------------------------------------
 * Replaces the GELU of afin_palabra and afin_contexto between their two Linear layers, with the context MLP's first
 * layer on the key [E_t; E_{t-1}] (nucleo:649-652) split by linearity. y (B*L, ldy) fp32 holds, per token, the bias-free
 * products hp = W_p E_t at columns [0, m), za = W_a E_t at [m, m + mc) and zb = W_b E_t at [m + mc, m + 2 mc), where
 * [W_a | W_b] = afin_contexto[0].weight. hidden_fwd writes g (B*L, m + mc) = [gelu(hp + b_word) | gelu(za + zb[t-1] +
 * b_ctx)] (no zb term at t = 0; gelu in the exact erf form). hidden_bwd, from dg (B*L, m + mc), writes columns
 * [0, m + 2 mc) of dy (B*L, ldd): the gradients of hp, za and zb (zb's at t is the context pre-activation's gradient
 * at t + 1, 0 at a row's last position); the biases' gradients are then the column sums of dy's first m + mc
 * columns. m and mc multiples of 4; rows, g, dg and the biases 16-byte aligned. */
int asrn_hidden_fwd(const float* y, int64_t ldy, const float* b_word, const float* b_ctx, int64_t B, int64_t L,
                    int32_t m, int32_t mc, float* g, void* stream);
int asrn_hidden_bwd(const float* y, int64_t ldy, const float* b_word, const float* b_ctx, int64_t B, int64_t L,
                    int32_t m, int32_t mc, const float* dg, float* dy, int64_t ldd, void* stream);

/* ---- a0 (part): the hash MLPs from their first layers to phi, fused (asrn/nucleo.py:644-659) ---------------------
 * Replaces the GELU and both second layers of afin_palabra and afin_contexto (and the block-diagonal GEMM they would
 * be): with y as for asrn_hidden_fwd, hash_fwd writes phi (B*L, Pw + Pc) = [gelu(hp + b_word) W2w^T + b2w |
 * gelu(za + zb[t-1] + b_ctx) W2c^T + b2c], W2w (Pw, m) = afin_palabra[2].weight, W2c (Pc, mc) = afin_contexto[2].weight.
 * hash_bwd, from dphi (B*L, Pw + Pc), writes columns [0, m + 2 mc) of dy (B*L, ldd) as asrn_hidden_bwd does, and
 * dparams = [dW2w (Pw*m) | dW2c (Pc*mc) | db2w (Pw) | db2c (Pc) | db_word (m) | db_ctx (mc)], summed over the tokens
 * in a fixed order. The second layers run on the matrix cores. m, mc multiples of 4 in [4, 64] with (m + mc) / 4
 * dividing 256; Pw, Pc in [1, 64]; y, dy rows and the first-layer biases 16-byte aligned.
 * hash_fwd with ids non-null also writes the sign hash of the phi it stores (CapaASRN._ids, asrn/nucleo.py:661-664):
 * ids (B*T, L) int32, table tau's id from the signs (strict > 0) of columns [tau*nb, tau*nb + nb), for
 * asrn_bucket_sort with a null phi; T*nb = Pw + Pc, 1 <= T <= 32, 1 <= nb <= 14.
 * workspace: asrn_hash_bwd_workspace(...) bytes, 256-byte aligned. */
int asrn_hash_fwd(const float* y, int64_t ldy, const float* b_word, const float* b_ctx, const float* w2_word,
                  const float* b2_word, const float* w2_ctx, const float* b2_ctx, int64_t B, int64_t L, int32_t m,
                  int32_t mc, int32_t p_word, int32_t p_ctx, float* phi, int32_t* ids, int32_t T, int32_t nb,
                  void* stream);
int64_t asrn_hash_bwd_workspace(int64_t B, int64_t L, int32_t m, int32_t mc, int32_t p_word, int32_t p_ctx);
int asrn_hash_bwd(const float* y, int64_t ldy, const float* b_word, const float* b_ctx, const float* w2_word,
                  const float* w2_ctx, int64_t B, int64_t L, int32_t m, int32_t mc, int32_t p_word, int32_t p_ctx,
                  const float* dphi, float* dy, int64_t ldd, float* dparams, void* workspace, int64_t workspace_bytes,
                  void* stream);

/* ---- column sums -----------------------------------------------------------------------------------------------
 * No counterpart in the reference's FFI: the reductions PyTorch's autograd runs for it (the bias gradients of its
 * nn.Linear projections, asrn/nucleo.py:591-630, and the parameter sums of the candidate backward, nucleo:465-515).
 * out (cols) fp32 = the sum over the rows of x (rows, cols) with row stride ld, fp32 or bf16 (bf16 != 0), summed in
 * fp32 in a fixed order. workspace: asrn_column_sums_workspace(rows, cols) bytes (0: none needed). */
int64_t asrn_column_sums_workspace(int64_t rows, int64_t cols);
int asrn_column_sums(const void* x, int32_t bf16, int64_t rows, int64_t cols, int64_t ld, float* out,
                     void* workspace, int64_t workspace_bytes, void* stream);

/* ---- products of small matrices ---------------------------------------------------------------------------------
 * No counterpart in the reference's FFI. The layer applies W_o W_v to the gathered sum of embedding rows (the two
 * linear maps the reference applies one after the other, V = v(E shifted) at asrn/nucleo.py:683 and aporte =
 * o(salida) at asrn/estable.py:402); this forms W_o W_v and the two products of its backward. C (M, N) = op(A) op(B) in fp32, op(X) = X or X^T (trans != 0), row-major with leading
 * dimensions lda, ldb, ldc; each element sums over k in order. M, N, K <= 8192. */
int asrn_small_gemm(const float* A, int64_t lda, int32_t trans_a, const float* B, int64_t ldb, int32_t trans_b,
                    float* C, int64_t ldc, int32_t M, int32_t N, int32_t K, void* stream);

/* ---- batched block copies -------------------------------------------------------------------------------------
 * No counterpart in the reference's FFI: the layer assembles its fused GEMMs' weights from the parameters (the
 * torch.cat / block_diag calls it would make every step) and scatters their gradients back, each in one launch.
 * n <= 16 blocks, given as host arrays: block i copies rows[i] x cols[i] fp32 from src[i] (row stride sld[i]) to
 * dst[i] (row stride dld[i]), or writes zeros when src[i] is null. */
int asrn_copy_blocks(int32_t n, const float* const* src, float* const* dst, const int64_t* sld, const int64_t* dld,
                     const int64_t* rows, const int64_t* cols, void* stream);

/* ---- a9: clock --------------------------------------------------------------------------------------------------
 * Bt = cumsum(beta) over L in fp64 (asrn/estable.py:418). mode 0: prefix sums; 1: suffix sums (the backward of the
 * cumsum); 2: prefix sums each rounded to fp32 (stored in fp64) with the running sum kept in fp64, the unprotected
 * core layer's fp32 clock (asrn/nucleo.py:882, beta.cumsum(1) in fp32, which the CPU accumulates in double).
 * workspace: asrn_scan_workspace(B, L) bytes. */
int asrn_clock_scan(const double* x, double* y, int64_t B, int64_t L, int32_t mode, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* ---- a10: n-gram keys, stable key sort, repeated and seen flags -------------------------------------------------
 * Replaces _claves_de (asrn/nucleo.py:175-185), _ordenar_claves (asrn/nucleo.py:693-701) and the scatter of the seen
 * flags (asrn/estable.py:310-312).
 *   sig (B, L) fp32; coef (n) fp64 (the c_vistos buffer)
 *   keys (B, L, n) fp64 out: k_j(t) = (((0 + s_t c_0) + s_{t-1} c_1) + ...) with separate roundings, NaN when the
 *        group starts before the text
 *   order (B, n, L) int32 out: stable sort of each (b, j) row by key, NaN last
 *   repeated (B, n, L) uint8 out: key[order[i]] == key[order[i-1]]
 *   rank_k (B, n, L) int32 out: text position -> sorted index
 *   vistos (B, L, n) fp32 out: repeated scattered back to text order
 *   workspace: asrn_ngram_sort_workspace(B, L, n) bytes. */
int64_t asrn_ngram_sort_workspace(int64_t B, int64_t L, int32_t n);
int asrn_ngram_sort(const float* sig, const double* coef, int64_t B, int64_t L, int32_t n, double* keys,
                    int32_t* order, uint8_t* repeated, int32_t* rank_k, float* vistos, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* ---- a12: affine scan S_i = a_i S_{i-1} + b_i over rows of N (asrn/nucleo.py:188-196, 214-257, 518-537) --------
 * scan_bwd: l_i = g_i + a_{i+1} l_{i+1}; gb = l; ga_i = l_i S_{i-1}. workspace: asrn_scan_workspace(rows, N) bytes. */
int asrn_scan_fwd(const float* a, const float* b, float* S, int64_t rows, int64_t N, void* workspace,
                  int64_t workspace_bytes, void* stream);
int asrn_scan_bwd(const float* a, const float* S, const float* g, float* ga, float* gb, int64_t rows, int64_t N,
                  void* workspace, int64_t workspace_bytes, void* stream);

/* asrn_scan_fwd with no workspace argument and no allocation: no counterpart in the reference. It is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The chunk totals live in a static device array of asrn_scan_static_scratch_bytes() bytes (4 MiB) per GPU, held
 * until the process ends; sizes whose asrn_scan_workspace(rows, N) exceeds it are rejected with an error. Same
 * kernels and results as asrn_scan_fwd. Every call on one GPU shares that array: calls that overlap on one GPU race
 * (order them on one stream). */
int64_t asrn_scan_static_scratch_bytes(void);
int asrn_scan_fwd_static(const float* a, const float* b, float* S, int64_t rows, int64_t N, void* stream);

/* ---- a11: Hawkes intensities in key order (asrn/estable.py:313-318) ---------------------------------------------
 * Per (b, j) row in key order: dB_i = fp32(max(0, Bt[o_i] - Bt[o_{i-1}])), a_i = repeated_i exp(-kappa_j dB_i),
 * lambda = scan(a, a * alfa_{i-1}) with alfa = exp(log_alfa); hawkes[b, o_i, j] = lambda_i.
 *   hawkes (B, L, n) out; S_sorted (B, n, L) out (lambda in key order, kept for the backward)
 * hawkes_bwd: from dhawkes (B, L, n) gives dBt (B, L) fp64 and dlog_alfa (B, L) (overwritten) and dkappa (B, n)
 * per-row partials of d kappa_j. Workspaces: asrn_scan_workspace(B * n, L) bytes for hawkes_fwd,
 * asrn_hawkes_bwd_workspace(B, L, n) for hawkes_bwd. */
int asrn_hawkes_fwd(const int32_t* order, const uint8_t* repeated, const double* Bt, const float* log_alfa,
                    const float* kappa, int64_t B, int64_t L, int32_t n, float* hawkes, float* S_sorted,
                    void* workspace, int64_t workspace_bytes, void* stream);
int64_t asrn_hawkes_bwd_workspace(int64_t B, int64_t L, int32_t n);
int asrn_hawkes_bwd(const int32_t* order, const uint8_t* repeated, const int32_t* rank_k, const double* Bt,
                    const float* log_alfa, const float* kappa, const float* S_sorted, const float* dhawkes,
                    int64_t B, int64_t L, int32_t n, double* dBt, float* dlog_alfa, float* dkappa, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* ---- a11: repetition streak (asrn/estable.py:319-320) ----------------------------------------------------------
 * racha = scan(r exp(-kappa_r fp32(beta)), r) over the text with r = vistos[:, :, n-1].
 * streak_bwd: dbeta (B, L) fp64 (overwritten) and dkappa_r (B) per-row partials of d kappa_r.
 * workspace: asrn_scan_workspace(B, L) bytes. */
int asrn_streak_fwd(const float* vistos, const double* beta, const float* kappa_r, int64_t B, int64_t L, int32_t n,
                    float* racha, void* workspace, int64_t workspace_bytes, void* stream);
int asrn_streak_bwd(const float* vistos, const double* beta, const float* kappa_r, const float* racha,
                    const float* dracha, int64_t B, int64_t L, int32_t n, double* dbeta, float* dkappa_r,
                    void* workspace, int64_t workspace_bytes, void* stream);

/* ---- a11: the repetition branch's two scans in shared launches (asrn/estable.py:304-321) -----------------------
 * asrn_hawkes_fwd and asrn_streak_fwd in one pass, the same outputs: the B n Hawkes rows and the B streak rows share
 * the scan's launches (the totals, the chunks and, backward, the per-row sums); asrn_repetition_bwd likewise stands
 * for asrn_hawkes_bwd and asrn_streak_bwd. Workspaces: asrn_repetition_workspace(B, L, n) bytes forward,
 * asrn_repetition_bwd_workspace(B, L, n) backward. No reference counterpart as one call: the reference runs the two
 * scans one after the other in _repeticion. */
int64_t asrn_repetition_workspace(int64_t B, int64_t L, int32_t n);
int asrn_repetition_fwd(const int32_t* order, const uint8_t* repeated, const double* Bt, const float* log_alfa,
                        const float* kappa, const float* vistos, const double* beta, const float* kappa_r, int64_t B,
                        int64_t L, int32_t n, float* hawkes, float* S_sorted, float* racha, void* workspace,
                        int64_t workspace_bytes, void* stream);
int64_t asrn_repetition_bwd_workspace(int64_t B, int64_t L, int32_t n);
int asrn_repetition_bwd(const int32_t* order, const uint8_t* repeated, const int32_t* rank_k, const double* Bt,
                        const float* log_alfa, const float* kappa, const float* S_sorted, const float* dhawkes,
                        const float* vistos, const double* beta, const float* kappa_r, const float* racha,
                        const float* dracha, int64_t B, int64_t L, int32_t n, double* dBt, float* dlog_alfa,
                        float* dkappa, double* dbeta, float* dkappa_r, void* workspace, int64_t workspace_bytes,
                        void* stream);

/* ---- a13: the gate consumer (asrn/estable.py:376-403, asrn/nucleo.py:865-878) -------------------------------
 * Replaces the PyTorch ops of _combinar after W_o: with A = W_o salida (B*L, d) (fp32, or bf16 when aporte_bf16),
 * r = 1 / max(1, peso_total) and
 *   logit = (h . w_g + b_g) + (sen . w_conf + b_conf) + vistos . w_vistos + log1p(hawkes) . u_hawkes + f(racha),
 *   sen = [peso_total / T, clip(mejor, +-mejor_max) or 0 without candidates, pico / max(1, peso_total), peso_ctx / Tc],
 *   f(racha) = cumsum(d_racha)[i] + (x - i) d_racha[i + 1], x = min(log1p(racha) / racha_paso, nodes - 1),
 *   i = clamp(floor(x), 0, nodes - 2),
 * gives out = h + sigmoid(cap(logit)) r A (cap(l) = tope tanh(l / tope) when tope > 0; mejor_max < 0: no clip) and
 * the logit (B*L) kept for the backward. h, out fp32 (B*L, d); signals (B*L, 4) from asrn_candidates_fwd; vistos,
 * hawkes (B*L, n); racha (B*L); w_g (d), b_g (1), w_conf (4), b_conf (1), w_vistos (n), u_hawkes (n), d_racha (nodes).
 * d % 4 == 0, d <= 1024, 6 + 2 n + nodes <= 64.
 * gate_bwd: from dout gives dh (fp32), daporte (A's dtype), dhawkes (B*L, n), dracha (B*L) and dparams (d + 64) =
 * the gradients of [w_g | b_g | w_conf | b_conf | w_vistos | u_hawkes | d_racha | unused], summed over tokens in a
 * fixed order. workspace: asrn_gate_bwd_workspace(B*L, d) bytes. */
int asrn_gate_fwd(const float* h, const void* aporte, int32_t aporte_bf16, const float* signals, const float* vistos,
                  const float* hawkes, const float* racha, const float* w_g, const float* b_g, const float* w_conf,
                  const float* b_conf, const float* w_vistos, const float* u_hawkes, const float* d_racha, int64_t BL,
                  int32_t d, int32_t n, int32_t nodes, int32_t T, int32_t Tc, float racha_paso, float mejor_max,
                  float tope, float* logit, float* out, void* stream);
/* gate_step: the generation step's W_o product and gate in one launch, for a few fp32 tokens (replaces
 * _combinar's `self.o(salida)` and the gate after it, asrn/estable.py:376-403, in _Escritor.paso, asrn/nucleo.py:
 * 1797-1854): A = salida W_o^T with salida (BL, d) the step's attention output and w_o (d, d) = o.weight, then out and
 * logit exactly as gate_fwd gives them from A (its per-token logit and factor, computed alike). BL <= 2^20; h, salida,
 * w_o, w_g and out 16-byte aligned. */
int asrn_gate_step(const float* h, const float* salida, const float* w_o, const float* signals, const float* vistos,
                   const float* hawkes, const float* racha, const float* w_g, const float* b_g, const float* w_conf,
                   const float* b_conf, const float* w_vistos, const float* u_hawkes, const float* d_racha, int64_t BL,
                   int32_t d, int32_t n, int32_t nodes, int32_t T, int32_t Tc, float racha_paso, float mejor_max,
                   float tope, float* logit, float* out, void* stream);
int64_t asrn_gate_bwd_workspace(int64_t BL, int32_t d);
int asrn_gate_bwd(const float* h, const void* aporte, int32_t aporte_bf16, const float* signals, const float* vistos,
                  const float* hawkes, const float* racha, const float* w_g, const float* b_g, const float* w_conf,
                  const float* b_conf, const float* w_vistos, const float* u_hawkes, const float* d_racha, int64_t BL,
                  int32_t d, int32_t n, int32_t nodes, int32_t T, int32_t Tc, float racha_paso, float mejor_max,
                  float tope, const float* logit, const float* dout, float* dh, void* daporte, float* dhawkes,
                  float* dracha, float* dparams, void* workspace, int64_t workspace_bytes, void* stream);

/* ---- a14: the O(1) generation step (asrn/nucleo.py:1585-1854, asrn/estable.py:359-372) ------------------------
 * Rings: rings (B*T, 2^nb, C) int32 positions (-1 empty), counts (B*T, 2^nb) int32. The r-th position to enter a
 * bucket sits in slot r % C (the C most recent are kept).
 *
 * ring_build replaces _anillo_desde (asrn/nucleo.py:1585-1607): rings of positions 0..n-1 from their stable bucket
 * sort (asrn_bucket_sort over those n positions: order and ids_sorted, rows of n). Fills and builds. */
int asrn_ring_build(const int32_t* order, const int32_t* ids_sorted, int64_t B, int64_t n, int32_t T, int32_t nb,
                    int32_t C, int32_t* rings, int32_t* counts, void* stream);

/* decode_attend replaces _candidatos + _atender_cand + _acc_cand (asrn/nucleo.py:1621-1631, asrn/estable.py:359-372,
 * asrn/nucleo.py:947-951), and with insert != 0 also _anillo_meter (asrn/nucleo.py:1610-1618) after the attention.
 * The caches are (B, cap, .) rows: phi (P = T*nb), V (d), Qc, Kc (cf), sig, Bt (fp64), log_alfa; row t is the
 * query (its phi, Qc, sig and Bt must be written), rows < t with a ring entry are the candidates (V[t-1] included).
 * Out: salida (B, d) summed over tables, signals (B, 4) = (peso_total, mejor, pico, peso_ctx) as in
 * asrn_candidates_fwd, ids (B, T) the query's bucket ids.
 * t_dev: null, or a device int64 holding the position, which the kernel then reads (a step captured once in a HIP
 * graph and replayed as the position advances); t is then checked as the largest position it will hold, and a
 * position outside [0, cap) writes nothing.
 * The clock term is la_k + rate * fp32(B_k - B_q) for both layers: the core layer's writer takes the difference of
 * its fp32 clock too (asrn/nucleo.py:937). leak: as in asrn_candidates_fwd (null, or a device int32 counter).
 * done: null, or a device int32 (B) holding zeros, kept by the caller across calls (each launch leaves it zero): with
 * it, when B ceil(d / 256) <= 256, each row's value columns are gathered by ceil(d / 256) workgroups (a row's value
 * rows are what one CU's share of bandwidth bounds), the last of them to finish reading the rings inserting t. The
 * outputs are the same but for the order of the value sums. Calls sharing one done buffer must not overlap. */
int asrn_decode_attend(const float* phi, const float* V, const float* Qc, const float* Kc, const float* sig,
                       const double* Bt, const float* log_alfa, const float* w_suf, const float* gamma,
                       int32_t* rings, int32_t* counts, int64_t B, int64_t cap, int64_t t, const int64_t* t_dev,
                       int32_t d, int32_t nb, int32_t cf, int32_t K, int32_t T, int32_t Tc, int32_t C,
                       float scale_phi, float scale_c, int32_t insert, float* salida, float* signals, int32_t* ids,
                       int32_t* leak, int32_t* done, void* stream);

/* Hawkes memory: per (b, j) group an open-addressing table of cap slots (a power of two, >= 2x the keys it can
 * hold): tab_keys (B*n, cap) uint64 key codes, tab_Bu (B*n, cap) fp64 clock of the last occurrence, tab_A (B*n, cap)
 * fp32 lambda + alfa there.
 * hawkes_table_load replaces _MemoriaHawkes.cargar (asrn/nucleo.py:1656-1681): the state after a text of L from its
 * asrn_ngram_sort outputs (keys, order, repeated) and asrn_hawkes_fwd's hawkes; cap >= 2 L.
 * hawkes_table_grow replaces _MemoriaHawkes._ranuras' doubling (asrn/nucleo.py:1649-1654): rehash into new_cap. */
int asrn_hawkes_table_load(const double* keys, const int32_t* order, const uint8_t* repeated, const float* hawkes,
                           const double* Bt, const float* log_alfa, int64_t B, int64_t L, int32_t n, int64_t cap,
                           uint64_t* tab_keys, double* tab_Bu, float* tab_A, void* stream);
int asrn_hawkes_table_grow(const uint64_t* old_keys, const double* old_Bu, const float* old_A, int64_t groups,
                           int64_t old_cap, uint64_t* new_keys, double* new_Bu, float* new_A, int64_t new_cap,
                           void* stream);

/* repetition_step replaces the clock advance (asrn/nucleo.py:1826), the step's n-gram keys (_claves_de,
 * asrn/nucleo.py:175-186), _MemoriaHawkes.paso (asrn/nucleo.py:1683-1714) and _repeticion_o1
 * (asrn/nucleo.py:953-960) for position t: Bt[:, t] = Bt[:, t-1] + beta_t (written), vistos and hawkes (B, n) out,
 * racha (B) updated in place. sig, Bt, log_alfa are (B, stride) caches; cap >= 2 (t + 1). t_dev: as for
 * asrn_decode_attend (a position outside [0, stride) writes nothing). reloj32 != 0: the core layer's fp32 clock,
 * Bt[:, t] = fp32(fp32(Bt[:, t-1]) + fp32(beta_t)) (its cache in fp32, asrn/nucleo.py:1826), stored in fp64. */
int asrn_repetition_step(const float* sig, double* Bt, const float* log_alfa, const double* beta_t,
                         const double* coef, const float* kappa, const float* kappa_r, int64_t B, int64_t stride,
                         int64_t t, const int64_t* t_dev, int32_t n, int64_t cap, uint64_t* tab_keys, double* tab_Bu,
                         float* tab_A, float* racha, float* vistos, float* hawkes, int32_t reloj32, void* stream);

/* decode_attend_repeat: asrn_decode_attend and asrn_repetition_step for one position in a single launch, no
 * counterpart in the reference's FFI (its step runs _repeticion_o1 and the attention one after the other,
 * asrn/nucleo.py:1826-1850). The first arguments are asrn_decode_attend's, the rest asrn_repetition_step's (sig, Bt,
 * log_alfa, B, t and t_dev shared; the caches' capacity cap is the step's stride; the Hawkes tables' capacity is
 * tab_cap). The outputs are those of the two calls made in that order, bit for bit: the attention forms the query's
 * clock Bt[t] = Bt[t-1] + beta_t as the step does instead of reading what the step writes. done: as for
 * asrn_decode_attend (the same bits as that call with the same done). */
int asrn_decode_attend_repeat(const float* phi, const float* V, const float* Qc, const float* Kc, const float* sig,
                              double* Bt, const float* log_alfa, const float* w_suf, const float* gamma, int32_t* rings,
                              int32_t* counts, int64_t B, int64_t cap, int64_t t, const int64_t* t_dev, int32_t d,
                              int32_t nb, int32_t cf, int32_t K, int32_t T, int32_t Tc, int32_t C, float scale_phi,
                              float scale_c, int32_t insert, float* salida, float* signals, int32_t* ids,
                              int32_t* leak, const double* beta_t, const double* coef, const float* kappa,
                              const float* kappa_r, int32_t n, int64_t tab_cap, uint64_t* tab_keys, double* tab_Bu,
                              float* tab_A, float* racha, float* vistos, float* hawkes, int32_t reloj32, int32_t* done,
                              void* stream);

/* embed_step: the generation loop step's embedding rows, no counterpart in the reference's FFI (its loop looks the
 * rows up with nn.Embedding, asrn/nucleo.py:1805, and keeps the previous one): e_t = emb[ids] and e_prev =
 * emb[text[:, *pos - 1]] (B, d) fp32, emb (V, d); *pos (a device int64) >= 1; rows 16-byte aligned. */
int asrn_embed_step(const float* emb, int64_t V, int32_t d, const int64_t* ids, const int64_t* text, int64_t ld_text,
                    const int64_t* pos, int64_t B, float* e_t, float* e_prev, void* stream);

/* decode_produce replaces the per-token producers of _Escritor.paso (asrn/nucleo.py:1797-1826): for the B new tokens
 * at position t (or *t_dev, as asrn_decode_attend), e, e_prev, h (B, d) fp32, pieza (B) int64, it writes into the
 * (B, cap, .) caches V[t-1] = W_v e (asrn/nucleo.py:683), phi[t] = the hash MLPs on [e; e_prev] (asrn/nucleo.py:644-659),
 * Qc[t], Kc[t] = cq hh, ck hh and log_alfa[t] with hh = LayerNorm(h) and the clock projection (asrn/estable.py:153-194),
 * sig[t] = pieza; beta (B) fp64 out. w_word (m, d) and w_ctx (mc, 2 d) are the MLPs' first layers as nn.Linear holds
 * them (w_ctx's first d columns act on e, its last d on e_prev); w_cq, w_ck (cf, d). d a multiple of 4, <= 1024;
 * m, mc, cf <= 64; the float4-read rows 16-byte aligned. workspace: asrn_decode_produce_workspace(B, m, mc) bytes. */
int64_t asrn_decode_produce_workspace(int64_t B, int32_t m, int32_t mc);
int asrn_decode_produce(const float* e, const float* e_prev, const float* h, const int64_t* pieza, int64_t B, int32_t d,
                        const float* w_v, const float* w_word, const float* w_ctx, const float* b_word,
                        const float* b_ctx, const float* w2_word, const float* b2_word, const float* w2_ctx,
                        const float* b2_ctx, int32_t m, int32_t mc, int32_t p_word, int32_t p_ctx, const float* ln_w,
                        const float* ln_b, float eps, const float* w_reloj, const float* b_reloj, float beta_max,
                        float log_alfa_min, const float* w_cq, const float* w_ck, int32_t cf, float* phi, float* V,
                        float* Qc, float* Kc, float* sig, float* log_alfa, int64_t cap, int64_t t,
                        const int64_t* t_dev, double* beta, void* workspace, int64_t workspace_bytes, void* stream);

/* decode_produce_e and decode_produce_h: asrn_decode_produce split by what the rows depend on, no counterpart in the
 * reference's FFI (its step runs each layer's producers in turn, asrn/nucleo.py:1797-1826). decode_produce_e writes,
 * for L layers at once (their pointers in host arrays of L; the layers share d, m, mc, p_word, p_ctx, the caches'
 * capacity cap and the position), what depends only on the new tokens' embedding rows e and e_prev and their ids:
 * V[t-1], phi[t] and sig[t]; the step can run it once, before its first layer. decode_produce_h then writes one
 * layer's Qc[t], Kc[t] and log_alfa[t] and its beta from that layer's input h. Together they write what
 * asrn_decode_produce writes, the same bits. workspace: asrn_decode_produce_e_workspace(L, B, m, mc) bytes. */
int64_t asrn_decode_produce_e_workspace(int32_t L, int64_t B, int32_t m, int32_t mc);
int asrn_decode_produce_e(int32_t L, const float* e, const float* e_prev, const int64_t* pieza, int64_t B, int32_t d,
                          const float* const* w_v, const float* const* w_word, const float* const* w_ctx,
                          const float* const* b_word, const float* const* b_ctx, const float* const* w2_word,
                          const float* const* b2_word, const float* const* w2_ctx, const float* const* b2_ctx,
                          int32_t m, int32_t mc, int32_t p_word, int32_t p_ctx, float* const* phi, float* const* V,
                          float* const* sig, int64_t cap, int64_t t, const int64_t* t_dev, void* workspace,
                          int64_t workspace_bytes, void* stream);
int asrn_decode_produce_h(const float* h, int64_t B, int32_t d, const float* ln_w, const float* ln_b, float eps,
                          const float* w_reloj, const float* b_reloj, float beta_max, float log_alfa_min,
                          const float* w_cq, const float* w_ck, int32_t cf, float* Qc, float* Kc, float* log_alfa,
                          int64_t cap, int64_t t, const int64_t* t_dev, double* beta, void* stream);
/* decode_produce_h on the output of a local block step left pending (asrn_block_step_ex with finish = 0; prev_*, its
 * arguments as asrn_block_step_ex takes them, prev_pos its position, workspace the one its call used): the layer input
 * is that block's output, formed here (h1 + the second feed-forward product + b2, written to prev_out, its z into its
 * ring) with the bits the block step's last kernel gives, then the producer's rows as asrn_decode_produce_h. h is
 * then not read. No counterpart in the reference: it saves the block step's last launch before every ASRN layer. */
int asrn_decode_produce_h_ex(const float* h, const float* prev_h1, const float* prev_b2, const float* prev_z,
                             float* prev_ring, int32_t prev_k, int32_t prev_ff, float* prev_out,
                             const int64_t* prev_pos, void* workspace, int64_t workspace_bytes, int64_t B, int32_t d,
                             const float* ln_w, const float* ln_b, float eps, const float* w_reloj,
                             const float* b_reloj, float beta_max, float log_alfa_min, const float* w_cq,
                             const float* w_ck, int32_t cf, float* Qc, float* Kc, float* log_alfa, int64_t cap,
                             int64_t t, const int64_t* t_dev, double* beta, void* stream);

/* ---- generation loop: n-gram sets and the per-token choice ------------------------------------------------------
 * The host side of escribir (asrn/nucleo.py:1965-2043) moved onto the device. The n-gram sets replace _Ngramas
 * (asrn/nucleo.py:1857-1889: Python dicts of token tuples, updated on the host after every token): per text row, an
 * open-addressing table `slots` of `cap` (a power of two) uint64 keys, all ones when empty, each key the n token ids of
 * an n-gram packed w = asrn_sample_bits(V) bits apiece (n * w <= 64), the oldest lowest; and a table of its contexts
 * (the first n - 1 ids, packed the same way): `ctx` (rows, cap) uint64, all ones when empty, `count` (rows, cap) int32,
 * zero to start, the number of distinct successors, and `succ` (rows, cap, asrn_ngram_set_successors()) int32, the
 * first of them.
 * asrn_sample_bits: the smallest w with 2^w - 1 > V - 1.
 * asrn_ngram_set_build: every n-gram of x (rows, L), row stride ldx, into row r's tables; L <= cap / 2. */
int32_t asrn_sample_bits(int64_t V);
int32_t asrn_ngram_set_successors(void);
int asrn_ngram_set_build(const int64_t* x, int64_t ldx, int64_t rows, int64_t L, int32_t n, int32_t w, uint64_t* slots,
                         uint64_t* ctx, int32_t* count, int32_t* succ, int64_t cap, void* stream);

/* asrn_sample replaces _frenar + _muestrear + _conservar_cita and the stop-token and bookkeeping lines of the
 * generation loop (asrn/nucleo.py:1909-1962, 2017-2036; there: a CPU multinomial and a .cpu() sync per token). Row b
 * of lg (B, V), stride ldl: penalty over text[pos - window, pos) (penalty != 1), bans from ban_slots (n-grams of the
 * generated tokens text[L0, pos), when pos - L0 >= ban_n; NULL: none) with the fallback to the plain logits when
 * nothing is left, the quote mask from quote_slots (when pos >= quote_n; NULL: none) and its mass at temperature 1,
 * temperature, top_k (0: none), top_p (>= 1: none), the softmax, the quote-mass correction, one draw by inverse CDF
 * from a uniform that is a function of (seed, b, pos), the stop token (< 0: none; done (B) uint8 and stop_step (B)
 * int32, -1 before, are kept). The token goes to tokens[b] and text[b * ld_text + pos], and its n-grams into both sets.
 * pos is read from *pos_dev at run time (so a captured step can advance it); a value outside [0, pos_max] writes
 * nothing, and pos_max < ld_text. work (B, V) fp32 and quote_bits (B, ceil(V/32)) are scratch; prob_out (B, V) gets
 * the final probabilities and logits_out (B, steps, V) the logits row at step pos - L0, when not NULL. */
int asrn_sample(const float* lg, int64_t ldl, float* work, uint32_t* quote_bits, float* prob_out, float* logits_out,
                int64_t steps, int64_t* text, int64_t ld_text, const int64_t* pos_dev, int64_t pos_max, int64_t L0,
                int64_t* tokens, uint8_t* done, int32_t* stop_step, uint64_t* quote_slots, uint64_t* quote_ctx,
                int32_t* quote_count, int32_t* quote_succ, int64_t quote_cap, int32_t quote_n, uint64_t* ban_slots,
                uint64_t* ban_ctx, int32_t* ban_count, int32_t* ban_succ, int64_t ban_cap, int32_t ban_n, int32_t w,
                int64_t B, int64_t V, float temperature, int32_t top_k, float top_p, float penalty, int32_t window,
                int64_t stop_token, uint64_t seed, void* stream);

/* ---- the model's local block, generation step -----------------------------------------------------------------
 * Replaces the local block's part of _Escritor.paso (asrn/nucleo.py:1811-1814: LayerNorm, the window cat, conv1d,
 * GELU, the adds, LayerNorm and the feed-forward layer, about a dozen launches per block) for mezcla 'conv' blocks
 * (BloqueLocal, nucleo:969-1014): out = h1 + W2 GELU(W1 LN2(h1) + b1) + b2 with h1 = h + GELU(conv([ring; LN1(h)])
 * + conv_b), for B rows h (stride ldh), fp32, in six launches (three products on the matrix cores in depth splits,
 * three row-wise kernels that prepare their operands and sum the splits in a fixed order). conv_w (d, d * k) is
 * nn.Conv1d's weight (d, d, k); w1 (ff, d), w2 (d, ff). ring (B, d, k - 1) holds LayerNorm1 of the k - 1 previous
 * positions, position t at slot t mod (k - 1); the step reads taps (pos + j) mod (k - 1) and writes LN1(h) at slot
 * pos mod (k - 1) (pos read from *pos at run time). z, h1, x2 (B, d) and x1 (B, d * k) are scratch outputs; out
 * (B, d). workspace: asrn_block_step_workspace(B, d, ff) bytes (the products' partial sums). */
int64_t asrn_block_step_workspace(int64_t B, int32_t d, int32_t ff);
int asrn_block_step(const float* h, int64_t ldh, float* ring, const int64_t* pos, int64_t B, int32_t d, int32_t k,
                    int32_t ff, const float* ln1_w, const float* ln1_b, const float* conv_w, const float* conv_b,
                    const float* ln2_w, const float* ln2_b, const float* w1, const float* b1, const float* w2,
                    const float* b2, float eps, float* z, float* x1, float* h1, float* x2, float* out,
                    void* workspace, int64_t workspace_bytes, void* stream);
/* block_step_ex: asrn_block_step for two blocks that follow each other (no layer between them), no counterpart in the
 * reference's FFI: the first block's last launch (its output and its ring's new row) is done by the second block's
 * first. finish = 0 leaves this block's output unfinished: out and the ring's row at pos are not written, and the
 * second feed-forward product's partials stay in the workspace. A call with prev_h1 != NULL then takes the input
 * from that pending block (the previous call, with this same workspace, B and d): its output prev_h1 + partials +
 * prev_b2 (in asrn_block_step's order) is formed here, written to prev_out (B, d) and used as h (h and ldh are then
 * ignored), and prev_z enters prev_ring at slot pos mod (prev_k - 1); prev_ff is its feed-forward width. Every
 * pending block must be taken by the next call. workspace: asrn_block_step_workspace(B, d, max(ff, prev_ff)). */
int asrn_block_step_ex(const float* h, int64_t ldh, const float* prev_h1, const float* prev_b2, const float* prev_z,
                       float* prev_ring, int32_t prev_k, int32_t prev_ff, float* prev_out, float* ring,
                       const int64_t* pos, int64_t B, int32_t d, int32_t k, int32_t ff, const float* ln1_w,
                       const float* ln1_b, const float* conv_w, const float* conv_b, const float* ln2_w,
                       const float* ln2_b, const float* w1, const float* b1, const float* w2, const float* b2,
                       float eps, float* z, float* x1, float* h1, float* x2, float* out, int32_t finish,
                       void* workspace, int64_t workspace_bytes, void* stream);
/* A block step left pending (asrn_block_step_ex with finish = 0; prev_*, its arguments, pos its position, workspace the
 * one its call used) finished, then the model's final LayerNorm (ln_w, ln_b, eps; biased variance) of its output into
 * y (B, d): the block's output (written to prev_out) and ring row with the bits its last kernel gives. pos_next: null,
 * or where *pos + 1 is stored once every workgroup has used *pos (it may be pos itself; a generation loop step's
 * advance), with done a device int32 holding 0, kept by the caller across calls (each launch leaves it 0); calls
 * sharing one done must not overlap. No counterpart in the reference: one launch for the last block's end, the final
 * norm and the position's advance (nucleo:1854). */
int asrn_block_finish_norm(const float* prev_h1, const float* prev_b2, const float* prev_z, float* prev_ring,
                           int32_t prev_k, int32_t prev_ff, float* prev_out, const int64_t* pos, int64_t B, int32_t d,
                           const float* ln_w, const float* ln_b, float eps, float* y, void* workspace,
                           int64_t workspace_bytes, int64_t* pos_next, int32_t* done, void* stream);

/* ---- the model's loss: cross-entropy ---------------------------------------------------------------------------
 * Replaces F.cross_entropy(logits.float().reshape(-1, V), y.reshape(-1), ignore_index) of ModeloASRN.perdida and the
 * training loop (asrn/nucleo.py:1108, 2301): the same fp32 arithmetic on fp32 or bf16 logits (logits_bf16), without
 * the fp32 copy of the logits. logits (rows, V) with row stride ld (16-byte aligned rows), target (rows) int64.
 * fwd: lse (rows) = logsumexp of the row, loss (rows) = lse - logits[target] (0 where target == ignore_index, NaN
 * for a target outside [0, V)); the caller reduces the rows (mean over the rows not ignored, or sum).
 * bwd: dlogits (rows, V), row stride ldd, in the logits' dtype = (softmax - onehot(target)) * *scale (scale a device
 * float: d loss / count for the mean), 0 for ignored rows; bf16 rounded to nearest even. */
int asrn_cross_entropy_fwd(const void* logits, int32_t logits_bf16, int64_t ld, const int64_t* target, int64_t rows,
                           int64_t V, int64_t ignore_index, float* lse, float* loss, void* stream);
int asrn_cross_entropy_bwd(const void* logits, int32_t logits_bf16, int64_t ld, const int64_t* target,
                           const float* lse, int64_t rows, int64_t V, int64_t ignore_index, const float* scale,
                           void* dlogits, int64_t ldd, void* stream);

/* ---- the model's local block: the causal convolution's columns ----------------------------------------------
 * Replaces F.pad + unfold + reshape of the 'conv' BloqueLocal's convolution (asrn/nucleo.py:969-1014, nn.Conv1d over
 * the left-padded sequence) and the cast of those columns to the autocast dtype. fwd: z (B, L, d) fp32, row stride
 * ldz -> cols (B, L, d * k) with cols[b, t, c * k + j] = z[b, t + j - (k - 1), c] (0 before the row's start), in
 * fp32 or bf16 (cols_bf16, rounded to nearest even), 16-byte aligned. bwd: dcols (B, L, d * k) of that dtype ->
 * dz (B, L, d) fp32, row stride lddz: dz[b, s, c] = sum over j (ascending) of dcols[b, s + k - 1 - j, c * k + j]
 * (windows inside the row). 1 <= k <= 16. */
int asrn_conv_window_fwd(const float* z, int64_t ldz, int64_t B, int64_t L, int32_t d, int32_t k, int32_t cols_bf16,
                         void* cols, void* stream);
int asrn_conv_window_bwd(const void* dcols, int32_t cols_bf16, int64_t B, int64_t L, int32_t d, int32_t k, float* dz,
                         int64_t lddz, void* stream);

/* ---- the model's LayerNorms ------------------------------------------------------------------------------------
 * Replaces torch.nn.LayerNorm of the local blocks (ln1, ln2) and the final ln_f (asrn/nucleo.py:969-1014,
 * 1047-1125) as it runs in fp32 under autocast, with the cast of its output to bf16 for the next product, and, in the
 * backward, the residual path's gradient addition. fwd: x (rows, d) fp32, row stride ldx -> y = (x - mean) rstd gamma
 * + beta (biased variance, rstd = 1 / sqrt(var + eps)) in fp32 or bf16 (out_bf16, rounded to nearest even), row
 * stride ldy, and stats (rows, 2) = (mean, rstd). bwd: from dy (fp32 or bf16, row stride lddy) -> dx (rows, d) fp32,
 * row stride ldx (overwritten; plus dres (rows, d), row stride ldx, when not null), and dparams (2 d) = [d gamma |
 * d beta] summed over rows in a fixed order. d a multiple of 4, <= 1024; rows 16-byte aligned (8 for bf16).
 * workspace: asrn_layer_norm_bwd_workspace(rows, d) bytes, 256-byte aligned. */
int asrn_layer_norm_fwd(const float* x, int64_t ldx, const float* gamma, const float* beta, int64_t rows, int32_t d,
                        float eps, int32_t out_bf16, void* y, int64_t ldy, float* stats, void* stream);
int64_t asrn_layer_norm_bwd_workspace(int64_t rows, int32_t d);
int asrn_layer_norm_bwd(const float* x, int64_t ldx, const float* gamma, const float* stats, int64_t rows, int32_t d,
                        const void* dy, int32_t dy_bf16, int64_t lddy, const float* dres, float* dx, float* dparams,
                        void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ASRN_HIP_H */
