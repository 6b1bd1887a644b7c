/*
 * mingru_hip.h — C ABI of libmingru_hip.so, the MI355X (gfx950) kernels behind
 * the minGRU / minLM training step.
 *
 * Conventions (every entry point):
 *   - Plain pointers to device memory, element counts and strides in ELEMENTS.
 *     No framework types cross this boundary.
 *   - `stream` is a hipStream_t passed as void* (NULL = legacy default stream).
 *     All work is enqueued on it; nothing synchronises the host.
 *   - The library never allocates device memory. Scratch space ("workspace")
 *     is passed in by the caller; its size comes from the matching
 *     *_workspace_bytes() query. A workspace must not be shared by two calls
 *     that may run concurrently.
 *   - Return 0 on success, a nonzero MG_ERR_* code otherwise; the message of
 *     the last failure on the calling thread is returned by mg_last_error().
 *   - dtype codes: MG_F32 = 0 (float), MG_BF16 = 1 (bfloat16).
 *   - Rounding to bf16: round-to-nearest-even for activations and weights.
 *     Gradients written in bf16 (mg_scan_bwd's dhidden/dgate,
 *     mg_add_rmsnorm_bwd's ddelta, the loss heads' dlogits, mg_gelu_bwd's
 *     dpre, mg_gemm's GELU-gradient epilogue) round stochastically: up with
 *     probability equal to the dropped fraction of a bf16 ulp, from a hash of
 *     the element's index and value (deterministic, no generator state).
 *     Round-to-nearest errors of a near-uniform softmax's gradient repeat
 *     across the rows of a label and add up in the weight gradients;
 *     stochastic rounding keeps them unbiased.
 */
#ifndef MINGRU_HIP_H
#define MINGRU_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MG_F32 0
#define MG_BF16 1

#define MG_OK 0
#define MG_ERR_ARG 1      /* bad shape, stride, alignment or null pointer */
#define MG_ERR_DTYPE 2    /* unsupported dtype combination */
#define MG_ERR_WORKSPACE 3 /* workspace missing, too small or not initialised */
#define MG_ERR_HIP 4      /* a HIP runtime call or kernel launch failed */
#define MG_ERR_STALL 5    /* a scan's look-back wait gave up (see mg_scan_workspace_check) */

/* Library version (major*10000 + minor*100 + patch): 206 = 0.2.6, the ABI
 * declared in this file (0.2.1 to 0.2.5 add entry points to 0.2.0 and change
 * none; 0.2.6 changes no signature: mg_gemm also splits small bf16 products
 * along K, see mg_gemm). */
int mg_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* mg_last_error(void);

/* ------------------------------------------------------------------------
 * Gate math + log-space associative scan (minGRU parallel path).
 *
 * Replaces, for seq_len > 1, reference mingru/minGRU.py:53-69:
 *   log_coeffs = -softplus(gate)                       (:56)
 *   log_values = -softplus(-gate) + log_g(hidden)      (:58-60, log_g :27-28)
 *   optional prev_hidden seeding (cat/pad)             (:62-64)
 *   heinsen_associative_scan_log(...)                  (:16-20, called :66)
 *   out[:, -seq_len:], next_prev_hidden = out[:, -1:]  (:67, :69)
 * and, for seq_len == 1, the sequential lerp path     (:47-52)
 * (a scan of length one is that lerp).
 *
 * Computes h_t = a_t h_{t-1} + z_t g(hidden_t), z_t = sigmoid(gate_t),
 * a_t = 1 - z_t, g(x) = x + 0.5 (x >= 0) | sigmoid(x) (x < 0), h_{-1} = h0
 * (or 0 when h0 is NULL), in fp32, for every (b, d) channel.
 *
 * Layout: element (b, t, d) of hidden/gate is at  b*in_sb + t*in_ld + d,
 *         of h at b*out_sb + t*out_ld + d. h0, h_last: dense [B, Di] fp32.
 *   The two column halves of the to_hidden_and_gate output [B, T, 2*Di]
 *   are passed as hidden = base, gate = base + Di, in_ld = 2*Di,
 *   in_sb = T*2*Di.
 * Requirements: Di % 4 == 0, strides % 4 == 0, pointers 8-byte aligned
 *   (bf16) or 16-byte aligned (fp32), 128 * row stride < 2^31.
 * h_last (nullable): fp32 [B, Di], receives h_{T-1}.
 * ckpt (nullable): fp32 [ceil(T/8), B, Di]; ckpt[j] receives h_{8j+7}, the
 *   state entering step 8j+8. mg_scan_bwd reads it instead of h when h is
 *   bf16 (required there for fp32-accurate gradients).
 * Supported (in_dtype, out_dtype): (BF16, BF16), (F32, F32), (BF16, F32).
 * ---------------------------------------------------------------------- */
size_t mg_scan_ckpt_elems(int B, int T, int Di);

/* Look-back workspace (a header, ticket counters and look-back words; serves
 * both directions). mg_scan_workspace_init zero-fills it on `stream` and
 * writes the header for one (B, T, Di); the kernels then keep it consistent
 * from call to call, so calls do no clearing of their own.
 *
 * One stream per workspace: the calls on a workspace must run one after the
 * other (one stream, or ordered by events). Calls that may overlap need
 * separate workspaces. The library keeps no record of workspaces: each
 * kernel checks the header on the device. A workspace that was never
 * initialised, was initialised for another shape, or was corrupted (for
 * instance by overlapping calls) makes the kernel exit early. A look-back
 * wait that stays unanswered for max_polls polls gives up. Either way the
 * results are invalid and a bit is set in the header's error word, which
 * mg_scan_workspace_check reads: it synchronises `stream` and returns
 * MG_OK, MG_ERR_WORKSPACE (uninitialised or wrong shape), MG_ERR_STALL (a
 * wait gave up; corrupted counters end this way, sometimes also drawing a
 * ticket past the last tile) or MG_ERR_WORKSPACE for such a ticket alone.
 * The error stays until the workspace is
 * initialised again. mg_scan_workspace_set_max_polls changes the poll limit
 * (default 2^22 polls, about a second; at least 1), on `stream`. */
size_t mg_scan_workspace_bytes(int B, int T, int Di);
int mg_scan_workspace_init(void* workspace, size_t workspace_bytes, int B, int T, int Di, void* stream);
int mg_scan_workspace_set_max_polls(void* workspace, uint32_t max_polls, void* stream);
int mg_scan_workspace_check(const void* workspace, void* stream);

/* Asynchronous form of mg_scan_workspace_check, for a training loop that
 * must not synchronise every step: enqueues on `stream` one single-thread
 * kernel that ORs the workspace header's error bits (1 = missing header or
 * another shape, 2 = a ticket past the last tile, 4 = a wait gave up) into
 * *host_word, which must be pinned host memory (hipHostMalloc). The word is
 * written only when a bit is set; the caller clears it and reads it at any
 * later point (after the stream has passed the poll, e.g. at its next
 * synchronisation), then calls mg_scan_workspace_check for the message.
 * Same purpose as mg_scan_workspace_check (the error convention of the
 * scan calls, which replace reference mingru/minGRU.py:16-20,53-69); no
 * reference counterpart of its own. */
int mg_scan_workspace_poll(const void* workspace, uint32_t* host_word, void* stream);

int mg_scan_fwd(int in_dtype, const void* hidden, const void* gate,
                int64_t in_sb, int64_t in_ld,
                const float* h0,
                int out_dtype, void* h, int64_t out_sb, int64_t out_ld,
                float* h_last, float* ckpt,
                int B, int T, int Di,
                void* workspace, size_t workspace_bytes, void* stream);

/* mg_scan_fwd with the scan state joining the residual stream (the minGRU
 * branch of reference mingru/minLM.py:121-125 at expansion 1, where the
 * minGRU output is h itself): x_out = res + h, fp32, with res and x_out at
 * (out_sb, out_ld); h itself is not written, only its fp32 checkpoints
 * (ckpt, required: mg_scan_ckpt_elems(B, T, Di) floats), from which
 * mg_scan_bwd (called with h = NULL and this ckpt) rebuilds it. h0, h_last,
 * the workspace and the errors as for mg_scan_fwd; in_dtype MG_BF16 or
 * MG_F32. res and x_out may be the same buffer. */
int mg_scan_fwd_residual(int in_dtype, const void* hidden, const void* gate, int64_t in_sb, int64_t in_ld,
                         const float* h0, const float* res, float* x_out, int64_t out_sb, int64_t out_ld,
                         float* h_last, float* ckpt, int B, int T, int Di, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Allocation-free mg_scan_fwd. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same arguments and
 * results as mg_scan_fwd without the workspace: the look-back scratch is a
 * file-scope device array of mg_scan_fwd_noalloc_max_bytes() bytes (16 MiB +
 * 64 KiB; each device the library runs on holds its own copy until the
 * process ends), re-initialised on `stream` by a kernel at every call (no
 * memset). Shapes needing more look-back scratch than that (more than ~2 M
 * channel-tiles: B * Di * ceil(T / 128) > 2^21, e.g. cfg2's B16 T8192 Di2048
 * fits exactly) are refused with MG_ERR_ARG. It calls no hipMalloc, hipFree
 * or allocating library routine. All calls on one device share the array:
 * calls that may overlap on one device race. */
size_t mg_scan_fwd_noalloc_max_bytes(void);
int mg_scan_fwd_noalloc(int in_dtype, const void* hidden, const void* gate,
                        int64_t in_sb, int64_t in_ld,
                        const float* h0,
                        int out_dtype, void* h, int64_t out_sb, int64_t out_ld,
                        float* h_last, float* ckpt,
                        int B, int T, int Di, void* stream);

/* The error word of the allocation-free scratch, as mg_scan_workspace_check
 * reports a workspace's: synchronises `stream`, reads the scratch header of
 * the current device and returns MG_OK, MG_ERR_WORKSPACE or MG_ERR_STALL for
 * the last mg_scan_fwd_noalloc call on this device (each call re-initialises
 * the header, so earlier calls' errors are gone). Allocates nothing. No
 * counterpart in the reference: for the same callers as mg_scan_fwd_noalloc. */
int mg_scan_fwd_noalloc_check(void* stream);

/* Backward of mg_scan_fwd: autograd of reference mingru/minGRU.py:16-20,
 * :53-69 through gate, hidden and prev_hidden, in closed form:
 *   lambda_t  = dh_t + a_{t+1} lambda_{t+1},
 *   dgate_t   = lambda_t z_t (1 - z_t) (g(hidden_t) - h_{t-1}),
 *   dhidden_t = lambda_t z_t g'(hidden_t)   (g'(0) = 0, as relu'(0) = 0),
 *   dh0       = a_0 lambda_0.
 * h: the forward's output (same layout, dtype out_dtype); NULL when ckpt is
 * given (then out_dtype only sets dh's dtype). h_{t-1} is read once per 8
 * steps from ckpt when given (the forward's fp32 checkpoints), else once per
 * 4 steps from h, and rebuilt in fp32 in between.
 * dh: gradient of h, dtype out_dtype, element (b,t,d) at b*g_sb + t*g_ld + d.
 * dh_last (nullable): fp32 [B, Di], gradient of h_last, added to dh_{T-1}.
 * dhidden/dgate: dtype in_dtype, element (b,t,d) at b*d_sb + t*d_ld + d
 *   (for the packed [B, T, 2*Di] gradient buffer: dhidden = base,
 *   dgate = base + Di, d_ld = 2*Di, d_sb = T*2*Di). The caller's buffers
 *   must hold every element so addressed.
 * dh0 (nullable): fp32 [B, Di]. */
int mg_scan_bwd(int in_dtype, const void* hidden, const void* gate,
                int64_t in_sb, int64_t in_ld,
                const float* h0,
                int out_dtype, const void* h, int64_t out_sb, int64_t out_ld,
                const float* ckpt,
                const void* dh, int64_t g_sb, int64_t g_ld,
                const float* dh_last,
                void* dhidden, void* dgate, int64_t d_sb, int64_t d_ld, float* dh0,
                int B, int T, int Di,
                void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Fused residual add + RMSNorm (pre-norm blocks of minLM).
 *
 * Replaces reference mingru/minLM.py:119-125 (norm(x) before minGRU and the
 * residual add after it), :130 (ff_norm(x), residual add), :137 (final
 * norm), with torch.nn.RMSNorm(dim) (:67, :69, :74): y = x * w /
 * sqrt(mean(x^2) + eps). The reference's eps=None means torch.finfo(fp32).eps
 * = 2^-23 for its fp32 activations; callers pass that eps.
 *
 * Rows of D contiguous elements (D % 4 == 0, D <= 4096), N rows.
 * Forward:  xn = x + delta (delta nullable: xn = x, x_out unused),
 *           x_out = xn (fp32), y = xn * rstd * w (y_dtype), rstd[row] (nullable).
 *           y and y_lo rows have stride ldy (>= D, % 4 == 0). y_lo (nullable,
 *           bf16 y only) receives bf16(y_fp32 - y): with y it forms a hi/lo
 *           pair equal to the fp32 value to ~2^-16 relative, the operand
 *           form of mg_gemm's MG_GEMM_HILO products.
 * Backward: dx = rstd * (dy*w - xn*rstd * mean(dy*w * xn*rstd)) + dres
 *           (dres nullable), written to dx (fp32, nullable) and to ddelta
 *           (ddelta_dtype, nullable); dw = sum over rows of dy * xn * rstd
 *           (written, not accumulated). xn is the forward's x_out (or x when
 *           the forward had no delta). workspace: fp32 partial rows,
 *           mg_add_rmsnorm_bwd_workspace_bytes(N, D) bytes.
 * ---------------------------------------------------------------------- */
int mg_add_rmsnorm_fwd(const float* x, int delta_dtype, const void* delta,
                       const float* w, float* x_out, int y_dtype, void* y,
                       void* y_lo, int64_t ldy,
                       float* rstd, int64_t N, int D, float eps, void* stream);

size_t mg_add_rmsnorm_bwd_workspace_bytes(int64_t N, int D);

int mg_add_rmsnorm_bwd(const float* xn, const float* w, const float* rstd,
                       int dy_dtype, const void* dy, const float* dres,
                       float* dx, int ddelta_dtype, void* ddelta, float* dw,
                       int64_t N, int D, void* workspace,
                       size_t workspace_bytes, void* stream);

/* mg_add_rmsnorm_bwd with dy multiplied by the fp32 device scalar *dy_scale
 * (NULL: 1) as it is loaded: the upstream gradient of a loss (reference
 * train.py:800, (loss / grad_accum).backward()) applied without a separate
 * pass over dy; results equal scaling dy in fp32 first. */
int mg_add_rmsnorm_bwd_scaled(const float* xn, const float* w, const float* rstd,
                              int dy_dtype, const void* dy, const float* dy_scale,
                              const float* dres, float* dx, int ddelta_dtype,
                              void* ddelta, float* dw, int64_t N, int D,
                              void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Cross-entropy loss head, forward and gradient in one pass.
 *
 * Replaces reference mingru/minLM.py:146-149 (F.cross_entropy over the
 * transposed logits, mean reduction) and its autograd backward (log-softmax
 * backward). logits: [N, V] row-major (fp32 or bf16), labels: int64 [N].
 * Writes dlogits ([N, V], fp32 or bf16) = (softmax(logits) - onehot(label)) * scale
 * and loss_part[p] = sum of the per-row losses of partition p, for
 * p < mg_cross_entropy_partials(N) (mean loss = sum(loss_part) / N).
 * bad_label (nullable, int, zeroed by the caller): set to 1 if a label is
 * outside [0, V). V % 4 == 0, V <= 1024.
 * ---------------------------------------------------------------------- */
int mg_cross_entropy_partials(int64_t N);
int mg_cross_entropy_fwd_bwd(int logits_dtype, const void* logits,
                             const int64_t* labels, int dlogits_dtype,
                             void* dlogits, float* loss_part, int* bad_label,
                             int64_t N, int V, float scale, void* stream);

/* ------------------------------------------------------------------------
 * Schedule-Free AdamW step over many parameter tensors in one launch.
 *
 * Replaces schedulefree.AdamWScheduleFree.step (called at reference
 * train.py:808; package pinned at requirements.txt:44) in train mode, per
 * element, with y = the parameter, z the base iterate, v the second moment:
 *   v <- beta2 v + (1 - beta2) g^2
 *   u  = g / (sqrt(v / bias_correction2) + eps) + weight_decay * y
 *   y <- (1 - ckp1) y + ckp1 z + y_lr u;   z <- z - lr u
 * and, when p_bf16 is set, p_bf16 <- bf16(y). The scalars (ckp1 = c_{k+1},
 * y_lr = lr (beta1 (1 - ckp1) - 1), bias_correction2 = 1 - beta2^(k+1)) are
 * the package's per-step values, computed by the caller in double precision
 * (one_minus_beta2 too: 1 - 0.999 rounded once, as the package's addcmul
 * value, not 1 - fp32(0.999)).
 * tensors: device array of ntensors mg_sf_tensor; tensor t owns chunks
 * [chunk_start_t, chunk_start_{t+1}) of mg_sf_adamw_chunk_elems() elements;
 * nchunks = the total.
 * ---------------------------------------------------------------------- */
typedef struct mg_sf_tensor {
  float* p;
  const float* g;
  float* z;
  float* v;
  uint16_t* p_bf16; /* nullable: bf16 copy of p, written with it */
  int64_t n;
  int64_t chunk_start;
  /* 0: p_bf16 is a dense bf16 copy [n]. C > 0 (C % 4 == 0, n % C == 0, n < 2^31): p
   * viewed as [n / C, C] and p_bf16 its hi/lo pair [n / C, 2 C] (row r:
   * hi = bf16(p[r, :]) then lo = bf16(p[r, :] - hi), as mg_split_hilo
   * writes it), the operand form of the fp32-accurate products. */
  int64_t pair_cols;
} mg_sf_tensor;

int64_t mg_sf_adamw_chunk_elems(void);
int mg_sf_adamw_step(const void* tensors, int ntensors, int64_t nchunks,
                     float beta2, float one_minus_beta2,
                     float bias_correction2, float eps, float weight_decay,
                     float ckp1, float y_lr, float lr, void* stream);

/* ------------------------------------------------------------------------
 * bf16 matrix product on MFMA with fp32 accumulation, plus fused epilogues.
 *
 * Replaces the nn.Linear products of the hot path and their autograd
 * backward: to_hidden_and_gate (reference mingru/minGRU.py:45), to_out
 * (:71), the FeedForward Linear-GELU-Linear (mingru/minLM.py:17-23, :130)
 * and to_logits (mingru/minLM.py:75, :138).
 *
 *   C[m, n] (=|+=) epilogue( sum_k A(m, k) B(k, n) ),  0 <= m < M, n < N, k < K
 * Operand layouts (bf16):
 *   MG_KCONTIG : element (row, k) at p + row * ld + k  (A = X [M, K]; B = W [N, K])
 *   MG_MNCONTIG: element (row, k) at p + k * ld + row  (A = dY as dY^T; B = X as X^T)
 * so Y = X W^T is (A = X, KCONTIG; B = W, KCONTIG), dX = dY W is
 * (A = dY, KCONTIG; B = W, MNCONTIG) and dW = dY^T X is (A = dY, MNCONTIG;
 * B = X, MNCONTIG) with K = number of rows (tokens).
 * C: [M, N] row-major (ldc), fp32 or bf16 (RNE).
 * Epilogues:
 *   MG_EPI_NONE       C = acc
 *   MG_EPI_BIAS       C = acc + bias[n]                   (bias fp32 [N])
 *   MG_EPI_BIAS_GELU  aux = bf16(acc + bias[n]); C = gelu(aux)   (bf16 C, aux [M, N] bf16, ldaux)
 *   MG_EPI_GELU_GRAD  C = acc * gelu'(aux[m][n])                  (bf16 C, aux as written above)
 *   gelu(x) = x/2 (1 + erf(x/sqrt(2))), nn.GELU()'s exact form.
 * flags (bit set):
 *   MG_GEMM_ACCUMULATE (fp32 C, no epilogue): C += A B.
 *   MG_GEMM_DETERMINISTIC: never split along K.
 *   MG_GEMM_STOCHASTIC: a bf16 C (epilogue NONE) is rounded stochastically,
 *     as gradients are (see the conventions above); the GELU-gradient
 *     epilogue always is.
 *   MG_GEMM_HILO: fp32-accurate product of operands stored as bf16 hi/lo
 *     pairs. A and B must both be K-contiguous; each row holds K hi values
 *     followed by K lo values (x = hi + lo; lda, ldb >= 2K), as written by
 *     mg_add_rmsnorm_fwd's y/y_lo or mg_split_hilo. Computes
 *     A_hi B_hi + A_lo B_hi + A_hi B_lo in fp32 (three times the MFMA work;
 *     the dropped A_lo B_lo term is ~2^-16 relative). Used where bf16
 *     rounding of a product would move a result across the kink of the
 *     reference's g(x) at 0 (the hidden half of to_hidden_and_gate, to_out).
 * Split along K: products with few output tiles (fp32 outputs with no
 *   epilogue; bf16 outputs with none or MG_EPI_BIAS, not hi/lo) are split along
 *   K over several workgroups when a workspace is given. Each writes its fp32
 *   partial tile there and a second kernel adds the partials, in split order,
 *   into C (plus C's old value when accumulating; plus the bias, then one
 *   rounding to bf16, nearest or stochastic as the flags ask), so results
 *   repeat bit for bit either way (split and unsplit sums differ in order).
 *   workspace: mg_gemm_workspace_bytes(...) bytes (0: the product never
 *   splits), 16-byte aligned; NULL runs unsplit. Calls sharing a workspace
 *   must be ordered on one stream.
 * Kernel choice (results do not depend on it): bf16 outputs with more
 *   256 x 256 tiles than CUs run one persistent workgroup per CU; K-split
 *   products lay their workgroups out so that each XCD's share one split.
 *   MG_GEMM_PERSIST=0 / MG_GEMM_XCD_SPLIT=0 in the environment turn these
 *   off (read per call).
 * Requirements: N % 8 == 0; K % 8 == 0 if an operand is K-contiguous;
 *   M % 8 == 0 if A is MN-contiguous; lda, ldb, ldaux % 8 == 0; ldc % 8 == 0
 *   (bf16 C) or % 4 == 0 (fp32 C); A, B, C, bias, aux 16-byte aligned; each
 *   operand spans less than 2 GiB.
 * ---------------------------------------------------------------------- */
#define MG_KCONTIG 0
#define MG_MNCONTIG 1
#define MG_EPI_NONE 0
#define MG_EPI_BIAS 1
#define MG_EPI_BIAS_GELU 2
#define MG_EPI_GELU_GRAD 3
#define MG_GEMM_ACCUMULATE 1
#define MG_GEMM_DETERMINISTIC 2
#define MG_GEMM_HILO 4
#define MG_GEMM_STOCHASTIC 8

int mg_gemm(int a_layout, const void* A, int64_t lda,
            int b_layout, const void* B, int64_t ldb,
            int M, int N, int K,
            int epilogue, const float* bias, void* aux, int64_t ldaux,
            int c_dtype, void* C, int64_t ldc, int flags,
            void* workspace, size_t workspace_bytes, void* stream);
/* C[m, n] = sum_k A(m, k) B(n, k) for K-contiguous hi/lo pairs A [M, 2K] and
 * B [N, 2K] (rows [hi (K) | lo (K)], lda, ldb >= 2K), bf16 C [M, N]: the
 * columns n < hilo_cols to fp32 accuracy (A_hi B_hi + A_lo B_hi + A_hi B_lo,
 * as MG_GEMM_HILO), the others from the hi halves alone (A_hi B_hi), in one
 * persistent launch. It is the forward of reference mingru/minGRU.py:45
 * (to_hidden_and_gate) with the hidden half accurate and the gate half a
 * plain bf16 product, where two mg_gemm calls would each fill and drain the
 * pipeline. K % 128 == 0, N % 8 == 0, hilo_cols a multiple of 256 below N,
 * leading dimensions multiples of 8, 16-byte aligned operands. */
int mg_gemm_hilo_prefix(const void* A, int64_t lda, const void* B, int64_t ldb, int M, int N, int K, int hilo_cols,
                        void* C, int64_t ldc, void* stream);
size_t mg_gemm_workspace_bytes(int a_layout, int b_layout, int M, int N, int K, int epilogue,
                               int c_dtype, int flags);

/* Two weight gradients over the same K rows in one launch: the autograd of
 * the FeedForward's two nn.Linear weights (reference mingru/minLM.py:17-23,
 * :130), dW_i = dY_i^T X_i, i.e. mg_gemm(MG_MNCONTIG, dy_i, ld_dy_i,
 * MG_MNCONTIG, x_i, ld_x_i, M_i, N_i, K, MG_EPI_NONE, ..., MG_F32, dw_i,
 * ldc_i, flags, ...) for i = 0, 1 (dy_i [K, M_i], x_i [K, N_i]; dw_i fp32,
 * written, or added with MG_GEMM_ACCUMULATE). When both have at least 16
 * 256 x 256 tiles and fewer than one per CU together, they share one K-split
 * launch. Each product then has half the splits it would have alone, and
 * half the partial tiles are written and summed. Otherwise each product
 * runs alone, as mg_gemm. Results repeat bit for bit (the sum order depends
 * on the shapes only). flags: MG_GEMM_ACCUMULATE, MG_GEMM_DETERMINISTIC
 * (the products then run alone, unsplit). workspace:
 * mg_gemm_wgrad_pair_workspace_bytes(...) bytes, 16-byte aligned (NULL: alone,
 * unsplit). Requirements as mg_gemm's for these layouts. */
int mg_gemm_wgrad_pair(const void* dy0, int64_t ld_dy0, const void* x0, int64_t ld_x0, int M0, int N0,
                       float* dw0, int64_t ldc0,
                       const void* dy1, int64_t ld_dy1, const void* x1, int64_t ld_x1, int M1, int N1,
                       float* dw1, int64_t ldc1, int K, int flags,
                       void* workspace, size_t workspace_bytes, void* stream);
size_t mg_gemm_wgrad_pair_workspace_bytes(int M0, int N0, int M1, int N1, int K, int flags);

/* fp32 -> bf16 hi/lo pairs for MG_GEMM_HILO operands: out[r, c] =
 * bf16(x[r, c]) (RNE), out[r, cols + c] = bf16(x[r, c] - out[r, c]), for
 * rows x cols (cols % 4 == 0; ldx >= cols, ldo >= 2 cols, both % 4 == 0;
 * x 16-byte and out 8-byte aligned). No reference counterpart: it prepares
 * the operands of the accurate forms of reference mingru/minGRU.py:45 and :71. */
int mg_split_hilo(const float* x, int64_t ldx, int64_t rows, int cols, void* out, int64_t ldo, void* stream);

/* fp32 -> three bf16 limbs per value: h = bf16(x), m = bf16(x - h), l =
 * bf16(x - h - m) (h + m + l == x; the differences are exact in fp32),
 * written as nseg (1..8) segments, segment s holding limb (pattern >> 2s) & 3
 * (0 h, 1 m, 2 l). stack_rows 0: the segments side by side along the
 * columns, out[r, s cols + c] (ldo >= nseg cols), the form of a K-contiguous
 * operand whose K grows nseg-fold; 1: stacked along the rows, out[s rows + r,
 * c] (ldo >= cols), the form of an MN-contiguous one. Operands split with the
 * patterns (h, m, h, m, l, h) and (h, h, m, m, h, l) make one plain mg_gemm
 * product over 6K equal to the fp32 product to ~2^-24 relative (the six limb
 * products through 2^-16). rows x cols with cols % 4 == 0; ldx, ldo % 4 == 0;
 * x 16-byte and out 8-byte aligned. No reference counterpart: it prepares
 * the operands of the fp32 nn.Linear products (reference mingru/minGRU.py:45,
 * :71, mingru/minLM.py:17-23, :138 in fp32). */
int mg_split_limbs(const float* x, int64_t ldx, int64_t rows, int cols, int pattern, int nseg, int stack_rows,
                   void* out, int64_t ldo, void* stream);

/* fp32 -> bf16 with stochastic rounding (as the gradient stores, keyed by the
 * element index and `salt`), n % 4 == 0 dense elements; x 16-byte and out
 * 8-byte aligned. For an fp32 gradient that must enter a bf16 product (the
 * backward of to_out, reference mingru/minGRU.py:71). */
int mg_round_bf16_sr(const float* x, int64_t n, void* out, uint32_t salt, void* stream);

/* ------------------------------------------------------------------------
 * Streaming loss head: logits GEMM + log-softmax + cross-entropy + gradient.
 *
 * Replaces reference mingru/minLM.py:138 (to_logits) and :146-149
 * (F.cross_entropy over the transposed logits, mean reduction) with its
 * backward through the logits, without writing the logits:
 *   logits = E W^T          E: bf16 [N, D] (lde), W: bf16 [V, D] (ldw)
 *   loss_part[b]  = sum over the rows of block b of (lse_n - logits[n, label_n])
 *   dlogits[n, j] = (softmax(logits_n)_j - [j == label_n]) * scale   (bf16, ldd)
 * Mean loss = sum(loss_part) / N with scale = 1/N; loss_part holds
 * mg_logits_cross_entropy_partials(N) values (one per 64 rows).
 * bad_label (nullable, zeroed by the caller) is set to 1 for a label outside
 * [0, V). Requirements: D % 8 == 0, 8 <= V <= 256, V % 8 == 0, lde, ldw % 8
 * == 0, ldd % 4 == 0, E and W 16-byte aligned, labels int64.
 * ---------------------------------------------------------------------- */
int mg_logits_cross_entropy_partials(int64_t N);
int mg_logits_cross_entropy(const void* embed, int64_t lde, const void* w, int64_t ldw,
                            const int64_t* labels, void* dlogits, int64_t ldd,
                            float* loss_part, int* bad_label, int N, int D, int V,
                            float scale, void* stream);

/* ------------------------------------------------------------------------
 * Bias gradients of the FeedForward linears (reference mingru/minLM.py:17-23:
 * autograd of nn.Linear's bias and of nn.GELU), over N token rows.
 *
 * mg_column_sum: out[c] = sum_n x[n, c]  (x fp32 or bf16, row stride ld;
 *   out fp32 [C], written).
 * mg_gelu_bwd:   dpre[n, c] = bf16(dh[n, c] * gelu'(pre[n, c])) (dh fp32 or
 *   bf16 per dh_dtype, pre and dpre bf16, gelu(x) = x/2 (1 + erf(x/sqrt 2))),
 *   and when dbias is given, dbias[c] = sum_n dpre[n, c] (of the bf16
 *   values; fp32 [C], written).
 * Both sum in a fixed order (reproducible) through a workspace of
 * mg_column_sum_workspace_bytes(N, C) bytes. C % 8 == 0, strides % 8 == 0,
 * 16-byte aligned pointers.
 * ---------------------------------------------------------------------- */
size_t mg_column_sum_workspace_bytes(int64_t N, int C);
int mg_column_sum(int dtype, const void* x, int64_t ld, int64_t N, int C, float* out,
                  void* workspace, size_t workspace_bytes, void* stream);
int mg_gelu_bwd(int dh_dtype, const void* dh, int64_t ld_dh, const void* pre, int64_t ld_pre,
                void* dpre, int64_t ld_out, float* dbias, int64_t N, int C,
                void* workspace, size_t workspace_bytes, void* stream);

/* mg_gelu_bwd (with dbias = db1, over C1 columns) and mg_column_sum of dy
 * (bf16 [N, C2], row stride ld_dy, into db2) in one launch, then both
 * reductions in one more: the elementwise work of the FeedForward backward
 * (reference mingru/minLM.py:17-23: GELU's backward and both Linear biases'
 * gradients). Results equal the two separate calls' bit for bit. Workspace:
 * mg_ff_bias_bwd_workspace_bytes(N, C1, C2). Shapes and alignment as above. */
size_t mg_ff_bias_bwd_workspace_bytes(int64_t N, int C1, int C2);
int mg_ff_bias_bwd(int dh_dtype, const void* dh, int64_t ld_dh, const void* pre, int64_t ld_pre, void* dpre,
                   int64_t ld_out, float* db1, int64_t N, int C1, const void* dy, int64_t ld_dy, float* db2, int C2,
                   void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Token-embedding weight gradient (reference mingru/minLM.py:92,99: the
 * backward of nn.Embedding):
 *   dw[v, :] = sum over t with ids[t] == v of dx[t, :]
 * (ids int64 [N]; dx fp32 [N, D], row stride ldx; dw fp32 [V, D], row stride
 * ldw, written, zero rows for ids without tokens). Sums in a fixed order
 * (token order within chunks of 64 positions, chunks in order), so results
 * repeat bit for bit. No host round trip (torch's version copies a segment
 * count to the host). Ids outside [0, V) are skipped.
 * 1 <= V <= 512, D % 4 == 0, strides % 4 == 0, dx/dw 16-byte aligned, N < 2^31;
 * workspace of mg_embedding_bwd_workspace_bytes(N, D, V) bytes, 16-byte aligned.
 * ---------------------------------------------------------------------- */
size_t mg_embedding_bwd_workspace_bytes(int64_t N, int D, int V);
int mg_embedding_bwd(const int64_t* ids, const float* dx, int64_t ldx, int64_t N, int D, int V,
                     float* dw, int64_t ldw, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * One-token decode step (generation), batch 1..8, bf16 weights, fp32
 * residual stream and recurrence state; replaces the per-token call of
 * minLM.forward in reference generate.py:199-212 (mingru/minLM.py:97-138 on
 * one position, minGRU's one-step path mingru/minGRU.py:45-52 and to_out
 * :41,71). No conv, no dropout. Per layer:
 *   mg_decode_mingru (expansion 1.0, Di = D): x = (tokens ? emb[tokens] :
 *     x_in) + pending (bf16, nullable); n = bf16(RMSNorm(x) * norm_w);
 *     [hidden | gate] = bf16(n W_hg^T) (W_hg bf16 [2D, D]); state = a state +
 *     z g(hidden) (fp32 [B, D], in place); x_out = x + state. Tokens are
 *     clamped into [0, V).
 *   mg_decode_mingru_expanded (expansion != 1.0): the same with Di channels
 *     (W_hg bf16 [2 Di, D], state fp32 [B, Di]); the step's output goes to
 *     h_out = bf16(state) [B, Di] instead of the residual stream, then
 *   mg_decode_to_out: x_out = x + h W_out^T (W_out bf16 [D, Di], fp32 sum),
 *     x formed as in mg_decode_mingru from the same tokens / x_in / pending.
 *   mg_decode_ff: n = bf16(RMSNorm(x) * norm_w); act = bf16(gelu(bf16(n W1^T
 *     + b1))) (W1 bf16 [F, D], b1 bf16 [F], act bf16 [B, F] scratch);
 *     pending_out = bf16(act W2^T + b2) (W2 bf16 [D, F], b2 bf16 [D]).
 *   mg_decode_head: logits = bf16(bf16(RMSNorm(x_in + pending) * norm_w)
 *     W_out^T) (W_out bf16 [V, D], logits bf16 [B, V]).
 * RMSNorm: x / sqrt(mean(x^2) + eps). D <= 2048; F and Di <= 8192; all
 * multiples of 8 (F also of 4 rows per wave); weights, act, h, x / x_in /
 * emb and norm_w 16-byte aligned, pending 8-byte aligned.
 * ---------------------------------------------------------------------- */
int mg_decode_mingru(int B, int D, const int64_t* tokens, const float* emb, int V, const float* x_in,
                     const void* pending, float* x_out, const float* norm_w, const void* w_hg,
                     float* state, float eps, void* stream);
int mg_decode_mingru_expanded(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                              const float* x_in, const void* pending, void* h_out, const float* norm_w,
                              const void* w_hg, float* state, float eps, void* stream);
int mg_decode_to_out(int B, int D, int Di, const int64_t* tokens, const float* emb, int V, const float* x_in,
                     const void* pending, const void* h, const void* w_out, float* x_out, void* stream);
int mg_decode_ff(int B, int D, int F, const float* x, const float* norm_w, const void* w1,
                 const void* b1, void* act, const void* w2, const void* b2, void* pending_out,
                 float eps, void* stream);
int mg_decode_head(int B, int D, int V, const float* x_in, const void* pending, const float* norm_w,
                   const void* w_out, void* logits, float eps, void* stream);

/* The same steps for a model kept in fp32 (reference generate.py:277-278,
 * --use-f32, which loads the model without a cast): fp32 weights, biases,
 * pending, act, h and logits, and no rounding point (the norm output and the
 * projections stay fp32). mg_decode_mingru_f32 writes x_out (expansion 1.0,
 * Di == D) or h_out (Di != D), exactly one of them. Staged rows (F, Di) are
 * at most 8192 long at batch 1-4 and 4096 at batch 5-8; pending 16-byte
 * aligned. */
int mg_decode_mingru_f32(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                         const float* x_in, const float* pending, float* x_out, float* h_out,
                         const float* norm_w, const float* w_hg, float* state, float eps, void* stream);
int mg_decode_to_out_f32(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                         const float* x_in, const float* pending, const float* h, const float* w_out,
                         float* x_out, void* stream);
int mg_decode_ff_f32(int B, int D, int F, const float* x, const float* norm_w, const float* w1,
                     const float* b1, float* act, const float* w2, const float* b2, float* pending_out,
                     float eps, void* stream);
int mg_decode_head_f32(int B, int D, int V, const float* x_in, const float* pending, const float* norm_w,
                       const float* w_out, float* logits, float eps, void* stream);

/* The same steps for a model cast with .to(torch.float16) (reference
 * generate.py:143-144, --use-f32 --use-fp16): fp16 weights, biases, pending,
 * act, h and logits (void* here: IEEE binary16), and the bf16 steps' rounding
 * points at fp16; limits and alignments as the bf16 steps. */
int mg_decode_mingru_f16(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                         const float* x_in, const void* pending, float* x_out, void* h_out,
                         const float* norm_w, const void* w_hg, float* state, float eps, void* stream);
int mg_decode_to_out_f16(int B, int D, int Di, const int64_t* tokens, const float* emb, int V,
                         const float* x_in, const void* pending, const void* h, const void* w_out,
                         float* x_out, void* stream);
int mg_decode_ff_f16(int B, int D, int F, const float* x, const float* norm_w, const void* w1,
                     const void* b1, void* act, const void* w2, const void* b2, void* pending_out,
                     float eps, void* stream);
int mg_decode_head_f16(int B, int D, int V, const float* x_in, const void* pending, const float* norm_w,
                       const void* w_out, void* logits, float eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MINGRU_HIP_H */
