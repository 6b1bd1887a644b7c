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
 *   - dtype codes: MG_F32 = 0 (float), MG_BF16 = 1 (bfloat16, RNE rounding).
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
#define MG_ERR_WORKSPACE 3 /* workspace missing or too small */
#define MG_ERR_HIP 4      /* a HIP runtime call or kernel launch failed */

/* Library version (major*10000 + minor*100 + patch). */
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
 * Supported (in_dtype, out_dtype): (BF16, BF16), (F32, F32), (BF16, F32).
 * ---------------------------------------------------------------------- */
size_t mg_scan_workspace_bytes(int B, int T, int Di);  /* serves fwd and bwd */

int mg_scan_fwd(int in_dtype, const void* hidden, const void* gate,
                int64_t in_sb, int64_t in_ld,
                const float* h0,
                int out_dtype, void* h, int64_t out_sb, int64_t out_ld,
                float* h_last,
                int B, int T, int Di,
                void* workspace, size_t workspace_bytes, void* stream);

/* Backward of mg_scan_fwd: autograd of reference mingru/minGRU.py:16-20,
 * :53-69 through gate, hidden and prev_hidden, in closed form:
 *   lambda_t  = dh_t + a_{t+1} lambda_{t+1},
 *   dgate_t   = lambda_t z_t (1 - z_t) (g(hidden_t) - h_{t-1}),
 *   dhidden_t = lambda_t z_t g'(hidden_t)   (g'(0) = 0, as relu'(0) = 0),
 *   dh0       = a_0 lambda_0.
 * h: the forward's output (same layout, dtype out_dtype); h_{t-1} is read
 * from it once per 4-step run and rebuilt in fp32 inside the run.
 * dh: gradient of h, dtype out_dtype, element (b,t,d) at b*g_sb + t*g_ld + d.
 * dh_last (nullable): fp32 [B, Di], gradient of h_last, added to dh_{T-1}.
 * dhidden/dgate: same layout and dtype as hidden/gate (in_sb, in_ld).
 * dh0 (nullable): fp32 [B, Di]. */
int mg_scan_bwd(int in_dtype, const void* hidden, const void* gate,
                int64_t in_sb, int64_t in_ld,
                const float* h0,
                int out_dtype, const void* h, int64_t out_sb, int64_t out_ld,
                const void* dh, int64_t g_sb, int64_t g_ld,
                const float* dh_last,
                void* dhidden, void* dgate, float* dh0,
                int B, int T, int Di,
                void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MINGRU_HIP_H */
