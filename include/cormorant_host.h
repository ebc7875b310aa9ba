/*
 * cormorant_host.h -- C ABI of libcormo_host.so: the reference's host-CPU ops (its HostNode and
 * LlmNode reference() bodies) in IEEE double with glibc's exp / erf / tanh, in the reference's
 * operation order, written back with round half to even and saturation to raw int16 (NaN -> 0):
 * the bit-exact CPU side of the simulator, for the ops the reference runs on the host rather
 * than on a unit.
 *
 * Conventions: HOST pointers; inputs are float64 VALUES (raw * 2^-f, as the reference's
 * simulator passes them); int16 outputs are raw lanes at 2^-8 (Q8.8, DataType.host_quantize,
 * dtype.py:214-219) or at the given per-channel exponents (quantize_exp, dtype.py:278-286).
 * Return 0, or -1 for a null pointer or an impossible shape.  Thread-safe (no state).
 */
#ifndef CORMORANT_HOST_H
#define CORMORANT_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int cmh_abi_version(void);

/* ONNX Softmax on the host: SoftmaxNode.reference (inference-scheduler/src/host_nodes.py:1037-1041):
 * e = exp(x - max) per row of n, summed left to right, y = e / sum in Q8.8. */
int cmh_softmax(const double* x, int16_t* y, uint64_t rows, uint64_t n);

/* LayerNormalization on the host: LayerNormNode.reference (host_nodes.py:1134-1148): mean and
 * variance as left-to-right sums / n, inv = 1 / sqrt(var + eps); tf_form 0: (x - mean) inv gamma +
 * beta, 1: x (inv gamma) + (beta - mean inv gamma); gamma / beta float32 [n] or NULL (1 / 0). */
int cmh_layernorm(const double* x, int16_t* y, uint64_t rows, uint64_t n, const float* gamma, const float* beta,
                  double eps, int tf_form);

/* GELU on the host: GeluNode.values (host_nodes.py:1228-1240): tanh_form 1:
 * x (0.5 (1 + tanh(p2 (x + p1 x^3)))), p1 = c1, p2 = c2; 0: x (0.5 (1 + erf(u))), u = x / p1 (div)
 * or x p1; Q8.8 out. */
int cmh_gelu(const double* x, int16_t* y, uint64_t n, int tanh_form, double p1, double p2, int div);

/* LlmRMSNorm on the host: LlmRMSNormNode.reference (llm_nodes.py:676-688): rows of n (a W-wide row
 * as W / n of them), r = 1 / sqrt(sum(h^2) / n + eps), y = (h r) gamma at f_out[W] per channel. */
int cmh_rmsnorm(const double* h, int16_t* y, uint64_t rows, uint32_t n, uint32_t W, const float* gamma, double eps,
                const int32_t* f_out);

/* LlmSiluMul on the host: LlmSiluMulNode.reference (llm_nodes.py:741-751): silu of g's raw at the
 * gate exponent f_gate[c] (t = floor(g 2^f) / 2^f, t / (1 + exp(-t)), 0 for t <= -700, the
 * silu_table entry, :322-332) times u, at f_out[c]; rows of n. */
int cmh_silu_mul(const double* g, const double* u, int16_t* y, uint64_t rows, uint32_t n, const int32_t* f_gate,
                 const int32_t* f_out);

/* LlmResAdd (llm_nodes.py:586-609): y = float32(h + d).  LlmDequant / LlmToHost
 * (:1722-1780): y = float32(x). */
int cmh_resadd_f32(const double* h, const double* d, float* y, uint64_t count);
int cmh_to_f32(const double* x, float* y, uint64_t count);

/* LlmAttention (the host attention of the xattn policy): LlmAttentionNode.reference
 * (llm_nodes.py:923-955).  For t < n (clamped: 0 <= n <= T, pos + n <= C): the caches' row
 * pos + t <- RoPE(k0[t]) at f_ck and v[t] at f_cv (raw int16, group-major [KV][C][HD], written in
 * place); then per head h of group g = h / (H / KV): qr = RoPE(q0[t][h]) unquantised, scores
 * s_j = dot8(qr K_j) scale over the keys j <= pos + t (dot8: 8 lanes over d in order, then
 * ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7))), e = exp(s - max), P = e / (left-to-right
 * sum), out[t][h] = sum_j P_j V_j left to right, at f_out; rows t >= n are 0.  cos / sin are the
 * float32 [C][HD / 2] tables. */
typedef struct cmh_attn_args {
    const double* q0;       /* [T][H][HD] values */
    const double* k0;       /* [T][KV][HD] values */
    const double* v;        /* [T][KV HD] values */
    int16_t* ck;            /* [KV][C][HD] raw at f_ck (per channel of KV HD) */
    int16_t* cv;            /* [KV][C][HD] raw at f_cv */
    const int32_t* f_ck;
    const int32_t* f_cv;
    const float* cos;       /* [C][HD / 2] */
    const float* sin;
    int16_t* out;           /* [T][H][HD] raw at f_out (per channel of H HD) */
    const int32_t* f_out;
    double scale;           /* 1 / sqrt(HD) */
    uint32_t T, H, KV, HD, C, pos;
    int64_t n;
} cmh_attn_args;
int cmh_attention(const cmh_attn_args* a);

#ifdef __cplusplus
}
#endif

#endif /* CORMORANT_HOST_H */
