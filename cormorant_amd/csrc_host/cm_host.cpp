// cm_host.cpp -- the reference's host-CPU ops (the ops its boards run on the ARM core, and its
// simulator's HostNode / LlmNode reference() bodies) in IEEE double with the C library's exp,
// erf and tanh -- glibc's, the library behind the reference's Python `math` calls -- in the
// reference's operation order (left-to-right sums, its dot-product lane order), written back
// with round half to even and saturation (DataType.host_quantize / quantize_exp,
// inference-scheduler/src/dtype.py:214-219, 278-286).
//
// Built with g++ -O2 -ffp-contract=off: no fused multiply-adds, no reassociation, so every
// operation rounds where the reference's does.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "../../include/cormorant_host.h"

namespace {

// Round half to even at 2^-f and saturate to int16 (NaN -> 0): the write-back of a host op's
// double result (host_st / llm_st).  `scale` = 2^f.
inline int16_t st16(double v, double scale) {
    if (std::isnan(v)) v = 0.0;
    double r = std::nearbyint(v * scale);
    if (r < -32768.0) r = -32768.0;
    if (r > 32767.0) r = 32767.0;
    return (int16_t)r;
}

inline double p2(int f) { return std::ldexp(1.0, f); }

// rope (llm_nodes.py:304-312): y = x c + rot s over one head of HD values, c / s the float32
// cos / sin rows repeated over both halves, rot = [-x[half:], x[:half]].
inline void rope_row(const double* x, const float* cos_row, const float* sin_row, uint32_t HD, double* y) {
    const uint32_t half = HD / 2;
    for (uint32_t d = 0; d < HD; d++) {
        const double c = (double)cos_row[d % half], s = (double)sin_row[d % half];
        const double rot = d < half ? -x[d + half] : x[d - half];
        y[d] = x[d] * c + rot * s;
    }
}

}  // namespace

extern "C" {

int cmh_abi_version(void) { return 100; }

int cmh_softmax(const double* x, int16_t* y, uint64_t rows, uint64_t n) {
    if (!x || !y || n == 0) return -1;
    std::vector<double> e(n);
    for (uint64_t r = 0; r < rows; r++) {
        const double* xr = x + r * n;
        double m = xr[0];                            // the row maximum; a NaN propagates (numpy's max)
        for (uint64_t i = 1; i < n && !std::isnan(m); i++)
            if (std::isnan(xr[i]) || xr[i] > m) m = xr[i];
        double s = 0.0;
        for (uint64_t i = 0; i < n; i++) {
            e[i] = std::exp(xr[i] - m);
            s += e[i];
        }
        for (uint64_t i = 0; i < n; i++) y[r * n + i] = st16(e[i] / s, 256.0);
    }
    return 0;
}

int cmh_layernorm(const double* x, int16_t* y, uint64_t rows, uint64_t n, const float* gamma, const float* beta,
                  double eps, int tf_form) {
    if (!x || !y || n == 0) return -1;
    const double nd = (double)n;
    for (uint64_t r = 0; r < rows; r++) {
        const double* xr = x + r * n;
        double sum = 0.0;
        for (uint64_t i = 0; i < n; i++) sum += xr[i];
        const double mean = sum / nd;
        double ss = 0.0;
        for (uint64_t i = 0; i < n; i++) {
            const double d = xr[i] - mean;
            ss += d * d;
        }
        const double var = ss / nd;
        const double inv = 1.0 / std::sqrt(var + eps);
        for (uint64_t i = 0; i < n; i++) {
            const double ga = gamma ? (double)gamma[i] : 1.0, be = beta ? (double)beta[i] : 0.0;
            double v;
            if (tf_form) {
                const double g = inv * ga;
                v = xr[i] * g + (be - mean * g);
            } else {
                v = (xr[i] - mean) * inv * ga + be;
            }
            y[r * n + i] = st16(v, 256.0);
        }
    }
    return 0;
}

int cmh_gelu(const double* x, int16_t* y, uint64_t n, int tanh_form, double p1, double p2v, int div) {
    if (!x || !y) return -1;
    for (uint64_t i = 0; i < n; i++) {
        const double v = x[i];
        double r;
        if (tanh_form) {
            r = v * (0.5 * (1.0 + std::tanh(p2v * (v + p1 * (v * v * v)))));
        } else {
            const double u = div ? v / p1 : v * p1;
            r = v * (0.5 * (1.0 + std::erf(u)));
        }
        y[i] = st16(r, 256.0);
    }
    return 0;
}

int cmh_rmsnorm(const double* h, int16_t* y, uint64_t rows, uint32_t n, uint32_t W, const float* gamma, double eps,
                const int32_t* f_out) {
    if (!h || !y || !gamma || !f_out || n == 0 || W % n) return -1;
    for (uint64_t r = 0; r < rows; r++) {            // rows of n; row r sits at column (r n) % W of its W-row
        const double* hr = h + r * n;
        double ss = 0.0;
        for (uint32_t i = 0; i < n; i++) ss += hr[i] * hr[i];
        const double rr = 1.0 / std::sqrt(ss / (double)n + eps);
        const uint64_t c0 = (r * n) % W;
        for (uint32_t i = 0; i < n; i++) y[r * n + i] = st16((hr[i] * rr) * (double)gamma[i], p2(f_out[c0 + i]));
    }
    return 0;
}

int cmh_silu_mul(const double* g, const double* u, int16_t* y, uint64_t rows, uint32_t n, const int32_t* f_gate,
                 const int32_t* f_out) {
    if (!g || !u || !y || !f_gate || !f_out) return -1;
    for (uint64_t r = 0; r < rows; r++)
        for (uint32_t c = 0; c < n; c++) {
            const uint64_t i = r * n + c;
            const double d = p2(f_gate[c]);
            // the table entry of g's raw (silu_table, llm_nodes.py:322-332): t = raw / 2^f
            const double t = (std::floor(g[i] * d) + 0.0) / d;
            const double s = t > -700.0 ? t / (1.0 + std::exp(-t)) : 0.0;
            y[i] = st16(s * u[i], p2(f_out[c]));
        }
    return 0;
}

int cmh_resadd_f32(const double* h, const double* d, float* y, uint64_t count) {
    if (!h || !d || !y) return -1;
    for (uint64_t i = 0; i < count; i++) y[i] = (float)(h[i] + d[i]);
    return 0;
}

int cmh_to_f32(const double* x, float* y, uint64_t count) {
    if (!x || !y) return -1;
    for (uint64_t i = 0; i < count; i++) y[i] = (float)x[i];
    return 0;
}

int cmh_attention(const cmh_attn_args* a) {
    if (!a || !a->q0 || !a->k0 || !a->v || !a->ck || !a->cv || !a->out || !a->cos || !a->sin) return -1;
    const uint32_t T = a->T, H = a->H, KV = a->KV, HD = a->HD, C = a->C;
    if (KV == 0 || H % KV || HD % 8 || HD == 0 || C == 0) return -1;
    const uint32_t G = H / KV, W = KV * HD;
    const uint32_t half = HD / 2;
    int64_t nn = a->n;
    if (a->pos >= C) nn = 0;
    else {
        if (nn > (int64_t)T) nn = T;
        if (nn > (int64_t)(C - a->pos)) nn = C - a->pos;
        if (nn < 0) nn = 0;
    }
    const uint32_t n = (uint32_t)nn, pos = a->pos;
    std::vector<double> buf(HD), kr(HD);
    // the new rows into the caches at their exponents (raw int16, group-major [KV][C][HD])
    for (uint32_t t = 0; t < n; t++) {
        const uint32_t p = pos + t;
        const float* cr = a->cos + (uint64_t)p * half;
        const float* sr = a->sin + (uint64_t)p * half;
        for (uint32_t g = 0; g < KV; g++) {
            rope_row(a->k0 + ((uint64_t)t * KV + g) * HD, cr, sr, HD, kr.data());
            for (uint32_t d = 0; d < HD; d++) {
                const uint32_t c = g * HD + d;
                a->ck[((uint64_t)g * C + p) * HD + d] = st16(kr[d], p2(a->f_ck[c]));
                a->cv[((uint64_t)g * C + p) * HD + d] = st16(a->v[(uint64_t)t * W + c], p2(a->f_cv[c]));
            }
        }
    }
    std::vector<double> s(C), e(C), qr(HD), o(HD);
    for (uint32_t t = 0; t < T; t++)
        for (uint32_t h = 0; h < H; h++)
            for (uint32_t d = 0; d < HD; d++) a->out[((uint64_t)t * H + h) * HD + d] = 0;
    for (uint32_t t = 0; t < n; t++) {
        const uint32_t p = pos + t, keys = p + 1;
        const float* cr = a->cos + (uint64_t)p * half;
        const float* sr = a->sin + (uint64_t)p * half;
        for (uint32_t h = 0; h < H; h++) {
            const uint32_t g = h / G;
            rope_row(a->q0 + ((uint64_t)t * H + h) * HD, cr, sr, HD, qr.data());   // unquantised
            // dot8 (llm_nodes.py:292-301): 8 lanes acc_l = sum_a prod[8 a + l] in order, then
            // ((acc0 + acc1) + (acc2 + acc3)) + ((acc4 + acc5) + (acc6 + acc7)); times the scale
            double mx = 0.0;
            for (uint32_t j = 0; j < keys; j++) {
                double acc[8];
                for (int l = 0; l < 8; l++) acc[l] = 0.0;
                const int16_t* kj = a->ck + ((uint64_t)g * C + j) * HD;
                for (uint32_t aa = 0; aa < HD / 8; aa++)
                    for (int l = 0; l < 8; l++) {
                        const uint32_t d = 8 * aa + l;
                        const double kv = std::ldexp((double)kj[d], -a->f_ck[g * HD + d]);
                        const double prod = qr[d] * kv;
                        acc[l] = aa == 0 ? prod : acc[l] + prod;
                    }
                const double dot = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
                s[j] = dot * a->scale;
                if (j == 0 || s[j] > mx) mx = s[j];
            }
            double sum = 0.0;
            for (uint32_t j = 0; j < keys; j++) {
                e[j] = std::exp(s[j] - mx);
                sum += e[j];
            }
            for (uint32_t d = 0; d < HD; d++) o[d] = 0.0;
            for (uint32_t j = 0; j < keys; j++) {
                const double pr = e[j] / sum;
                const int16_t* vj = a->cv + ((uint64_t)g * C + j) * HD;
                for (uint32_t d = 0; d < HD; d++) {
                    const double term = pr * std::ldexp((double)vj[d], -a->f_cv[g * HD + d]);
                    o[d] = j == 0 ? term : o[d] + term;
                }
            }
            for (uint32_t d = 0; d < HD; d++)
                a->out[((uint64_t)t * H + h) * HD + d] = st16(o[d], p2(a->f_out[h * HD + d]));
        }
    }
    return 0;
}

}  // extern "C"
