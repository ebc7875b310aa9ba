/*
 * cm_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C CPU restatement of the integer arithmetic that the reference's fixed-point
 * simulator (inference-scheduler/src/codegen/_simulate.py and the spec modules it calls)
 * predicts for the five units: VectorOP (element-wise, activation unit, softmax unit),
 * Matmul, Conv, Pooling and RowOps.  It is the checker that the HIP library is compared
 * against; the library never links, loads or calls it.  Only tests/, the smoke check and
 * bench.py's CPU-baseline leg use it.
 *
 * Every routine works on raw two's-complement lanes (value = raw * 2^-f) and follows the
 * register-level geometry of the unit it models.  Each one names the reference lines it
 * restates.  Pinning of each function (golden fixtures, ROM text, closed forms) is listed
 * in oracle/README.md.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef int64_t i64;
typedef uint64_t u64;
typedef __int128 i128;

/* ------------------------------------------------------------------ helpers */
static inline i64 sat16(i64 v) { return v > 32767 ? 32767 : (v < -32768 ? -32768 : v); }
static inline i64 sat16w(i128 v) { return v > 32767 ? 32767 : (v < -32768 ? -32768 : (i64)v); }
static inline i64 sat32w(i128 v) {
    return v > 2147483647 ? 2147483647 : (v < -2147483647LL - 1 ? -2147483647LL - 1 : (i64)v);
}
/* floor(v / 2^k) (arithmetic shift; gcc shifts signed values arithmetically) */
static inline i64 floor_shr(i64 v, int k) { return v >> k; }
/* round half to even of v / 2^k (rowops_spec.py:48-56); k <= 0 shifts left */
static inline i128 rne_shr128(i128 v, int k) {
    if (k <= 0) return v << (-k);
    i128 q = v >> k;
    i128 r = v - (q << k);
    i128 half = (i128)1 << (k - 1);
    int up = (r > half) || (r == half && (q & 1));
    return q + up;
}
static inline i64 wrap32(i64 v) { return (i64)(int32_t)(uint32_t)(u64)v; }

/* ------------------------------------------------------------------ activation tables */
/* vectorop_act.py:60-79 (act_values, libm = glibc through Python's math module,
 * host_nodes.py:150-162) then DataType.host_quantize (dtype.py:214-219): clip to the
 * Q8.8 range, round half to even (np.round == nearbyint under FE_TONEAREST). */
enum { ACT_NONE = 0, ACT_RELU = 1, ACT_RELU6 = 2, ACT_LEAKY = 3, ACT_SILU = 4, ACT_GELU = 5,
       ACT_GELU_TANH = 6 };
enum { OP_ADD = 0, OP_SUB = 1, OP_MUL = 2, OP_DIV = 3, OP_RELU = 4, OP_RELU6 = 5, OP_LEAKY = 6,
       OP_SILU = 7, OP_GELU = 8, OP_GELU_TANH = 9, OP_SOFTMAX = 10, OP_SOFTMAX_T = 11 };

static double act_value(int act, double x) {
    switch (act) {
    case ACT_SILU: return x / (1.0 + exp(-x));
    case ACT_GELU: return x * (0.5 * (1.0 + erf(x / sqrt(2.0))));
    case ACT_GELU_TANH:
        return x * (0.5 * (1.0 + tanh(sqrt(2.0 / M_PI) * (x + 0.044715 * (x * x * x)))));
    default: return x;
    }
}

static i64 host_quantize_q88(double v) {
    if (v != v) return 0;                       /* NaN -> 0 */
    double r = v * 256.0;
    if (r > 32767.0) r = 32767.0;
    if (r < -32768.0) r = -32768.0;
    return (i64)nearbyint(r);
}

static int16_t g_act_tab[3][65536];
static int g_act_ready = 0;

static void act_tables_build(void) {
    if (g_act_ready) return;
    for (int a = 0; a < 3; a++)
        for (int raw = -32768; raw < 32768; raw++)
            g_act_tab[a][raw + 32768] =
                (int16_t)host_quantize_q88(act_value(ACT_SILU + a, (double)raw / 256.0));
    g_act_ready = 1;
}

/* The kernel table of one unit activation over every Q8.8 input, ascending raw
 * (vectorop_act.kernel_table, vectorop_act.py:107-114). */
int oracle_act_table(int act, int16_t* out65536) {
    if (act < ACT_SILU || act > ACT_GELU_TANH) return -1;
    act_tables_build();
    memcpy(out65536, g_act_tab[act - ACT_SILU], sizeof(int16_t) * 65536);
    return 0;
}

/* One activation of the unit on a truncated op result t (raw int16).
 * LeakyReLU: x >= 0 ? x : x * (alpha & 0xFFFF) / 2^16 in double, exact, then RNE
 * (vectorop_act.py:66-67): for raw t that is rne(t * alpha / 2^16). */
static i64 apply_act(int act, i64 t, unsigned alpha) {
    switch (act) {
    case ACT_RELU: return t < 0 ? 0 : t;
    case ACT_RELU6: return t < 0 ? 0 : (t > 1536 ? 1536 : t);
    case ACT_LEAKY:
        if (t >= 0) return t;
        return sat16w(rne_shr128((i128)t * (i64)(alpha & 0xFFFFu), 16));
    case ACT_SILU: case ACT_GELU: case ACT_GELU_TANH:
        act_tables_build();
        return g_act_tab[act - ACT_SILU][t + 32768];
    default: return t;
    }
}

/* job_act (nodes.py:159-162; VectorOP.h:146-149) */
static unsigned job_act(unsigned op, unsigned act) {
    return (op >= OP_LEAKY && op <= OP_GELU_TANH) ? op - (OP_LEAKY - ACT_LEAKY) : act;
}

/* ------------------------------------------------------------------ softmax unit */
/* TAB[k] = round(2^16 * 2^(-k/4096)) (vectorop_smx.py:29-34) */
static i64 g_smx_tab[4096];
static int g_smx_ready = 0;
static void smx_build(void) {
    if (g_smx_ready) return;
    for (int k = 0; k < 4096; k++) g_smx_tab[k] = (i64)nearbyint(ldexp(exp2(-(double)k / 4096.0), 16));
    g_smx_ready = 1;
}
int oracle_smx_table(int32_t* out4096) {
    smx_build();
    for (int k = 0; k < 4096; k++) out4096[k] = (int32_t)g_smx_tab[k];
    return 0;
}

/* smx_valid: v = min(n, valid0 + (q mod period)) (vectorop_smx.causal_valid,
 * vectorop_smx.py:75-79) */
static unsigned smx_valid(unsigned q, unsigned n, unsigned mask) {
    unsigned valid0 = mask & 0xFFFFu, period = mask >> 16;
    unsigned v = valid0 + (period ? q % period : 0u);
    return v < n ? v : n;
}

/* One vector (vectorop_smx.softmax_raw, vectorop_smx.py:50-66): x[j] at stride xs,
 * p[j] at stride 1. */
static void smx_vector(const int16_t* x, long xs, unsigned n, unsigned v, unsigned cm,
                       unsigned cfg, int16_t* p, i64* e) {
    smx_build();
    unsigned cs = cfg & 63u, fp = (cfg >> 8) & 31u;
    cm &= 0xFFFFFFu;
    if (v > n) v = n;
    i64 m = INT64_MIN;
    for (unsigned j = 0; j < v; j++) if (x[j * xs] > m) m = x[j * xs];
    i64 S = 0;
    for (unsigned j = 0; j < v; j++) {
        u64 y = ((u64)(m - x[j * xs]) * cm) >> cs;
        u64 sh = y >> 12;
        e[j] = sh >= 63 ? 0 : (g_smx_tab[y & 4095] >> sh);
        S += e[j];
    }
    u64 R = S > 0 ? ((u64)1 << 40) / (u64)S : 0;
    for (unsigned j = 0; j < n; j++) {
        if (j >= v) { p[j] = 0; continue; }
        u64 q = ((u64)e[j] * R + ((u64)1 << (40 - fp - 1))) >> (40 - fp);
        p[j] = (int16_t)(q > 32767 ? 32767 : q);
    }
}

/* ------------------------------------------------------------------ VectorOP */
/* The register contract (VectorOP.h:277-333): c[o*(a_inc+b_inc) + i] =
 * act(op(a[o*a_inc + i], b[o*b_inc + i])), o < outer, i < size; ops 10/11 are the softmax
 * unit (VectorOP.cpp:383-433): row mode reads rows at stride a_inc and writes them at
 * stride b_inc; column mode reads s[size keys][outer queries] (row stride a_inc) and writes
 * P[q][size] at stride b_inc for q < outer & ~15.  Whole 8-lane words are written: the
 * lanes of a run's last word past size are 0 (VectorOP.h:229-236) -- this routine writes
 * them too, so `c` must cover them.
 *
 * Arithmetic follows the simulator (_simulate.py:721-765, dtype.py:371-383):
 *   ADD/SUB sat16(a +- b); MUL sat16(floor(a*b / 2^8));
 *   DIV sat16(trunc(a * 2^8 / b)); b == 0: +32767 for a > 0, -32768 for a < 0 (the
 *       simulator's +-inf saturated), 0 for 0/0 (its NaN, written back as 0 the way
 *       host_quantize does) -- the board returns 0 for every b == 0 (VectorOP.cpp:35-38);
 *   RELU / RELU6; the act register (or the activation op's own) after the op. */
int oracle_vectorop(const int16_t* a, const int16_t* b, int16_t* c, unsigned size, unsigned op,
                    unsigned outer, unsigned a_inc, unsigned b_inc, unsigned act,
                    unsigned alpha, unsigned smx_cm, unsigned smx_cfg, unsigned smx_mask) {
    if (op > OP_SOFTMAX_T) return -1;
    unsigned padded = (size + 7u) & ~7u;
    if (op == OP_SOFTMAX || op == OP_SOFTMAX_T) {
        i64* e = (i64*)malloc(sizeof(i64) * (size ? size : 1));
        int16_t* p = (int16_t*)malloc(sizeof(int16_t) * (padded ? padded : 8));
        unsigned nq = op == OP_SOFTMAX ? outer : (outer & ~15u);
        for (unsigned q = 0; q < nq; q++) {
            const int16_t* x = op == OP_SOFTMAX ? a + (size_t)q * a_inc : a + q;
            long xs = op == OP_SOFTMAX ? 1 : (long)a_inc;
            smx_vector(x, xs, size, smx_valid(q, size, smx_mask), smx_cm, smx_cfg, p, e);
            for (unsigned j = size; j < padded; j++) p[j] = 0;
            memcpy(c + (size_t)q * b_inc, p, sizeof(int16_t) * padded);
        }
        free(e); free(p);
        return 0;
    }
    unsigned ja = job_act(op, act);
    int unary = op >= OP_RELU;
    for (unsigned o = 0; o < outer; o++) {
        const int16_t* ar = a + (size_t)o * a_inc;
        const int16_t* br = unary ? NULL : b + (size_t)o * b_inc;
        int16_t* cr = c + (size_t)o * (a_inc + b_inc);
        for (unsigned i = 0; i < padded; i++) {
            i64 av = i < size ? ar[i] : 0, bv = (!unary && i < size) ? br[i] : 0, r;
            switch (op) {
            case OP_ADD: r = sat16(av + bv); break;
            case OP_SUB: r = sat16(av - bv); break;
            case OP_MUL: r = sat16(floor_shr(av * bv, 8)); break;
            case OP_DIV:
                if (bv == 0) r = av > 0 ? 32767 : (av < 0 ? -32768 : 0);
                else r = sat16((av * 256) / bv);       /* C division truncates toward 0 */
                break;
            case OP_RELU: r = av < 0 ? 0 : av; break;
            case OP_RELU6: r = av < 0 ? 0 : (av > 1536 ? 1536 : av); break;
            default: r = av; break;                    /* activation ops: job_act */
            }
            cr[i] = (int16_t)apply_act((int)ja, r, alpha);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ Matmul */
/* B[kk][j] of one batch slice in one of the three images (MatmulKernel.h:91-156):
 * row-major [k][m]; packed tile-major (kTileM = 32): ((j/32)*k + kk)*32 + j%32 (packed 2: the
 * library's transposed image [m][k], j*k + kk);
 * GEMV kernel-width image kw: (c*m + j)*kw + jj with c = (kk/(16kw))*16 + kk%16,
 * jj = (kk/16) % kw (matmul_gemv_index). */
static i64 mm_b(const int16_t* b, unsigned kk, unsigned j, unsigned k, unsigned m,
                unsigned packed, unsigned kw) {
    if (kw) {
        if (kw == 1) return b[(size_t)kk * m + j];
        unsigned c = (kk / (16 * kw)) * 16 + kk % 16, jj = (kk / 16) % kw;
        return b[((size_t)c * m + j) * kw + jj];
    }
    if (packed == 2) return b[(size_t)j * k + kk];          /* this build's transposed image [m][k] */
    if (packed) return b[((size_t)(j / 32) * k + kk) * 32 + (j % 32)];
    return b[(size_t)kk * m + j];
}

/* C = sat16(floor(sum A*B / 2^8)) per output (register names of MatmulKernel.h:228-242:
 * n rows of A, k inner, m columns of B).  wrap32 = 0: the exact sum (the simulator's Q8.8
 * branch, _simulate.py:620-633: float64 sums of on-grid products are exact, no int32 wrap);
 * wrap32 = 1: the sum wraps to int32 first (_matmul_exp, _simulate.py:814-835;
 * llm_nodes._kernel_out). */
int oracle_matmul(const int16_t* a, const int16_t* b, int16_t* c, unsigned n, unsigned k,
                  unsigned m, unsigned batch, long a_bs, long b_bs, long c_bs, unsigned b_packed,
                  unsigned gemv_kw, int wrap) {
    /* Rows are independent: one output row per iteration, over every core.  Each row's sums
     * are formed from B's column j as a contiguous run of k (the transposed image packed == 2
     * as it is, any other image gathered once per batch slice); the int32-wrap sums are exact
     * mod 2^32 in uint32 arithmetic, the saturating ones exact in int64. */
    for (unsigned bt = 0; bt < batch; bt++) {
        const int16_t* A = a + (long)bt * a_bs;
        const int16_t* B = b + (long)bt * b_bs;
        int16_t* C = c + (long)bt * c_bs;
        int16_t* Bt = NULL;
        if (b_packed != 2 || gemv_kw) {
            Bt = (int16_t*)malloc((size_t)m * k * sizeof(int16_t));
            if (!Bt) return -1;
#pragma omp parallel for schedule(static)
            for (long j = 0; j < (long)m; j++)
                for (unsigned kk = 0; kk < k; kk++) Bt[(size_t)j * k + kk] = (int16_t)mm_b(B, kk, (unsigned)j, k, m, b_packed, gemv_kw);
        }
        const int16_t* BT = Bt ? Bt : B;
#pragma omp parallel for schedule(static)
        for (long i = 0; i < (long)n; i++) {
            const int16_t* Ar = A + (size_t)i * k;
            for (unsigned j = 0; j < m; j++) {
                const int16_t* Br = BT + (size_t)j * k;
                i64 acc;
                if (wrap) {
                    uint32_t s = 0;
                    for (unsigned kk = 0; kk < k; kk++) s += (uint32_t)((int32_t)Ar[kk] * (int32_t)Br[kk]);
                    acc = (i64)(int32_t)s;
                } else {
                    i64 s = 0;
                    for (unsigned kk = 0; kk < k; kk++) s += (i64)((int32_t)Ar[kk] * (int32_t)Br[kk]);
                    acc = s;
                }
                C[(size_t)i * m + j] = (int16_t)sat16(floor_shr(acc, 8));
            }
        }
        free(Bt);
    }
    return 0;
}

/* ------------------------------------------------------------------ Conv */
/* Packed weight geometry (ConvKernel.h:136-159, nodes.py:1097-1150): tiles of 16 input
 * channels, the last one 8 lanes when at most 8 channels remain; depthwise rows of
 * roundup(kh*kw, 8); bias [roundup(out_ch, 8)]. */
static unsigned cv_ic_tiles(unsigned in_ch) { return (in_ch + 15) / 16; }
static unsigned cv_last_lanes(unsigned in_ch) {
    unsigned rem = in_ch - (cv_ic_tiles(in_ch) - 1) * 16;
    return rem <= 8 ? 8 : 16;
}
static unsigned cv_tile_lanes(unsigned in_ch, unsigned t) {
    return t + 1 == cv_ic_tiles(in_ch) ? cv_last_lanes(in_ch) : 16;
}
static unsigned cv_per_m(unsigned in_ch, unsigned kh, unsigned kw) {
    return kh * kw * ((cv_ic_tiles(in_ch) - 1) * 16 + cv_last_lanes(in_ch));
}
static size_t cv_w_index(unsigned mo, unsigned ic, unsigned khi, unsigned kwi, unsigned in_ch,
                         unsigned kh, unsigned kw) {
    unsigned t = ic / 16, l = ic % 16;
    return (size_t)mo * cv_per_m(in_ch, kh, kw) + (size_t)t * kh * kw * 16 +
           (size_t)(khi * kw + kwi) * cv_tile_lanes(in_ch, t) + l;
}

/* Y = sat16(floor((bias << 8 + sum x*w) / 2^8)) (simulator: _conv2d_ref /
 * _depthwise_conv2d_ref + truncate, _simulate.py:121-197, 643-660; the pow2 branch
 * _conv_exp wraps the sum to int32 first, :784-812).  Implicit zero padding; the y channel
 * pattern of ConvKernel.h:250-258 (plane of channel c at (c mod y_cn)*y_cs + (c div y_cn)*y_gs,
 * y_cs = 0 dense, y_cn = 0 one group). */
int oracle_conv(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                unsigned batch, unsigned in_ch, unsigned in_h, unsigned in_w, unsigned out_ch,
                unsigned out_h, unsigned out_w, unsigned kh, unsigned kw, unsigned sh,
                unsigned sw, unsigned dh, unsigned dw, unsigned pt, unsigned pl,
                unsigned has_bias, unsigned is_dw, unsigned y_cs, unsigned y_cn, unsigned y_gs,
                int wrap) {
    size_t plane = (size_t)out_h * out_w;
    size_t cs = y_cs ? y_cs : plane;
    unsigned dws = (kh * kw + 7) & ~7u;
    for (unsigned nb = 0; nb < batch; nb++)
        for (unsigned mo = 0; mo < out_ch; mo++) {
            size_t cbase = y_cn ? (size_t)(mo % y_cn) * cs + (size_t)(mo / y_cn) * y_gs
                                : (size_t)mo * cs;
            int16_t* yp = y + (size_t)nb * out_ch * plane + cbase;
            for (unsigned oh = 0; oh < out_h; oh++)
                for (unsigned ow = 0; ow < out_w; ow++) {
                    i64 acc = has_bias ? (i64)bias[mo] * 256 : 0;
                    for (unsigned khi = 0; khi < kh; khi++) {
                        long ih = (long)oh * sh + (long)khi * dh - (long)pt;
                        if (ih < 0 || ih >= (long)in_h) continue;
                        for (unsigned kwi = 0; kwi < kw; kwi++) {
                            long iw = (long)ow * sw + (long)kwi * dw - (long)pl;
                            if (iw < 0 || iw >= (long)in_w) continue;
                            if (is_dw) {
                                acc += (i64)x[(((size_t)nb * in_ch + mo) * in_h + ih) * in_w + iw] *
                                       w[(size_t)mo * dws + khi * kw + kwi];
                            } else {
                                for (unsigned ic = 0; ic < in_ch; ic++)
                                    acc += (i64)x[(((size_t)nb * in_ch + ic) * in_h + ih) * in_w + iw] *
                                           w[cv_w_index(mo, ic, khi, kwi, in_ch, kh, kw)];
                            }
                        }
                    }
                    if (wrap) acc = wrap32(acc);
                    yp[(size_t)oh * out_w + ow] = (int16_t)sat16(floor_shr(acc, 8));
                }
        }
    return 0;
}

/* ------------------------------------------------------------------ Pooling */
/* _pool_poly_sqrt (_simulate.py:230-272) in integers: S = sum x^2 (the value S * 2^-16),
 * S = m * 4^k * 2^16 with m in [1, 4) cut to 16 fraction bits, Horner with the 2^-15
 * coefficients floor(0.0077, -0.0943, 0.6432, 0.4434 * 2^15) = 252, -3091, 21076, 14529 and
 * every partial floored at 2^-20, the result scaled by 2^k and floored at 2^-16.  Returns
 * the result at 2^-16. */
static i64 pool_poly_sqrt(i64 S) {
    if (S <= 0) return 0;
    int e = 63 - __builtin_clzll((u64)S);              /* floor(log2 S) */
    int d = e - 16;
    int k = d >= 0 ? d / 2 : -((-d + 1) / 2);           /* floor(d / 2) */
    i64 M = 2 * k >= 0 ? (S >> (2 * k)) : (S << (-2 * k));   /* m at 2^-16, in [2^16, 2^18) */
    const i64 C3 = 252, C2 = -3091, C1 = 21076, C0 = 14529;
    i64 T1 = floor_shr(C3 * M + C2 * 65536, 11);          /* 2^-31 -> 2^-20 */
    i64 T2 = floor_shr(T1 * M + C1 * 2097152, 16);         /* 2^-36 -> 2^-20 */
    i64 T3 = floor_shr(T2 * M + C0 * 2097152, 16);
    return k >= 4 ? (T3 << (k - 4)) : floor_shr(T3, 4 - k);
}

/* _pool2d_ref + truncate (_simulate.py:275-358, 701-719) with the PoolingKernel register
 * geometry (PoolingKernel.h:120-140): MAX over in-bounds taps (none: -32768); AVG
 * floor(sum * round(2^23/d) / 2^23) with d = pool_h*pool_w (count_include_pad) or the valid
 * taps (at least 1); LP1 sum |x|; LP2 the polynomial square root.  Then sat16. */
int oracle_pool(const int16_t* x, int16_t* y, unsigned batch, unsigned ch, unsigned in_h,
                unsigned in_w, unsigned out_h, unsigned out_w, unsigned ph, unsigned pw,
                unsigned sh, unsigned sw, unsigned pt, unsigned pl, unsigned dh, unsigned dw,
                unsigned type, unsigned lp, unsigned cip) {
    for (size_t nc = 0; nc < (size_t)batch * ch; nc++) {
        const int16_t* xp = x + nc * in_h * in_w;
        int16_t* yp = y + nc * out_h * out_w;
        for (unsigned oh = 0; oh < out_h; oh++)
            for (unsigned ow = 0; ow < out_w; ow++) {
                i64 mx = INT64_MIN, sum = 0;
                unsigned valid = 0;
                for (unsigned a = 0; a < ph; a++)
                    for (unsigned b = 0; b < pw; b++) {
                        long ih = (long)oh * sh + (long)a * dh - (long)pt;
                        long iw = (long)ow * sw + (long)b * dw - (long)pl;
                        if (ih < 0 || ih >= (long)in_h || iw < 0 || iw >= (long)in_w) continue;
                        i64 v = xp[(size_t)ih * in_w + iw];
                        valid++;
                        if (v > mx) mx = v;
                        if (type == 1) sum += v;
                        else if (type == 2) sum += lp == 1 ? (v < 0 ? -v : v) : v * v;
                    }
                i64 r;
                if (type == 0) r = valid ? mx : -32768;
                else if (type == 1) {
                    i64 d = cip ? (i64)ph * pw : (i64)valid;
                    if (d < 1) d = 1;
                    i64 inv = ((1LL << 23) + d / 2) / d;
                    r = floor_shr(sum * inv, 23);
                } else if (lp == 1) r = sum;
                else r = floor_shr(pool_poly_sqrt(sum), 8);
                yp[(size_t)oh * out_w + ow] = (int16_t)sat16(r);
            }
    }
    return 0;
}

/* ------------------------------------------------------------------ RowOps */
/* rowops_spec.py restated on byte images with the unit's register contract
 * (doc/kernels/ROWOPS_RTL_KERNEL.md section 1; rowops_spec.py:48-616). */
enum { RO_COPY = 1, RO_ADDX = 2, RO_DEQUANT = 3, RO_MULACT = 4, RO_NORM = 5, RO_ROPE = 6,
       RO_XPOSE = 7, RO_TLOAD = 8, RO_FOLD = 9, RO_GATE = 10 };
#define RO_B_EN (1u << 12)
#define RO_P_BCAST (1u << 13)
#define RO_P_KEEP (1u << 14)
#define RO_RELU (1u << 15)
#define RO_LN (1u << 16)
#define RO_SCALE (1u << 17)

/* rsqrt table: y0[idx] = round(2^47 / sqrt((idx + 0.5) 2^19)), idx in [2048, 8192)
 * (rowops_spec.py:92-102) */
static uint32_t g_rsqrt[8192];
/* sigmoid table T[i] = round(2^24 / (1 + exp(-i/256))), i <= 4096 (rowops_spec.py:337-343) */
static i64 g_sig[4097];
static int g_ro_ready = 0;

static void ro_tables_build(void) {
    if (g_ro_ready) return;
    for (int i = 0; i < 8192; i++) {
        if (i < 2048) { g_rsqrt[i] = 0; continue; }
        double v = rint(ldexp(1.0, 47) / sqrt((i + 0.5) * 524288.0));
        g_rsqrt[i] = (uint32_t)(v > 4294967295.0 ? 4294967295.0 : v);
    }
    for (int i = 0; i <= 4096; i++) g_sig[i] = (i64)rint(ldexp(1.0, 24) / (1.0 + exp(-(double)i / 256.0)));
    g_ro_ready = 1;
}

/* The 64 KiB table image (rowops_spec.table_image, rowops_spec.py:605-616). */
int oracle_rowops_table_image(uint8_t* img) {
    ro_tables_build();
    memset(img, 0, 65536);
    for (int i = 0; i < 4096; i++) {
        u64 d = (u64)(g_sig[i + 1] - g_sig[i]) & 0xFFFFFF, t = (u64)g_sig[i] & 0x1FFFFFF;
        u64 v = (d << 25) | t;
        for (int b = 0; b < 8; b++) img[8 * i + b] = (uint8_t)(v >> (8 * b));
    }
    for (int i = 0; i < 8192; i++)
        for (int b = 0; b < 4; b++) img[32768 + 4 * i + b] = (uint8_t)(g_rsqrt[i] >> (8 * b));
    return 0;
}

/* rsqrt_bf (rowops_spec.py:104-121) */
static void rsqrt_bf(i128 D, u64* Rm, int* sh) {
    int e = 0;
    for (i128 t = D; t; t >>= 1) e++;
    int d = e - 32;
    if (d & 1) d += 1;
    i128 Dm = d >= 0 ? (D >> d) : (D << (-d));
    u64 y0 = g_rsqrt[(size_t)(Dm >> 19)];
    u64 t = (u64)(((i128)Dm * (i128)y0) >> 32);
    u64 u = (u64)(((i128)t * (i128)y0) >> 32);
    i128 y1 = (i128)y0 + (((i128)y0 * ((i128)((i64)1 << 30) - (i128)u)) >> 31);
    if (y1 < ((i128)1 << 31)) y1 = (i128)1 << 31;
    if (y1 > ((i128)1 << 32) - 1) y1 = ((i128)1 << 32) - 1;
    *Rm = (u64)y1;
    *sh = 47 + d / 2;
}

/* sig_q / silu_q (rowops_spec.py:346-365): sigma at 2^-24 of g = gv 2^-14 */
static i64 sig_q(i64 gv) {
    i64 a = gv < 0 ? -gv : gv;
    int big = a >= ((i64)16 << 14);
    i64 ai = big ? ((i64)16 << 14) - 1 : a;
    i64 idx = ai >> 6, fr = ai & 63;
    i64 s = g_sig[idx] + (((g_sig[idx + 1] - g_sig[idx]) * fr) >> 6);
    if (big) s = (i64)1 << 24;
    return gv < 0 ? ((i64)1 << 24) - s : s;
}
static i64 silu_q(i64 gv) { return (i64)rne_shr128((i128)gv * sig_q(gv), 18); }

/* fold_elem (rowops_spec.py:450-460) */
static i64 fold_elem(i64 x, unsigned m, unsigned s) {
    i64 u = x < 0 ? -x : x, den = (i64)(x < 0 ? m : 1u) << s;
    i64 q = u / den, r = u - q * den;
    q += (2 * r > den || (2 * r == den && (q & 1))) ? 1 : 0;
    return x < 0 ? -q : q;
}

/* float32(v * 2^-sh) rounded to nearest even (DEQUANT, ROWOPS_RTL_KERNEL.md 1.4 op 3) */
static uint32_t ro_float_bits(i64 v, int sh) {
    if (v == 0) return 0;
    float f = (float)ldexp((double)v, -sh);   /* |v| < 2^32: exact in double, one rounding */
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline i64 rd16(const uint8_t* p) { return (int16_t)(p[0] | (p[1] << 8)); }
static inline i64 rd32(const uint8_t* p) {
    return (int32_t)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
}
static inline i64 rd_kind(const uint8_t* p, int k) { return k == 0 ? rd16(p) : rd32(p); }
static inline void wr_kind(uint8_t* p, i64 v, int k) {
    int nb = k == 0 ? 2 : 4;
    for (int i = 0; i < nb; i++) p[i] = (uint8_t)((u64)v >> (8 * i));
}

typedef struct { i64 g, bq; int sa, sb, sc; } ro_param;

/* The unit's parameter RAM (rowops_ref.h PState; ROWOPS_RTL_KERNEL.md 1.3): a job that
 * loads parameters copies its block in (n entries, or entry 0 with P_BCAST); a P_KEEP job
 * reads what the last load left.  XPOSE, TLOAD, FOLD and empty jobs leave it alone. */
static uint8_t g_pram[4096 * 16];
static int g_pram_valid = 0, g_pram_bcast = 0;
void oracle_rowops_reset_params(void) { g_pram_valid = 0; g_pram_bcast = 0; }

static ro_param ro_read_param(const uint8_t* p, unsigned c, int bcast) {
    const uint8_t* e = p + 16 * (bcast ? 0 : c);
    ro_param q;
    q.g = rd32(e);
    q.bq = (i64)((int32_t)((uint32_t)rd32(e + 4) << 10) >> 10);
    q.sa = e[8] & 63; q.sb = e[9] & 63; q.sc = e[10] & 63;
    return q;
}

/* One row-ops job on byte images a, b, c, p (each the base the registers point at; strides
 * in bytes).  Writes whole 16-byte words per row (the lanes past n zero), as the unit does.
 * The table image defaults to the spec's (oracle_rowops_table_image). */
int oracle_rowops(const uint8_t* a, const uint8_t* b, uint8_t* c, const uint8_t* p,
                  unsigned op, unsigned n, unsigned c1, unsigned c2, unsigned a_s1, unsigned a_s2,
                  unsigned b_s1, unsigned b_s2, unsigned c_s1, unsigned c_s2, long long eps,
                  unsigned aux, unsigned bq_sh, unsigned win_lo, unsigned win_hi) {
    ro_tables_build();
    unsigned code = op & 15;
    int ak = (op >> 4) & 3, bk = (op >> 6) & 3, ck = (op >> 8) & 3;
    int ben = (op & RO_B_EN) != 0, bc = (op & RO_P_BCAST) != 0;
    if (code == RO_TLOAD) return 0;
    if (code == RO_FOLD) {
        unsigned s = aux & 15, dv = (aux >> 4) & 127;
        if (n == 0 || c1 == 0 || c2 == 0 || dv == 0) return 0;
        size_t o = 0;
        for (u64 k = 0; k < c2; k++)
            for (u64 r = 0; r < c1; r++)
                for (u64 j = 0; j < n; j++, o++) {
                    i64 col = (i64)(int32_t)b_s2 + (i64)r * b_s1 + (i64)j;
                    i64 v = 0;
                    if (col >= (i64)win_lo && col < (i64)win_hi)
                        v = fold_elem(rd16(a + (i64)k * (int32_t)a_s2 + 2 * col), dv, s);
                    wr_kind(c + 2 * o, v, 0);
                }
        for (; (2 * o) % 16; o++) wr_kind(c + 2 * o, 0, 0);
        return 0;
    }
    if (n == 0 || c1 == 0 || c2 == 0 || n > 4096) return 0;
    int p_op = code == RO_COPY || code == RO_ADDX || code == RO_DEQUANT || code == RO_MULACT ||
               code == RO_GATE || code == RO_NORM || code == RO_ROPE;
    if (p_op) {
        if (!(op & RO_P_KEEP) || !g_pram_valid) {
            if (!(op & RO_P_KEEP)) {
                memcpy(g_pram, p, 16u * (bc ? 1u : n));
                g_pram_valid = 1;
                g_pram_bcast = bc;
            }
        }
        if (g_pram_valid) { p = g_pram; bc = g_pram_bcast; }
    }
    int abytes = ak == 0 ? 2 : 4, bbytes = bk == 0 ? 2 : 4, cbytes = ck == 0 ? 2 : 4;
    i64* row = (i64*)malloc(sizeof(i64) * n);
    for (u64 i2 = 0; i2 < c2; i2++)
        for (u64 i1 = 0; i1 < c1; i1++) {
            const uint8_t* ra = a + i2 * a_s2 + i1 * a_s1;
            const uint8_t* rb = b ? b + i2 * b_s2 + i1 * b_s1 : NULL;
            uint8_t* rc = c + i2 * c_s2 + i1 * c_s1;
            if (code == RO_XPOSE) {
                unsigned R = aux & 15, L = n;
                if (R == 0 || R > 8) continue;
                /* a tile of R rows (b_s1 apart) of L; column d becomes a granule of R at
                 * rc + d*b_s2 (ROWOPS_RTL_KERNEL.md 1.4 op 7) */
                for (unsigned d = 0; d < L; d++)
                    for (unsigned r = 0; r < R; r++)
                        wr_kind(rc + (u64)d * b_s2 + 2 * r, rd16(ra + (u64)r * b_s1 + 2ull * d), 0);
                if (b_s2 == 2 * R)
                    for (u64 o = 2ull * R * L; o % 16; o += 2) wr_kind(rc + o, 0, 0);
                continue;
            }
            if (code == RO_NORM) {
                int ln = (op & RO_LN) != 0;
                i128 S1 = 0, S2 = 0;
                for (unsigned j = 0; j < n; j++) {
                    row[j] = rd_kind(ra + (u64)abytes * j, ak);
                    S1 += row[j];
                    S2 += (i128)row[j] * row[j];
                }
                i128 D = ln ? ((i128)n * S2 - S1 * S1 + (i128)eps) : (S2 + (i128)eps);
                if (D <= 0) D = 1;
                u64 Rm; int sh;
                rsqrt_bf(D, &Rm, &sh);
                for (unsigned j = 0; j < n; j++) {
                    ro_param q = ro_read_param(p, j, bc);
                    i128 A = ln ? ((i128)n * row[j] - S1) : (i128)row[j];
                    i128 P1 = (A * (i128)Rm) >> (sh - 24);
                    i128 s = P1 * (i128)q.g + ((i128)q.bq << bq_sh);
                    wr_kind(rc + 2ull * j, sat16w(rne_shr128(s, q.sc)), 0);
                }
                for (u64 o = 2ull * n; o % 16; o += 2) wr_kind(rc + o, 0, 0);
                continue;
            }
            if (code == RO_ROPE) {
                unsigned HD = aux & 0xFFF, half = HD / 2;
                if (HD == 0 || (HD & 15) || HD > 128 || n % HD) { free(row); return 0; }
                for (unsigned j = 0; j < n; j++) row[j] = rd16(ra + 2ull * j);
                for (unsigned j = 0; j < n; j++) {
                    ro_param q = ro_read_param(p, j, bc);
                    unsigned d = j % HD;
                    i64 cs = rd32(rb + 4ull * d), sn = rd32(rb + 4ull * (HD + d));
                    i64 rot = d < half ? -row[j + half] : row[j - half];
                    i128 s = (((i128)row[j] * cs) << q.sa) + (((i128)rot * sn) << q.sb);
                    wr_kind(rc + 2ull * j, sat16w(rne_shr128(s, q.sc)), 0);
                }
                for (u64 o = 2ull * n; o % 16; o += 2) wr_kind(rc + o, 0, 0);
                continue;
            }
            if (code == RO_COPY || code == RO_ADDX || code == RO_DEQUANT || code == RO_MULACT ||
                code == RO_GATE) {
                int zero_a = (code == RO_COPY || code == RO_ADDX) && (i1 < win_lo || i1 >= win_hi);
                int cb = code == RO_DEQUANT ? 4 : cbytes;
                for (unsigned j = 0; j < n; j++) {
                    ro_param q = ro_read_param(p, j, bc);
                    i64 xv = zero_a ? 0 : rd_kind(ra + (u64)abytes * j, ak);
                    i64 yv = (ben && code != RO_DEQUANT) ? rd_kind(rb + (u64)bbytes * j, bk) : 0;
                    i64 r;
                    if (code == RO_COPY || code == RO_ADDX) {
                        i128 s = ((i128)xv << q.sa) + ((i128)yv << q.sb) + ((i128)q.bq << bq_sh);
                        i128 v = rne_shr128((op & RO_SCALE) ? s * (i128)q.g : s, q.sc);
                        r = ck == 0 ? sat16w(v) : sat32w(v);
                        if ((op & RO_RELU) && r < 0) r = 0;
                        wr_kind(rc + (u64)cbytes * j, r, ck == 0 ? 0 : 1);
                    } else if (code == RO_DEQUANT) {
                        r = (i64)ro_float_bits(xv, q.sc);
                        wr_kind(rc + 4ull * j, r, 1);
                    } else if (code == RO_GATE) {
                        i64 th = 2 * sig_q(xv << q.sa) - ((i64)1 << 24);
                        i64 sg = sig_q(yv << q.sb);
                        wr_kind(rc + (u64)cbytes * j, sat16w(rne_shr128((i128)th * sg, q.sc)), 0);
                    } else {
                        i64 gv = xv << q.sa;
                        wr_kind(rc + (u64)cbytes * j, sat16w(rne_shr128((i128)silu_q(gv) * yv, q.sc)), 0);
                    }
                }
                for (u64 o = (u64)cb * n; o % 16; o++) rc[o] = 0;
                continue;
            }
        }
    free(row);
    return 0;
}
