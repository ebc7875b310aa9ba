"""CPU restatements of three row-ops nodes' ``reference()`` for the graph-level checker: the
Transpose on the unit (a numpy transpose), LlmAttnPrep on the unit (RoPE of q / k, the V
re-round, the q.K^T x image, the cache rows) and VitAttnPrep on the unit (the bias adds into
the q image and the caches).  TEST INFRASTRUCTURE ONLY (the checker,
never the thing measured or shipped).  Nothing here imports the product: the spec functions
are restated from inference-scheduler/src/rowops_spec.py.
"""
import numpy as np

ROPE_BITS = 23                         # cos / sin as int24 at 2^-23 (rowops_spec.py:263)
I16_LO, I16_HI = -32768, 32767


def sat16(v):
    return np.clip(v, I16_LO, I16_HI)


def rne_shr_vec(v, k):
    """Round half to even of v / 2^k with a per-element shift k >= 0 (rowops_spec.py:292-300)."""
    v = np.asarray(v, np.int64)
    k = np.broadcast_to(np.asarray(k, np.int64), v.shape)
    kk = np.maximum(k, 1)
    q = v >> kk
    r = v - (q << kk)
    half = np.int64(1) << (kk - 1)
    up = (r > half) | ((r == half) & ((q & 1) == 1))
    return np.where(k > 0, q + up, v)


def rope_tables_raw(cos, sin):
    """int24 at 2^-23 of float cos / sin tables (rowops_spec.py:267-271)."""
    return (np.rint(np.asarray(cos, np.float64) * 2.0 ** ROPE_BITS).astype(np.int64),
            np.rint(np.asarray(sin, np.float64) * 2.0 ** ROPE_BITS).astype(np.int64))


def rope(x_raw, f_x, c_raw, s_raw, f_out):
    """Rotate-half RoPE of int16 x [T][nh][HD] at 2^-f_x (per head or per channel) with int24
    cos / sin rows [T][HD] into int16 at 2^-f_out: one rounding of the exact sum x c + rot(x) s,
    both products first shifted to the finer exponent of their pair (rowops_spec.py:303-322)."""
    x_raw = np.asarray(x_raw, np.int64)
    T, nh, HD = x_raw.shape
    half = HD // 2
    f_x = np.asarray(f_x, np.int64)
    f_x = np.broadcast_to(f_x[:, None] if f_x.ndim == 1 else f_x, (nh, HD))
    f_out = np.asarray(f_out, np.int64)
    f_out = np.broadcast_to(f_out[:, None] if f_out.ndim == 1 else f_out, (nh, HD))
    f_rot = np.concatenate([f_x[:, half:], f_x[:, :half]], axis=1)
    fp = np.maximum(f_x, f_rot)
    rot = np.concatenate([-x_raw[..., half:], x_raw[..., :half]], axis=-1)
    num = (((x_raw * c_raw[:, None, :]) << (fp - f_x)[None])
           + ((rot * s_raw[:, None, :]) << (fp - f_rot)[None]))
    return sat16(rne_shr_vec(num, (fp + ROPE_BITS - f_out)[None]))


def clamp_n(pos, n, T, C, q=16):
    """(valid rows, keys) as llm_nodes.attn_keys (llm_nodes.py:960-968)."""
    n = max(0, min(int(n), T, C - int(pos))) if int(pos) < C else 0
    k = -(-(int(pos) + n) // q) * q
    return n, max(q, min(k, C))


def attn_prep(q0, k0, v, pos, n, ck, cv, f_q0, f_k0, f_v, f_kc, f_vc, fq, cos, sin, H, KV, HD, Q=16):
    """AttnPrepRoNode.reference (rowops_nodes.py:1111-1131) on float64 values: returns the q.K^T x
    image qx [KV][HD][G T] (raw integers: the conv input image); the logical caches ck / cv
    [C][KV HD] (values) receive rows [pos, pos + n) in place.  f_*: per-channel exponents of q0
    [H HD], k0 / v / the caches [KV HD]; fq: one per head."""
    G = H // KV
    T = np.asarray(q0).size // (H * HD)
    C = ck.shape[0]
    n, _ = clamp_n(pos, n, T, C, Q)
    qx = np.zeros((KV, HD, G * T))
    if n == 0:
        return qx
    p2 = lambda e: np.power(2.0, np.asarray(e, np.float64))            # noqa: E731
    cos2 = np.concatenate([np.asarray(cos, np.float32)] * 2, 1).astype(np.float64)
    sin2 = np.concatenate([np.asarray(sin, np.float32)] * 2, 1).astype(np.float64)
    cr, sr = rope_tables_raw(cos2, sin2)
    q0 = np.asarray(q0, np.float64).reshape(T, H * HD)[:n]
    k0 = np.asarray(k0, np.float64).reshape(T, KV * HD)[:n]
    v = np.asarray(v, np.float64).reshape(T, KV * HD)[:n]
    xq = np.rint(q0 * p2(f_q0)[None, :]).astype(np.int64).reshape(n, H, HD)
    xk = np.rint(k0 * p2(f_k0)[None, :]).astype(np.int64).reshape(n, KV, HD)
    f_kc = np.asarray(f_kc, np.int64).reshape(KV, HD)
    yq = rope(xq, np.asarray(f_q0, np.int64).reshape(H, HD), cr[pos:pos + n], sr[pos:pos + n], np.asarray(fq))
    yk = rope(xk, np.asarray(f_k0, np.int64).reshape(KV, HD), cr[pos:pos + n], sr[pos:pos + n], f_kc)
    ck[pos:pos + n] = yk.reshape(n, -1) / p2(f_kc.reshape(-1))[None, :]
    vr = np.rint(v * p2(f_v)[None, :]).astype(np.int64)
    sa = np.maximum(np.asarray(f_vc, np.int64) - np.asarray(f_v, np.int64), 0)
    sc = np.maximum(np.asarray(f_v, np.int64) - np.asarray(f_vc, np.int64), 0)
    cv[pos:pos + n] = sat16(rne_shr_vec(vr << sa[None, :], sc[None, :])) / p2(f_vc)[None, :]
    for h in range(H):
        g, hh = divmod(h, G)
        qx[g, :, hh * T:hh * T + n] = yq[:, h, :].T                      # raw integers
    return qx


def transpose(x, perm):
    """TransposeRoNode.reference (rowops_nodes.py:293-295): numpy's transpose, a bit copy."""
    return np.ascontiguousarray(np.transpose(np.asarray(x), perm))


def bias_round(x_raw, f_x, bias, f_out):
    """A COPY with a bias (rowops_spec.py:195-203): per column sat16(rne_shr((x << (fp - f_x)) +
    round(bias 2^fp), fp - f_out)) with fp = bias_exp (the bias rounded once at 2^-fp)."""
    from oracle.rowops_adapt import bias_params
    x_raw = np.asarray(x_raw, np.int64)
    bq, sa, sc = bias_params(bias, f_x, f_out)
    return sat16(rne_shr_vec((x_raw << sa[None, :]) + bq[None, :], sc[None, :]))


def vit_attn_prep(q_raw, k_raw, v_raw, f_q0, f_k0, f_v0, bq, bk, bv, fq, fk, fv, H, HD, query_major=False):
    """VitAttnPrepRoNode.reference (rowops_nodes.py:1570-1593) without RoPE or key rows, on raw
    int16 rows [T][H HD] at their column exponents: (qx [H][HD][T], K cache rows [T][H HD],
    V cache rows [T][H HD]) -- k0 + bk at f_k per head into the K cache, v + bv at f_v per
    column into the V cache, q0 + bq at f_q per head transposed per head into qx; with
    ``query_major`` k takes the image path and q the K cache rows."""
    T = np.asarray(q_raw).shape[0]
    if query_major:
        q_raw, k_raw, f_q0, f_k0, bq, bk, fq, fk = k_raw, q_raw, f_k0, f_q0, bk, bq, fk, fq
    ck = bias_round(k_raw, f_k0, bk, np.repeat(np.asarray(fk, np.int64), HD))
    cv = bias_round(v_raw, f_v0, bv, fv)
    yq = bias_round(q_raw, f_q0, bq, np.repeat(np.asarray(fq, np.int64), HD))
    return yq.reshape(T, H, HD).transpose(1, 2, 0).copy(), ck, cv
