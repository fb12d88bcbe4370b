/*
 * qff_oracle_impl.h -- body of the CPU oracle, instantiated twice by
 * qff_oracle.c: once with R = float (the reference's own fp32 loop order)
 * and once with R = double (an fp64 "truth" used to size rounding error).
 *
 * TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this code, and only as the checker.
 *
 * Every function cites the reference file:line it restates. Paths are
 * relative to Sources/QwenFieldfareCore/ of the reference:
 *   LA   = Kernels/LinearAttention/QwenDeltaNetKernel.swift
 *   DN   = Metal/LinearAttention/deltanet.metal
 *   ATT  = Metal/Attention/attention.metal
 *   AW   = Kernels/Attention/Attention.swift
 *   RUN  = Runtime/Generation/QwenQ4ActiveExpertStreamingRunner.swift
 *
 * Macros expected from the includer: R (real type), SFX(name) (suffixes the
 * exported name), EXP/LOG1P/SQRT/FMA/COS/SIN/POW (math for R).
 */

/* ---- scalar activations: LA:5-20 (softplus uses log1p as the CPU path
 *      does; DN:12-16 writes log(1+exp(x)), identical up to rounding) ---- */
static inline R SFX(silu_)(R x) { return x / ((R)1 + EXP(-x)); }
static inline R SFX(sigmoid_)(R x) { return (R)1 / ((R)1 + EXP(-x)); }
static inline R SFX(softplus_)(R x) {
    if (x > (R)20) return x;
    if (x < (R)-20) return EXP(x);
    return LOG1P(EXP(x));
}

R SFX(qffo_silu)(R x) { return SFX(silu_)(x); }
R SFX(qffo_sigmoid)(R x) { return SFX(sigmoid_)(x); }
R SFX(qffo_softplus)(R x) { return SFX(softplus_)(x); }

/* ---- RMSNorm: LA:22-37 multiplies by (1 + w); the Metal input/head norms
 *      (DN:18-53, DN:614-632) multiply by w. `one_plus_w` selects. ---- */
void SFX(qffo_rmsnorm)(const R* x, const R* w, int d, R eps, int one_plus_w, R* out) {
    R ss = 0;
    for (int i = 0; i < d; ++i) ss += x[i] * x[i];
    R inv = (R)1 / SQRT(ss / (R)d + eps);
    for (int i = 0; i < d; ++i)
        out[i] = x[i] * inv * (one_plus_w ? ((R)1 + w[i]) : w[i]);
}

/* ---- row-major matvec: LA:153-167 (vDSP_mmul, [rows, cols] x [cols]) ---- */
void SFX(qffo_matvec)(const R* w, const R* x, int rows, int cols, R* y) {
    for (int r = 0; r < rows; ++r) {
        R acc = 0;
        for (int c = 0; c < cols; ++c) acc += w[(size_t)r * cols + c] * x[c];
        y[r] = acc;
    }
}

/* ---- causal depthwise conv, kernel 4: LA:39-59, DN:112-138.
 *      state is [dim][4]; slots 1..3 shift to 0..2, the new token goes to
 *      slot 3, out = silu(sum_j state[j] * w[j]) summed left to right. ---- */
void SFX(qffo_conv1d_step)(const R* in, R* state, const R* w, int dim, R* out) {
    for (int i = 0; i < dim; ++i) {
        R* s = state + (size_t)i * 4;
        const R* wi = w + (size_t)i * 4;
        s[0] = s[1]; s[1] = s[2]; s[2] = s[3]; s[3] = in[i];
        R acc = s[0] * wi[0] + s[1] * wi[1] + s[2] * wi[2] + s[3] * wi[3];
        out[i] = SFX(silu_)(acc);
    }
}

/* ---- L2 normalisation: LA:61-71, inv = 1/sqrt(sum(v^2) + eps) ---- */
void SFX(qffo_l2norm)(const R* v, int d, R eps, R* out) {
    R ss = 0;
    for (int i = 0; i < d; ++i) ss += v[i] * v[i];
    R inv = (R)1 / SQRT(ss + eps);
    for (int i = 0; i < d; ++i) out[i] = v[i] * inv;
}

/* ---- gated delta-rule step: LA:73-125. q, k, v are [32][128] (already
 *      expanded to v-heads), state is [32][128 rows = v][128 cols = k].
 *      Per head: decay the whole state, then per row kv = S_r.k,
 *      delta = (v_r - kv) * beta, S_r += k * delta; then o_r = S_r.q. ---- */
/* One value head of that step (LA:86-120 for one h): qh, kh, vh [128],
 * a, b the head's gate inputs, S [128][128], out [128]. */
void SFX(qffo_deltanet_head_step)(const R* qh, const R* kh, const R* vh, R a, R b,
                                  R a_log, R dt_bias, R* S, R* out) {
    R beta = SFX(sigmoid_)(b);
    R g = EXP(-EXP(a_log) * SFX(softplus_)(a + dt_bias));
    for (int i = 0; i < 128 * 128; ++i) S[i] *= g;
    for (int r = 0; r < 128; ++r) {
        R kv = 0;
        for (int c = 0; c < 128; ++c) kv += S[r * 128 + c] * kh[c];
        R delta = (vh[r] - kv) * beta;
        for (int c = 0; c < 128; ++c) S[r * 128 + c] += kh[c] * delta;
    }
    for (int r = 0; r < 128; ++r) {
        R o = 0;
        for (int c = 0; c < 128; ++c) o += S[r * 128 + c] * qh[c];
        out[r] = o;
    }
}

void SFX(qffo_deltanet_recurrent_step)(const R* q, const R* k, const R* v,
                                       const R* a, const R* b, const R* a_log,
                                       const R* dt_bias, R* state, R* out) {
    for (int h = 0; h < 32; ++h)
        SFX(qffo_deltanet_head_step)(q + h * 128, k + h * 128, v + h * 128, a[h], b[h],
                                     a_log[h], dt_bias[h], state + (size_t)h * 128 * 128,
                                     out + h * 128);
}

/* ---- gated RMSNorm: LA:127-151. out = o * inv * w_r * silu(z) ---- */
void SFX(qffo_gated_rmsnorm)(const R* core, const R* w, const R* z, R eps, R* out) {
    for (int h = 0; h < 32; ++h) {
        const R* c = core + h * 128;
        R ss = 0;
        for (int r = 0; r < 128; ++r) ss += c[r] * c[r];
        R inv = (R)1 / SQRT(ss / (R)128 + eps);
        for (int r = 0; r < 128; ++r)
            out[h * 128 + r] = c[r] * inv * w[r] * SFX(silu_)(z[h * 128 + r]);
    }
}

/* ---- one DeltaNet layer core for one token: LA:178-255 steps 3-6
 *      (conv, split + repeat-interleave q/k to 32 heads with head map h/2
 *      at LA:212-215, L2 norm, q scaled by 1/sqrt(128) at LA:210, the
 *      recurrent step, gated RMSNorm). The in/out projections of that
 *      function are separate oracle entries (matvec, q4). ----
 *   qkv [8192] pre-conv projection output, z [4096], a, b [32]
 *   conv_w [8192][4], norm_w [128], conv_state [8192][4],
 *   ssm [32][128][128] -> out [4096] */
void SFX(qffo_deltanet_token)(const R* qkv, const R* z, const R* a, const R* b,
                              const R* a_log, const R* dt_bias, const R* conv_w,
                              const R* norm_w, R eps, R* conv_state, R* ssm,
                              R* out) {
    R conv[8192];
    R q[32 * 128], k[32 * 128], v[32 * 128], core[32 * 128];
    SFX(qffo_conv1d_step)(qkv, conv_state, conv_w, 8192, conv);
    const R q_scale = (R)1 / SQRT((R)128);
    for (int h = 0; h < 32; ++h) {
        int src = h / 2;
        R tmp[128];
        SFX(qffo_l2norm)(conv + src * 128, 128, (R)1e-6, tmp);
        for (int i = 0; i < 128; ++i) q[h * 128 + i] = tmp[i] * q_scale;
        SFX(qffo_l2norm)(conv + 2048 + src * 128, 128, (R)1e-6, k + h * 128);
        for (int i = 0; i < 128; ++i) v[h * 128 + i] = conv[4096 + h * 128 + i];
    }
    SFX(qffo_deltanet_recurrent_step)(q, k, v, a, b, a_log, dt_bias, ssm, core);
    SFX(qffo_gated_rmsnorm)(core, norm_w, z, eps, out);
}

/* ---- T tokens of one sequence, one at a time: the reference has no
 *      prefill path and feeds prompts token by token (RUN:1545-1561).
 *      qkv [T][8192], z [T][4096], a, b [T][32] -> out [T][4096]. ---- */
void SFX(qffo_deltanet_sequence)(int T, const R* qkv, const R* z, const R* a,
                                 const R* b, const R* a_log, const R* dt_bias,
                                 const R* conv_w, const R* norm_w, R eps,
                                 R* conv_state, R* ssm, R* out) {
    for (int t = 0; t < T; ++t)
        SFX(qffo_deltanet_token)(qkv + (size_t)t * 8192, z + (size_t)t * 4096,
                                 a + (size_t)t * 32, b + (size_t)t * 32, a_log,
                                 dt_bias, conv_w, norm_w, eps, conv_state, ssm,
                                 out + (size_t)t * 4096);
}

/* ---- per-head RMSNorm with weight w: DN:614-632 ---- */
void SFX(qffo_head_rmsnorm)(R* x, const R* w, int nheads, int hd, R eps) {
    for (int h = 0; h < nheads; ++h) {
        R* xh = x + (size_t)h * hd;
        R ss = 0;
        for (int i = 0; i < hd; ++i) ss += xh[i] * xh[i];
        R inv = (R)1 / SQRT(ss / (R)hd + eps);
        for (int i = 0; i < hd; ++i) xh[i] = xh[i] * inv * w[i];
    }
}

/* ---- RoPE tables: RUN:1090-1099. freq_i = 1/theta^(2i/rot),
 *      angle = pos * freq_i, entries i and rot/2+i share the angle. ---- */
void SFX(qffo_rope_tables)(int pos, R theta, int rot, R* cos_t, R* sin_t) {
    int half = rot / 2;
    for (int i = 0; i < half; ++i) {
        R freq = (R)1 / POW(theta, (R)(2 * i) / (R)rot);
        R angle = (R)pos * freq;
        R c = COS(angle), s = SIN(angle);
        cos_t[i] = c; cos_t[half + i] = c;
        sin_t[i] = s; sin_t[half + i] = s;
    }
}

/* ---- partial rotate-half RoPE on the first `rot` dims: DN:634-651 ---- */
void SFX(qffo_rope_partial)(R* x, const R* cos_t, const R* sin_t, int nheads,
                            int hd, int rot) {
    int half = rot / 2;
    for (int h = 0; h < nheads; ++h) {
        R* xh = x + (size_t)h * hd;
        for (int i = 0; i < half; ++i) {
            R x0 = xh[i], x1 = xh[half + i];
            xh[i] = x0 * cos_t[i] + (-x1) * sin_t[i];
            xh[half + i] = x1 * cos_t[half + i] + x0 * sin_t[half + i];
        }
    }
}

/* ---- split-KV decode attention for one token: AW:129-157 (geometry
 *      NC = min(16, L), chunk = ceil(L / NC)), ATT:134-224 (partial: per
 *      position a 256-wide dot reduced as 8 sums of 32, scaled, online
 *      softmax) and ATT:342-377 (combine). q [nq][hd], K/V [L][nkv][hd]
 *      as real values (already rounded to the cache dtype) -> out [nq][hd]
 *      before the reference's final half() cast. num_chunks <= 0 selects
 *      the reference geometry; 1 gives the single-pass recurrence. ---- */
/* One q head of it (kv head kvh): qh [hd] -> out_h [hd]. */
void SFX(qffo_attention_decode_head)(const R* qh, const R* K, const R* V, int L,
                                     int nkv, int kvh, int hd, R scale, int num_chunks,
                                     R* out_h) {
    int NC = num_chunks > 0 ? num_chunks : (L < 16 ? (L < 1 ? 1 : L) : 16);
    int chunk_len = ((L < 1 ? 1 : L) + NC - 1) / NC;
    R* m_p = (R*)malloc(sizeof(R) * NC);
    R* d_p = (R*)malloc(sizeof(R) * NC);
    R* o_p = (R*)malloc(sizeof(R) * NC * hd);
    R* o_l = (R*)malloc(sizeof(R) * hd);
    {
        for (int c = 0; c < NC; ++c) {
            int p0 = c * chunk_len, p1 = p0 + chunk_len;
            if (p1 > L) p1 = L;
            R m = -(R)INFINITY, d = 0;
            for (int i = 0; i < hd; ++i) o_l[i] = 0;
            for (int p = p0; p < p1; ++p) {
                const R* kr = K + ((size_t)p * nkv + kvh) * hd;
                const R* vr = V + ((size_t)p * nkv + kvh) * hd;
                R s = 0;
                for (int g = 0; g < hd; g += 32) {
                    R part = 0;
                    for (int l = g; l < g + 32 && l < hd; ++l) part += qh[l] * kr[l];
                    s += part;
                }
                s *= scale;
                R m_new = m > s ? m : s;
                R alpha = EXP(m - m_new);
                R pe = EXP(s - m_new);
                d = d * alpha + pe;
                for (int i = 0; i < hd; ++i) o_l[i] = o_l[i] * alpha + pe * vr[i];
                m = m_new;
            }
            m_p[c] = m; d_p[c] = d;
            for (int i = 0; i < hd; ++i) o_p[(size_t)c * hd + i] = o_l[i];
        }
        R mg = -(R)INFINITY;
        for (int c = 0; c < NC; ++c) mg = mg > m_p[c] ? mg : m_p[c];
        R D = 0;
        for (int c = 0; c < NC; ++c) D += d_p[c] * EXP(m_p[c] - mg);
        R inv_d = D > 0 ? (R)1 / D : (R)0;
        for (int i = 0; i < hd; ++i) {
            R acc = 0;
            for (int c = 0; c < NC; ++c) acc += o_p[(size_t)c * hd + i] * EXP(m_p[c] - mg);
            out_h[i] = acc * inv_d;
        }
    }
    free(m_p); free(d_p); free(o_p); free(o_l);
}

void SFX(qffo_attention_decode)(const R* q, const R* K, const R* V, int L,
                                int nq, int nkv, int hd, R scale, int num_chunks,
                                R* out) {
    for (int h = 0; h < nq; ++h)
        SFX(qffo_attention_decode_head)(q + (size_t)h * hd, K, V, L, nkv, h / (nq / nkv), hd,
                                        scale, num_chunks, out + (size_t)h * hd);
}

/* ---- Q4 affine matvec, factored order of the generic kernel DN:816-861:
 *      per group of 64, dot = fma(q, x, dot), sum += x, then
 *      acc = fma(dot, scale, fma(sum, bias, acc)).
 *      w [rows][cols/8] u32, scales/biases [rows][cols/64] as reals. ---- */
void SFX(qffo_q4_matvec)(const uint32_t* w, const R* scales, const R* biases,
                         const R* x, int rows, int cols, R* y) {
    int groups = cols / 64;
    for (int r = 0; r < rows; ++r) {
        const uint32_t* wr = w + (size_t)r * (cols / 8);
        R acc = 0;
        for (int g = 0; g < groups; ++g) {
            R s = scales[(size_t)r * groups + g], bb = biases[(size_t)r * groups + g];
            R dot = 0, sum = 0;
            for (int u = 0; u < 8; ++u) {
                uint32_t word = wr[g * 8 + u];
                for (int n = 0; n < 8; ++n) {
                    R xv = x[g * 64 + u * 8 + n];
                    dot = FMA((R)((word >> (4 * n)) & 0xFu), xv, dot);
                    sum += xv;
                }
            }
            acc = FMA(dot, s, FMA(sum, bb, acc));
        }
        y[r] = acc;
    }
}
