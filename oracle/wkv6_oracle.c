/*
 * CPU oracle for the RWKV-6 WKV recurrence (TEST INFRASTRUCTURE ONLY).
 *
 * This file is the checker, never the product: only tests/, the smoke test
 * and the cpu_baseline leg of bench.py load it.  The GPU path never calls it.
 *
 * It restates, in plain C with fp64 state, the naive recurrent RWKV-6 that
 * flash-linear-attention's `fused_recurrent_rwkv6` computes at the call site
 *   /root/reference/rwkv_megatron/rwkv6_layer_specs.py:339
 *     o = fused_recurrent_rwkv6(r, k, v, w, u, scale=1.)[0]
 * with the argument conventions fixed by the caller (:330-341):
 *   r, k, w : [B, H, T, K]   (w is LOG-space decay: the caller passes -exp(decay), :336)
 *   v       : [B, H, T, V]
 *   u       : [H, K]         (time_first reshaped per head, :337)
 *   h0, hT  : [B, H, K, V]   fp32 state
 * fla itself is an absent submodule (/root/reference/.gitmodules:1-3), so the
 * recurrence is the published RWKV-6 definition:
 *   o_t[j]    = s * sum_i r_t[i] * (S_{t-1}[i,j] + u[i] k_t[i] v_t[j])
 *   S_t[i,j]  = exp(w_t[i]) * S_{t-1}[i,j] + k_t[i] v_t[j]
 * and the backward is the exact reverse-time recurrence derived from it:
 *   dr_t[i]  = s * sum_j dO_t[j] (S_{t-1}[i,j] + u[i] k_t[i] v_t[j])
 *   dk_t[i]  = sum_j dS_t[i,j] v_t[j] + s r_t[i] u[i] (v_t . dO_t)
 *   dv_t[j]  = sum_i dS_t[i,j] k_t[i] + s (sum_i r_t[i] u[i] k_t[i]) dO_t[j]
 *   dw_t[i]  = exp(w_t[i]) sum_j S_{t-1}[i,j] dS_t[i,j]
 *   du[i]   += s r_t[i] k_t[i] (v_t . dO_t)
 *   dS_{t-1} = diag(exp(w_t)) dS_t + s r_t dO_t^T,   dS_T = dhT (or 0),  dh0 = dS_0
 * The backward recomputes S inside 64-step segments from fp64 checkpoints
 * instead of storing every state.
 *
 * Build: see oracle/Makefile (gcc -O2 -fopenmp -shared).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define SEG 64

static void set_threads(int nthreads) {
    if (nthreads > 0) omp_set_num_threads(nthreads);
}

int wkv6_oracle_max_threads(void) { return omp_get_max_threads(); }

/* Forward over one (b,h) sequence; S is a K*V fp64 scratch holding the state. */
static void fwd_one(const float* r, const float* k, const float* v, const float* w,
                    const float* u, const float* h0, double s, int64_t T, int64_t K,
                    int64_t V, float* o, float* hT, double* S) {
    if (h0) {
        for (int64_t e = 0; e < K * V; ++e) S[e] = h0[e];
    } else {
        memset(S, 0, sizeof(double) * K * V);
    }
    for (int64_t t = 0; t < T; ++t) {
        const float* rt = r + t * K;
        const float* kt = k + t * K;
        const float* vt = v + t * V;
        const float* wt = w + t * K;
        float* ot = o + t * V;
        double bonus = 0.0; /* sum_i r_t[i] u[i] k_t[i] */
        for (int64_t i = 0; i < K; ++i) bonus += (double)rt[i] * u[i] * kt[i];
        for (int64_t j = 0; j < V; ++j) {
            double acc = bonus * vt[j];
            for (int64_t i = 0; i < K; ++i) acc += (double)rt[i] * S[i * V + j];
            ot[j] = (float)(s * acc);
        }
        for (int64_t i = 0; i < K; ++i) {
            double d = exp((double)wt[i]);
            double ki = kt[i];
            double* Si = S + i * V;
            for (int64_t j = 0; j < V; ++j) Si[j] = d * Si[j] + ki * vt[j];
        }
    }
    if (hT)
        for (int64_t e = 0; e < K * V; ++e) hT[e] = (float)S[e];
}

void wkv6_oracle_fwd(const float* r, const float* k, const float* v, const float* w,
                     const float* u, const float* h0, float scale, int64_t B, int64_t H,
                     int64_t T, int64_t K, int64_t V, float* o, float* hT, int nthreads) {
    set_threads(nthreads);
#pragma omp parallel
    {
        double* S = (double*)malloc(sizeof(double) * K * V);
#pragma omp for schedule(dynamic, 1)
        for (int64_t bh = 0; bh < B * H; ++bh) {
            int64_t h = bh % H;
            fwd_one(r + bh * T * K, k + bh * T * K, v + bh * T * V, w + bh * T * K, u + h * K,
                    h0 ? h0 + bh * K * V : NULL, (double)scale, T, K, V, o + bh * T * V,
                    hT ? hT + bh * K * V : NULL, S);
        }
        free(S);
    }
}

/* Backward over one (b,h) sequence.  du_part is this sequence's [K] share of du. */
static void bwd_one(const float* r, const float* k, const float* v, const float* w,
                    const float* u, const float* h0, const float* dO, const float* dhT,
                    double s, int64_t T, int64_t K, int64_t V, float* dr, float* dk,
                    float* dv, float* dw, double* du_part, float* dh0, double* ckpt,
                    double* seg, double* dS) {
    const int64_t KV = K * V;
    const int64_t nseg = (T + SEG - 1) / SEG;
    /* forward sweep keeping the state at the start of every segment */
    double* S = seg; /* reuse the first slot as running state */
    if (h0) {
        for (int64_t e = 0; e < KV; ++e) S[e] = h0[e];
    } else {
        memset(S, 0, sizeof(double) * KV);
    }
    for (int64_t g = 0; g < nseg; ++g) {
        memcpy(ckpt + g * KV, S, sizeof(double) * KV);
        int64_t t1 = (g + 1) * SEG < T ? (g + 1) * SEG : T;
        for (int64_t t = g * SEG; t < t1; ++t) {
            for (int64_t i = 0; i < K; ++i) {
                double d = exp((double)w[t * K + i]);
                double ki = k[t * K + i];
                for (int64_t j = 0; j < V; ++j)
                    S[i * V + j] = d * S[i * V + j] + ki * v[t * V + j];
            }
        }
    }
    if (dhT) {
        for (int64_t e = 0; e < KV; ++e) dS[e] = dhT[e];
    } else {
        memset(dS, 0, sizeof(double) * KV);
    }
    for (int64_t i = 0; i < K; ++i) du_part[i] = 0.0;
    for (int64_t g = nseg - 1; g >= 0; --g) {
        int64_t t0 = g * SEG;
        int64_t t1 = (g + 1) * SEG < T ? (g + 1) * SEG : T;
        /* seg[(t - t0) * KV] = S_{t-1} (state before token t) */
        memcpy(seg, ckpt + g * KV, sizeof(double) * KV);
        for (int64_t t = t0; t + 1 < t1; ++t) {
            double* Sp = seg + (t - t0) * KV;
            double* Sn = Sp + KV;
            for (int64_t i = 0; i < K; ++i) {
                double d = exp((double)w[t * K + i]);
                double ki = k[t * K + i];
                for (int64_t j = 0; j < V; ++j)
                    Sn[i * V + j] = d * Sp[i * V + j] + ki * v[t * V + j];
            }
        }
        for (int64_t t = t1 - 1; t >= t0; --t) {
            const double* Sp = seg + (t - t0) * KV;
            const float* rt = r + t * K;
            const float* kt = k + t * K;
            const float* vt = v + t * V;
            const float* wt = w + t * K;
            const float* dot = dO + t * V;
            double dd = 0.0, bonus = 0.0;
            for (int64_t j = 0; j < V; ++j) dd += (double)dot[j] * vt[j];
            for (int64_t i = 0; i < K; ++i) bonus += (double)rt[i] * u[i] * kt[i];
            for (int64_t i = 0; i < K; ++i) {
                double acc_r = 0.0, acc_k = 0.0, acc_w = 0.0;
                for (int64_t j = 0; j < V; ++j) {
                    acc_r += (double)dot[j] * Sp[i * V + j];
                    acc_k += dS[i * V + j] * vt[j];
                    acc_w += Sp[i * V + j] * dS[i * V + j];
                }
                dr[t * K + i] = (float)(s * (acc_r + (double)u[i] * kt[i] * dd));
                dk[t * K + i] = (float)(acc_k + s * (double)rt[i] * u[i] * dd);
                dw[t * K + i] = (float)(exp((double)wt[i]) * acc_w);
                du_part[i] += s * (double)rt[i] * kt[i] * dd;
            }
            for (int64_t j = 0; j < V; ++j) {
                double acc = 0.0;
                for (int64_t i = 0; i < K; ++i) acc += dS[i * V + j] * kt[i];
                dv[t * V + j] = (float)(acc + s * bonus * dot[j]);
            }
            for (int64_t i = 0; i < K; ++i) {
                double d = exp((double)wt[i]);
                double sri = s * rt[i];
                for (int64_t j = 0; j < V; ++j) dS[i * V + j] = d * dS[i * V + j] + sri * dot[j];
            }
        }
    }
    if (dh0)
        for (int64_t e = 0; e < KV; ++e) dh0[e] = (float)dS[e];
}

void wkv6_oracle_bwd(const float* r, const float* k, const float* v, const float* w,
                     const float* u, const float* h0, const float* dO, const float* dhT,
                     float scale, int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                     float* dr, float* dk, float* dv, float* dw, float* du, float* dh0,
                     int nthreads) {
    set_threads(nthreads);
    const int64_t KV = K * V;
    const int64_t nseg = (T + SEG - 1) / SEG;
    double* du_parts = (double*)calloc((size_t)(B * H * K), sizeof(double));
#pragma omp parallel
    {
        double* ckpt = (double*)malloc(sizeof(double) * KV * (nseg > 0 ? nseg : 1));
        double* seg = (double*)malloc(sizeof(double) * KV * SEG);
        double* dS = (double*)malloc(sizeof(double) * KV);
#pragma omp for schedule(dynamic, 1)
        for (int64_t bh = 0; bh < B * H; ++bh) {
            int64_t h = bh % H;
            bwd_one(r + bh * T * K, k + bh * T * K, v + bh * T * V, w + bh * T * K, u + h * K,
                    h0 ? h0 + bh * KV : NULL, dO + bh * T * V, dhT ? dhT + bh * KV : NULL,
                    (double)scale, T, K, V, dr + bh * T * K, dk + bh * T * K, dv + bh * T * V,
                    dw + bh * T * K, du_parts + bh * K, dh0 ? dh0 + bh * KV : NULL, ckpt, seg,
                    dS);
        }
        free(ckpt);
        free(seg);
        free(dS);
    }
    /* du[h, i] = sum_b du_part[b, h, i], in a fixed order */
    for (int64_t h = 0; h < H; ++h)
        for (int64_t i = 0; i < K; ++i) {
            double acc = 0.0;
            for (int64_t b = 0; b < B; ++b) acc += du_parts[(b * H + h) * K + i];
            du[h * K + i] = (float)acc;
        }
    free(du_parts);
}
