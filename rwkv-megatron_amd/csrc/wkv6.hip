// WKV6 forward / backward for MI355X (gfx950), K = V = 64.
//
// Replaces fla's fused_recurrent_rwkv6 / chunk_rwkv6 as called at
// /root/reference/rwkv_megatron/rwkv6_layer_specs.py:339.  The recurrence is
//   o_t = s * r_t^T (S_{t-1} + diag(u) k_t v_t^T),   S_t = diag(exp(w_t)) S_{t-1} + k_t v_t^T.
//
// Decomposition (three phases each way, all deterministic):
//   fwd_chunk_state  per (b,h,chunk): S_loc = sum_tau (k_tau e^{G_63 - G_tau}) v_tau^T  [MFMA]
//   state_scan_fwd   per (b,h,elem) : S_in(c+1) = e^{G_63(c)} S_in(c) + S_loc(c)  fp32, coalesced
//   fwd_chunk_output per (b,h,chunk): o = (r e^{G_{t-1}}) S_in + intra-chunk attention   [MFMA]
//   bwd_chunk_dstate per (b,h,chunk): dS_loc = s * sum_t (r_t e^{G_{t-1}}) dO_t^T        [MFMA]
//   state_scan_bwd   per (b,h,elem) : dS_out(c-1) = e^{G_63(c)} dS_out(c) + dS_loc(c)
//   bwd_chunk_grads  per (b,h,chunk): dr, dk, dv, dw, du-partials                        [MFMA]
//
// Inside a 64-token chunk G is the inclusive cumulative log-decay (kept in base-2
// units).  The intra-chunk attention A[t,tau] = sum_i r_t k_tau e^{G_{t-1}-G_tau}
// is evaluated per 16x16 sub-block with bf16 MFMA on factorised operands:
//   off-diagonal blocks use a reference point between source and target block,
//   so both factors are <= 1; diagonal blocks use the block midpoint, so each
//   factor is bounded by the decay of 8 tokens (finite while 8 consecutive
//   log-decays sum to > -88, i.e. |w| < ~11 per token).
// Every MFMA accumulates in fp32; the carried states are fp32.  In the dr / dk
// contractions the decay-scaled operand is split into bf16 hi + lo parts: dw is a
// cancelling suffix sum of r*dr - k*dk, and single-bf16 operands there would
// dominate its error.
#include "common.h"
#include "../../include/rwkv6_amd.h"

#define KD 64            // head size (K == V)
#define CL 64            // chunk length (tokens)
#define TS 72            // LDS row stride of a bf16 64x64 tile (elements): 144 B rows
#define GS 68            // LDS row stride of a token-major fp32 tile
#define GXS 68           // LDS row stride of a channel-major fp32 tile (65 used)
#define NTHR 256

typedef uint16_t tile_t[CL][TS];
typedef float gtile_t[CL][GS];

// ---------------------------------------------------------------------------
// tile movement
// ---------------------------------------------------------------------------

// Global [64 rows][64] bf16 (rows contiguous, 128 B each) -> LDS, optionally also
// transposed.  Rows >= nvalid read as zero.
__device__ __forceinline__ void load_tile(uint16_t (*tok)[TS], uint16_t (*tr)[TS],
                                          const uint16_t* __restrict__ src, int nvalid) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        int idx = p * NTHR + threadIdx.x;
        int row = idx >> 3, c8 = (idx & 7) * 8;
        uint4 val = make_uint4(0u, 0u, 0u, 0u);
        if (row < nvalid) val = *reinterpret_cast<const uint4*>(src + (size_t)row * KD + c8);
        if (tok) *reinterpret_cast<uint4*>(&tok[row][c8]) = val;
        if (tr) {
            uint32_t wv[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                tr[c8 + 2 * s][row] = (uint16_t)(wv[s] & 0xffffu);
                tr[c8 + 2 * s + 1][row] = (uint16_t)(wv[s] >> 16);
            }
        }
    }
}

// Token-major LDS tile -> global (rows < nvalid).
__device__ __forceinline__ void store_tile(uint16_t* __restrict__ dst, uint16_t (*tok)[TS],
                                           int nvalid) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        int idx = p * NTHR + threadIdx.x;
        int row = idx >> 3, c8 = (idx & 7) * 8;
        if (row < nvalid)
            *reinterpret_cast<uint4*>(dst + (size_t)row * KD + c8) =
                *reinterpret_cast<const uint4*>(&tok[row][c8]);
    }
}

// Inclusive cumulative log2-decay over the 64 tokens of a chunk, from a
// token-major bf16 w tile.  Writes token-major Gm[t][i] and/or channel-major
// shifted GtX[i][t+1] = G[t] with GtX[i][0] = 0 (so GtX[i][t] = G[t-1]).
// `tot` is 256 floats of scratch.  Ends with a barrier.
__device__ __forceinline__ void build_G(uint16_t (*Wm)[TS], float (*Gm)[GS],
                                        float (*GtX)[GXS], float* tot) {
    int i = threadIdx.x & 63, part = threadIdx.x >> 6;
    float loc[16];
    float run = 0.f;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        run += bf2f(Wm[16 * part + s][i]) * RW_L2E;
        loc[s] = run;
    }
    tot[part * 64 + i] = run;
    __syncthreads();
    float off = 0.f;
    for (int p = 0; p < part; ++p) off += tot[p * 64 + i];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        float g = loc[s] + off;
        if (Gm) Gm[16 * part + s][i] = g;
        if (GtX) GtX[i][16 * part + s + 1] = g;
    }
    if (GtX && part == 0) GtX[i][0] = 0.f;
    __syncthreads();
}

__device__ __forceinline__ float load_u(const void* u, int u_dtype, int idx) {
    return u_dtype == RWKV6_BF16 ? bf2f(reinterpret_cast<const uint16_t*>(u)[idx])
                                 : reinterpret_cast<const float*>(u)[idx];
}

// sum_i a[t][i] * b[t][i] * (u ? u[i] : 1) for each token t (256 threads, 4 per token).
__device__ __forceinline__ float row_dot(uint16_t (*A)[TS], uint16_t (*Bm)[TS], const float* u,
                                         int t, int q) {
    float f[8], g[8], acc = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        int c0 = 16 * q + 8 * h;
        unpack8(*reinterpret_cast<const uint4*>(&A[t][c0]), f);
        unpack8(*reinterpret_cast<const uint4*>(&Bm[t][c0]), g);
#pragma unroll
        for (int s = 0; s < 8; ++s) acc += f[s] * g[s] * (u ? u[c0 + s] : 1.f);
    }
    return warp_sum4(acc);
}

// ---------------------------------------------------------------------------
// phase A (forward): chunk-local state and chunk decay
// ---------------------------------------------------------------------------
// S_loc[i][j] = sum_tau k[tau][i] e^{G_63[i]-G_tau[i]} v[tau][j]   (fp32 out)
// decay[i]    = e^{G_63[i]}
__global__ void __launch_bounds__(NTHR)
wkv6_fwd_chunk_state(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                     const uint16_t* __restrict__ w, float* __restrict__ Sloc,
                     float* __restrict__ decay, int T, int NT) {
    __shared__ __attribute__((aligned(16))) tile_t Kt, Vt, Wm;
    __shared__ __attribute__((aligned(16))) float GtX[KD][GXS];
    __shared__ float tot[256];
    const int c = blockIdx.x, bh = blockIdx.y;
    const int t0 = c * CL, nvalid = min(CL, T - t0);
    const size_t base = ((size_t)bh * T + t0) * KD;
    load_tile(nullptr, Kt, k + base, nvalid);
    load_tile(nullptr, Vt, v + base, nvalid);
    load_tile(Wm, nullptr, w + base, nvalid);
    __syncthreads();
    build_G(Wm, nullptr, GtX, tot);

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int i = 16 * wv + lr;
    const float g63 = GtX[i][64];
    f32x4 acc[4] = {};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int tau0 = 32 * ks + 8 * lq;
        float kf[8];
        unpack8(*reinterpret_cast<const uint4*>(&Kt[i][tau0]), kf);
        bf16x8 a;
#pragma unroll
        for (int s = 0; s < 8; ++s) a[s] = (__bf16)(kf[s] * ex2(g63 - GtX[i][tau0 + s + 1]));
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) acc[tj] = mfma32(a, ld_bf16x8(&Vt[16 * tj + lr][tau0]), acc[tj]);
    }
    float* out = Sloc + ((size_t)bh * NT + c) * KD * KD;
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) out[(16 * wv + 4 * lq + rr) * KD + 16 * tj + lr] = acc[tj][rr];
    if (threadIdx.x < KD)
        decay[((size_t)bh * NT + c) * KD + threadIdx.x] = ex2(GtX[threadIdx.x][64]);
}

// ---------------------------------------------------------------------------
// phase B: state scans (fp32, one thread per state element, coalesced)
// ---------------------------------------------------------------------------
// Hs[c] = bf16(S_in(c)) for c = 0..NT (Hs[NT] = final state); hT = S_in(NT) fp32.
__global__ void __launch_bounds__(NTHR)
wkv6_state_scan_fwd(const float* __restrict__ Sloc, const float* __restrict__ decay,
                    const float* __restrict__ h0, uint16_t* __restrict__ Hs,
                    float* __restrict__ hT, int NT) {
    const int bh = blockIdx.x >> 4;
    const int e = ((blockIdx.x & 15) << 8) + threadIdx.x;
    const int i = e >> 6;
    float S = h0 ? h0[(size_t)bh * KD * KD + e] : 0.f;
    const float* sl = Sloc + (size_t)bh * NT * KD * KD + e;
    const float* dc = decay + (size_t)bh * NT * KD + i;
    uint16_t* hs = Hs + (size_t)bh * (NT + 1) * KD * KD + e;
    int c = 0;
    for (; c + 4 <= NT; c += 4) {
        float l0 = sl[(size_t)(c + 0) * KD * KD], l1 = sl[(size_t)(c + 1) * KD * KD];
        float l2 = sl[(size_t)(c + 2) * KD * KD], l3 = sl[(size_t)(c + 3) * KD * KD];
        float d0 = dc[(c + 0) * KD], d1 = dc[(c + 1) * KD], d2 = dc[(c + 2) * KD], d3 = dc[(c + 3) * KD];
        hs[(size_t)(c + 0) * KD * KD] = f2bf(S); S = d0 * S + l0;
        hs[(size_t)(c + 1) * KD * KD] = f2bf(S); S = d1 * S + l1;
        hs[(size_t)(c + 2) * KD * KD] = f2bf(S); S = d2 * S + l2;
        hs[(size_t)(c + 3) * KD * KD] = f2bf(S); S = d3 * S + l3;
    }
    for (; c < NT; ++c) {
        hs[(size_t)c * KD * KD] = f2bf(S);
        S = dc[c * KD] * S + sl[(size_t)c * KD * KD];
    }
    hs[(size_t)NT * KD * KD] = f2bf(S);
    if (hT) hT[(size_t)bh * KD * KD + e] = S;
}

// dHs[c] = bf16(dS_out(c)) (gradient w.r.t. the state after chunk c); dh0 = dS_in(0).
__global__ void __launch_bounds__(NTHR)
wkv6_state_scan_bwd(const float* __restrict__ dSloc, const float* __restrict__ decay,
                    const float* __restrict__ dhT, uint16_t* __restrict__ dHs,
                    float* __restrict__ dh0, int NT) {
    const int bh = blockIdx.x >> 4;
    const int e = ((blockIdx.x & 15) << 8) + threadIdx.x;
    const int i = e >> 6;
    float dS = dhT ? dhT[(size_t)bh * KD * KD + e] : 0.f;
    const float* sl = dSloc + (size_t)bh * NT * KD * KD + e;
    const float* dc = decay + (size_t)bh * NT * KD + i;
    uint16_t* hs = dHs + (size_t)bh * NT * KD * KD + e;
    int c = NT - 1;
    for (; c - 3 >= 0; c -= 4) {
        float l0 = sl[(size_t)(c - 0) * KD * KD], l1 = sl[(size_t)(c - 1) * KD * KD];
        float l2 = sl[(size_t)(c - 2) * KD * KD], l3 = sl[(size_t)(c - 3) * KD * KD];
        float d0 = dc[(c - 0) * KD], d1 = dc[(c - 1) * KD], d2 = dc[(c - 2) * KD], d3 = dc[(c - 3) * KD];
        hs[(size_t)(c - 0) * KD * KD] = f2bf(dS); dS = d0 * dS + l0;
        hs[(size_t)(c - 1) * KD * KD] = f2bf(dS); dS = d1 * dS + l1;
        hs[(size_t)(c - 2) * KD * KD] = f2bf(dS); dS = d2 * dS + l2;
        hs[(size_t)(c - 3) * KD * KD] = f2bf(dS); dS = d3 * dS + l3;
    }
    for (; c >= 0; --c) {
        hs[(size_t)c * KD * KD] = f2bf(dS);
        dS = dc[c * KD] * dS + sl[(size_t)c * KD * KD];
    }
    if (dh0) dh0[(size_t)bh * KD * KD + e] = dS;
}

// ---------------------------------------------------------------------------
// phase C (forward): chunk output
// ---------------------------------------------------------------------------
// Wave W owns target tokens t in [16W, 16W+16) and all 64 value columns.
//   o_t = s [ (r_t e^{G_{t-1}}) S_in + sum_{J<W} A_WJ v_J + A_WW v_W ]
// A_WJ (J<W): factors r_t e^{G_{t-1}-b_W} and k_tau e^{b_W-G_tau}, b_W = G_{16W-1}
// A_WW      : factors around mu_W = G_{16W+7}, strictly causal, u-bonus on the diagonal.
__global__ void __launch_bounds__(NTHR)
wkv6_fwd_chunk_output(const uint16_t* __restrict__ r, const uint16_t* __restrict__ k,
                      const uint16_t* __restrict__ v, const uint16_t* __restrict__ w,
                      const void* __restrict__ u, int u_dtype, const uint16_t* __restrict__ Hs,
                      uint16_t* __restrict__ o, float scale, int H, int T, int NT) {
    __shared__ __attribute__((aligned(16))) tile_t Rm, Km, Vt, Wm, St;
    __shared__ __attribute__((aligned(16))) gtile_t Gm;
    __shared__ float tot[256];
    __shared__ float us[KD], bonus[CL];
    const int c = blockIdx.x, bh = blockIdx.y, h = bh % H;
    const int t0 = c * CL, nvalid = min(CL, T - t0);
    const size_t base = ((size_t)bh * T + t0) * KD;
    load_tile(Rm, nullptr, r + base, nvalid);
    load_tile(Km, nullptr, k + base, nvalid);
    load_tile(nullptr, Vt, v + base, nvalid);
    load_tile(Wm, nullptr, w + base, nvalid);
    load_tile(nullptr, St, Hs + ((size_t)bh * (NT + 1) + c) * KD * KD, KD);   // St[j][i] = S_in[i][j]
    if (threadIdx.x < KD) us[threadIdx.x] = load_u(u, u_dtype, h * KD + threadIdx.x);
    __syncthreads();
    {
        float bsum = row_dot(Rm, Km, us, threadIdx.x >> 2, threadIdx.x & 3);
        if ((threadIdx.x & 3) == 0) bonus[threadIdx.x >> 2] = bsum;
    }
    build_G(Wm, Gm, nullptr, tot);

    const int lane = threadIdx.x & 63, W = threadIdx.x >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int t = 16 * W + lr;                    // this lane's target row for A/B fragments
    f32x4 acc[4] = {};
    // inter-chunk: (r_t e^{G_{t-1}}) S_in
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int i0 = 32 * ks + 8 * lq;
        float rf[8];
        unpack8(*reinterpret_cast<const uint4*>(&Rm[t][i0]), rf);
        bf16x8 a;
#pragma unroll
        for (int s = 0; s < 8; ++s) a[s] = (__bf16)(rf[s] * (t > 0 ? ex2(Gm[t - 1][i0 + s]) : 1.f));
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) acc[tj] = mfma32(a, ld_bf16x8(&St[16 * tj + lr][i0]), acc[tj]);
    }
    // intra-chunk sub-blocks J <= W
    for (int J = 0; J <= W; ++J) {
        const bool diag = (J == W);
        const int refrow = diag ? 16 * W + 7 : 16 * W - 1;     // b_W or mu_W (W>0 when !diag)
        const int tau = 16 * J + lr;
        f32x4 at = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int i0 = 32 * ks + 8 * lq;
            float kf[8], rf[8];
            unpack8(*reinterpret_cast<const uint4*>(&Km[tau][i0]), kf);
            unpack8(*reinterpret_cast<const uint4*>(&Rm[t][i0]), rf);
            bf16x8 ka, rb;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const float ref = Gm[refrow][i0 + s];
                ka[s] = (__bf16)(kf[s] * ex2(ref - Gm[tau][i0 + s]));
                const float gm1 = t > 0 ? Gm[t - 1][i0 + s] : 0.f;
                rb[s] = (__bf16)(rf[s] * ex2(gm1 - ref));
            }
            at = mfma32(ka, rb, at);      // at[rr] = A^T[tau = 16J+4lq+rr][t = 16W+lr]
        }
        bf16x4 aop;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            float x = at[rr];
            if (diag) {
                const int tl = 4 * lq + rr;              // source index within the block
                x = tl < lr ? x : (tl == lr ? bonus[t] : 0.f);
            }
            aop[rr] = (__bf16)x;
        }
#pragma unroll
        for (int tj = 0; tj < 4; ++tj)
            acc[tj] = mfma16(aop, ld_bf16x4(&Vt[16 * tj + lr][16 * J + 4 * lq]), acc[tj]);
    }
    // stage this wave's 16 rows through its own rows of Rm, then coalesced store
    __syncthreads();
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) Rm[16 * W + 4 * lq + rr][16 * tj + lr] = f2bf(scale * acc[tj][rr]);
    __syncthreads();
    store_tile(o + base, Rm, nvalid);
}

// ---------------------------------------------------------------------------
// phase A (backward): chunk-local dstate
// ---------------------------------------------------------------------------
// dS_loc[i][j] = s * sum_t r[t][i] e^{G_{t-1}[i]} dO[t][j]
__global__ void __launch_bounds__(NTHR)
wkv6_bwd_chunk_dstate(const uint16_t* __restrict__ r, const uint16_t* __restrict__ w,
                      const uint16_t* __restrict__ dO, float* __restrict__ dSloc, float scale,
                      int T, int NT) {
    __shared__ __attribute__((aligned(16))) tile_t Rt, Dt, Wm;
    __shared__ __attribute__((aligned(16))) float GtX[KD][GXS];
    __shared__ float tot[256];
    const int c = blockIdx.x, bh = blockIdx.y;
    const int t0 = c * CL, nvalid = min(CL, T - t0);
    const size_t base = ((size_t)bh * T + t0) * KD;
    load_tile(nullptr, Rt, r + base, nvalid);
    load_tile(nullptr, Dt, dO + base, nvalid);
    load_tile(Wm, nullptr, w + base, nvalid);
    __syncthreads();
    build_G(Wm, nullptr, GtX, tot);

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int i = 16 * wv + lr;
    f32x4 acc[4] = {};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int tt0 = 32 * ks + 8 * lq;
        float rf[8];
        unpack8(*reinterpret_cast<const uint4*>(&Rt[i][tt0]), rf);
        bf16x8 a;
#pragma unroll
        for (int s = 0; s < 8; ++s) a[s] = (__bf16)(rf[s] * ex2(GtX[i][tt0 + s]));   // G_{t-1}
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) acc[tj] = mfma32(a, ld_bf16x8(&Dt[16 * tj + lr][tt0]), acc[tj]);
    }
    float* out = dSloc + ((size_t)bh * NT + c) * KD * KD;
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
            out[(16 * wv + 4 * lq + rr) * KD + 16 * tj + lr] = scale * acc[tj][rr];
}

// ---------------------------------------------------------------------------
// phase C (backward): gradients of one chunk
// ---------------------------------------------------------------------------
// Wave W owns tokens [16W, 16W+16): as target (dr) and as source (dk, dv).
// With dA[t][tau] = dO_t . v_tau, s = scale, S_in / S_out the states before / after
// the chunk and dS_out the gradient of S_out:
//   dr_h[t] = s e^{G_{t-1}-b_W} (S_in e^{b_W} dO_t + sum_{J<W} dA k e^{b_W-G})
//           + s e^{G_{t-1}-mu_W} sum_{tau in W, tau<t} dA k e^{mu_W-G}
//   dk_h[tau] = e^{e_W-G_tau} (dS_out e^{G_63-e_W} v_tau + s sum_{I>W} dA r e^{G_{t-1}-e_W})
//             + e^{mu_W-G_tau} s sum_{t in W, t>tau} dA r e^{G_{t-1}-mu_W}
//   dv[tau] = (k_tau e^{G_63-G_tau}) dS_out + s sum_{t>=tau} A[t][tau] dO_t
//   dr = dr_h + s u k dd,  dk = dk_h + s u r dd,  dd_t = dO_t . v_t
//   dw[t] = sum_{m>t} (r dr_h - k dk_h)[m] - k_t dk_h[t] + D,  D = rowsum(S_out * dS_out)
//   du_part = s sum_t r_t k_t dd_t
struct BwdSmem {
    tile_t Rm, Km, Vm, Dm, Rt, Kt, Dt, Sm, dSm, dSt;
    gtile_t Gm;
    float GtX[KD][GXS];
    float tot[256];
    float us[KD], bonus[CL], dd[CL], Dv[KD];
};

__global__ void __launch_bounds__(NTHR)
wkv6_bwd_chunk_grads(const uint16_t* __restrict__ r, const uint16_t* __restrict__ k,
                     const uint16_t* __restrict__ v, const uint16_t* __restrict__ w,
                     const void* __restrict__ u, int u_dtype, const uint16_t* __restrict__ dO,
                     const uint16_t* __restrict__ Hs, const uint16_t* __restrict__ dHs,
                     uint16_t* __restrict__ dr, uint16_t* __restrict__ dk,
                     uint16_t* __restrict__ dv, uint16_t* __restrict__ dw,
                     float* __restrict__ du_part, float scale, int H, int T, int NT) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
    BwdSmem& sm = *reinterpret_cast<BwdSmem*>(smem_raw);
    const int c = blockIdx.x, bh = blockIdx.y, h = bh % H;
    const int t0 = c * CL, nvalid = min(CL, T - t0);
    const size_t base = ((size_t)bh * T + t0) * KD;
    load_tile(sm.Rm, sm.Rt, r + base, nvalid);
    load_tile(sm.Km, sm.Kt, k + base, nvalid);
    load_tile(sm.Vm, nullptr, v + base, nvalid);
    load_tile(sm.Dm, sm.Dt, dO + base, nvalid);
    // w goes through the dS^T tile as scratch before the states are loaded
    load_tile(sm.dSt, nullptr, w + base, nvalid);
    load_tile(sm.Sm, nullptr, Hs + ((size_t)bh * (NT + 1) + c) * KD * KD, KD);
    if (threadIdx.x < KD) sm.us[threadIdx.x] = load_u(u, u_dtype, h * KD + threadIdx.x);
    __syncthreads();
    {
        const int tq = threadIdx.x >> 2, q = threadIdx.x & 3;
        float bsum = row_dot(sm.Rm, sm.Km, sm.us, tq, q);
        float dsum = row_dot(sm.Dm, sm.Vm, nullptr, tq, q);
        if (q == 0) {
            sm.bonus[tq] = bsum;
            sm.dd[tq] = dsum;
        }
    }
    // G in both layouts (build_G ends with a barrier; it also publishes bonus/dd)
    {
        // build_G reads w from the scratch tile
        build_G(sm.dSt, sm.Gm, sm.GtX, sm.tot);
    }
    // now the states: dS_out in both layouts (overwrites the w scratch)
    load_tile(sm.dSm, sm.dSt, dHs + ((size_t)bh * NT + c) * KD * KD, KD);
    // du partial: s * sum_t r k dd  (thread: channel i, 16 tokens)
    {
        const int i = threadIdx.x & 63, part = threadIdx.x >> 6;
        float acc = 0.f;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int tt = 16 * part + s;
            acc += bf2f(sm.Rt[i][tt]) * bf2f(sm.Kt[i][tt]) * sm.dd[tt];
        }
        sm.tot[part * 64 + i] = acc;
    }
    __syncthreads();
    if (threadIdx.x < KD) {
        const int i = threadIdx.x;
        du_part[((size_t)bh * NT + c) * KD + i] =
            scale * (sm.tot[i] + sm.tot[64 + i] + sm.tot[128 + i] + sm.tot[192 + i]);
    }
    // D[i] = sum_j S_out[i][j] dS_out[i][j], S_out = Hs[c+1]
    {
        const int i = threadIdx.x >> 2, q = threadIdx.x & 3;
        const uint16_t* so = Hs + ((size_t)bh * (NT + 1) + c + 1) * KD * KD + i * KD + 16 * q;
        float f[8], g[8], acc = 0.f;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            unpack8(*reinterpret_cast<const uint4*>(so + 8 * hh), f);
            unpack8(*reinterpret_cast<const uint4*>(&sm.dSm[i][16 * q + 8 * hh]), g);
#pragma unroll
            for (int s = 0; s < 8; ++s) acc += f[s] * g[s];
        }
        acc = warp_sum4(acc);
        if (q == 0) sm.Dv[i] = acc;
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, W = threadIdx.x >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int rowW = 16 * W + lr;              // this lane's fragment row in block W
    const float* bW = W > 0 ? sm.Gm[16 * W - 1] : nullptr;
    const float* muW = sm.Gm[16 * W + 7];
    const float* eW = sm.Gm[16 * W + 15];
    const float* g63 = sm.Gm[63];

    // ---------------- dr (target rows t in W) ----------------
    f32x4 accR[4] = {}, accRd[4] = {};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int j0 = 32 * ks + 8 * lq;
        const bf16x8 a = ld_bf16x8(&sm.Dm[rowW][j0]);
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) {
            const int i = 16 * ti + lr;
            const float sc = bW ? ex2(bW[i]) : 1.f;
            float sf[8];
            unpack8(*reinterpret_cast<const uint4*>(&sm.Sm[i][j0]), sf);
#pragma unroll
            for (int s = 0; s < 8; ++s) sf[s] *= sc;
            bf16x8 bh, bl;
            split_bf16<8>(sf, bh, bl);
            accR[ti] = mfma32(a, bh, accR[ti]);
            accR[ti] = mfma32(a, bl, accR[ti]);
        }
    }
    for (int J = 0; J <= W; ++J) {
        const bool diag = (J == W);
        f32x4 at = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int j0 = 32 * ks + 8 * lq;
            at = mfma32(ld_bf16x8(&sm.Vm[16 * J + lr][j0]), ld_bf16x8(&sm.Dm[rowW][j0]), at);
        }
        // at[rr] = dA[t = 16W+lr][tau = 16J+4lq+rr]
        bf16x4 aop;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            float x = at[rr];
            if (diag && 4 * lq + rr >= lr) x = 0.f;
            aop[rr] = (__bf16)x;
        }
        const float* ref = diag ? muW : bW;
        const int tau0 = 16 * J + 4 * lq;
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) {
            const int i = 16 * ti + lr;
            float kf[4];
            unpack4(*reinterpret_cast<const uint2*>(&sm.Kt[i][tau0]), kf);
#pragma unroll
            for (int s = 0; s < 4; ++s) kf[s] *= ex2(ref[i] - sm.GtX[i][tau0 + s + 1]);
            bf16x4 bh, bl;
            split_bf16<4>(kf, bh, bl);
            if (diag) {
                accRd[ti] = mfma16(aop, bh, accRd[ti]);
                accRd[ti] = mfma16(aop, bl, accRd[ti]);
            } else {
                accR[ti] = mfma16(aop, bh, accR[ti]);
                accR[ti] = mfma16(aop, bl, accR[ti]);
            }
        }
    }
    // ---------------- dk (source rows tau in W) ----------------
    f32x4 accK[4] = {}, accKd[4] = {};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int j0 = 32 * ks + 8 * lq;
        const bf16x8 a = ld_bf16x8(&sm.Vm[rowW][j0]);
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) {
            const int i = 16 * ti + lr;
            const float sc = ex2(g63[i] - eW[i]);
            float sf[8];
            unpack8(*reinterpret_cast<const uint4*>(&sm.dSm[i][j0]), sf);
#pragma unroll
            for (int s = 0; s < 8; ++s) sf[s] *= sc;
            bf16x8 bh, bl;
            split_bf16<8>(sf, bh, bl);
            accK[ti] = mfma32(a, bh, accK[ti]);
            accK[ti] = mfma32(a, bl, accK[ti]);
        }
    }
    for (int I = W; I < 4; ++I) {
        const bool diag = (I == W);
        f32x4 at = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int j0 = 32 * ks + 8 * lq;
            at = mfma32(ld_bf16x8(&sm.Dm[16 * I + lr][j0]), ld_bf16x8(&sm.Vm[rowW][j0]), at);
        }
        // at[rr] = dA[t = 16I+4lq+rr][tau = 16W+lr]
        bf16x4 aop;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            float x = at[rr] * scale;
            if (diag && 4 * lq + rr <= lr) x = 0.f;
            aop[rr] = (__bf16)x;
        }
        const float* ref = diag ? muW : eW;
        const int tt0 = 16 * I + 4 * lq;
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) {
            const int i = 16 * ti + lr;
            float rf[4];
            unpack4(*reinterpret_cast<const uint2*>(&sm.Rt[i][tt0]), rf);
#pragma unroll
            for (int s = 0; s < 4; ++s) rf[s] *= ex2(sm.GtX[i][tt0 + s] - ref[i]);
            bf16x4 bh, bl;
            split_bf16<4>(rf, bh, bl);
            if (diag) {
                accKd[ti] = mfma16(aop, bh, accKd[ti]);
                accKd[ti] = mfma16(aop, bl, accKd[ti]);
            } else {
                accK[ti] = mfma16(aop, bh, accK[ti]);
                accK[ti] = mfma16(aop, bl, accK[ti]);
            }
        }
    }
    // ---------------- dv (source rows tau in W) ----------------
    f32x4 accV[4] = {};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int i0 = 32 * ks + 8 * lq;
        float kf[8];
        unpack8(*reinterpret_cast<const uint4*>(&sm.Km[rowW][i0]), kf);
        bf16x8 a;
#pragma unroll
        for (int s = 0; s < 8; ++s) a[s] = (__bf16)(kf[s] * ex2(g63[i0 + s] - sm.Gm[rowW][i0 + s]));
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) accV[tj] = mfma32(a, ld_bf16x8(&sm.dSt[16 * tj + lr][i0]), accV[tj]);
    }
    for (int I = W; I < 4; ++I) {
        const bool diag = (I == W);
        const float* ref = diag ? muW : eW;
        const int trow = 16 * I + lr;
        f32x4 at = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int i0 = 32 * ks + 8 * lq;
            float rf[8], kf[8];
            unpack8(*reinterpret_cast<const uint4*>(&sm.Rm[trow][i0]), rf);
            unpack8(*reinterpret_cast<const uint4*>(&sm.Km[rowW][i0]), kf);
            bf16x8 ra, kb;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const float gm1 = trow > 0 ? sm.Gm[trow - 1][i0 + s] : 0.f;
                ra[s] = (__bf16)(rf[s] * ex2(gm1 - ref[i0 + s]));
                kb[s] = (__bf16)(kf[s] * ex2(ref[i0 + s] - sm.Gm[rowW][i0 + s]));
            }
            at = mfma32(ra, kb, at);       // at[rr] = A[t = 16I+4lq+rr][tau = 16W+lr]
        }
        bf16x4 aop;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            float x = at[rr];
            if (diag) {
                const int tl = 4 * lq + rr;
                x = tl > lr ? x : (tl == lr ? sm.bonus[16 * W + lr] : 0.f);
            }
            aop[rr] = (__bf16)(x * scale);
        }
#pragma unroll
        for (int tj = 0; tj < 4; ++tj)
            accV[tj] = mfma16(aop, ld_bf16x4(&sm.Dt[16 * tj + lr][16 * I + 4 * lq]), accV[tj]);
    }

    // ---------------- epilogue ----------------
    // Accumulator element (lq, rr) of tile ti sits at token 16W+4lq+rr, channel 16ti+lr.
    float drh[4][4], dkh[4][4], xv[4][4], yv[4][4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
        const int i = 16 * ti + lr;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int tt = 16 * W + 4 * lq + rr;
            const float gm1 = sm.GtX[i][tt], g = sm.GtX[i][tt + 1];
            const float fR = bW ? ex2(gm1 - bW[i]) : ex2(gm1);
            drh[ti][rr] = scale * (fR * accR[ti][rr] + ex2(gm1 - muW[i]) * accRd[ti][rr]);
            dkh[ti][rr] = ex2(eW[i] - g) * accK[ti][rr] + ex2(muW[i] - g) * accKd[ti][rr];
            const float rv = bf2f(sm.Rt[i][tt]), kv = bf2f(sm.Kt[i][tt]);
            xv[ti][rr] = rv * drh[ti][rr] - kv * dkh[ti][rr];
            yv[ti][rr] = sm.Dv[i] - kv * dkh[ti][rr];
        }
    }
    __syncthreads();     // every wave is done with the MFMA operand tiles
    float (*Xs)[GS] = sm.Gm;                                            // x  (fp32)
    float (*Ys)[GXS] = sm.GtX;                                          // y  (fp32)
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
        const int i = 16 * ti + lr;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int tt = 16 * W + 4 * lq + rr;
            const float rv = bf2f(sm.Rm[tt][i]), kv = bf2f(sm.Km[tt][i]);
            const float sdd = scale * sm.dd[tt] * sm.us[i];
            Xs[tt][i] = xv[ti][rr];
            Ys[tt][i] = yv[ti][rr];
            sm.Rt[tt][i] = f2bf(drh[ti][rr] + sdd * kv);              // dr staging
            sm.Kt[tt][i] = f2bf(dkh[ti][rr] + sdd * rv);              // dk staging
        }
    }
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sm.Sm[16 * W + 4 * lq + rr][16 * tj + lr] = f2bf(accV[tj][rr]);
    __syncthreads();
    // dw: suffix sums over tokens, thread = (channel i, 16-token part)
    {
        const int i = threadIdx.x & 63, part = threadIdx.x >> 6;
        float tsum = 0.f;
#pragma unroll
        for (int s = 0; s < 16; ++s) tsum += Xs[16 * part + s][i];
        sm.tot[part * 64 + i] = tsum;
        __syncthreads();
        float run = 0.f;          // sum_{m > t} x[m]
        for (int p = part + 1; p < 4; ++p) run += sm.tot[p * 64 + i];
#pragma unroll
        for (int s = 15; s >= 0; --s) {
            const int tt = 16 * part + s;
            sm.Dt[tt][i] = f2bf(run + Ys[tt][i]);
            run += Xs[tt][i];
        }
    }
    __syncthreads();
    store_tile(dr + base, sm.Rt, nvalid);
    store_tile(dk + base, sm.Kt, nvalid);
    store_tile(dv + base, sm.Sm, nvalid);
    store_tile(dw + base, sm.Dt, nvalid);
}

// du[h][i] = sum_b sum_c du_part[b,h,c,i].  Thread (i, q): strided partial sum over the
// B*NT (b, c) pairs with p = q mod 4, then a fixed-order combine (deterministic).
__global__ void __launch_bounds__(NTHR)
wkv6_du_reduce(const float* __restrict__ du_part, void* __restrict__ du, int u_dtype, int B,
               int H, int NT) {
    __shared__ float part[4][KD];
    const int h = blockIdx.x, i = threadIdx.x & 63, q = threadIdx.x >> 6;
    float acc = 0.f;
    const int P = B * NT;
    for (int p = q; p < P; p += 4) {
        const int b = p / NT, c = p - b * NT;
        acc += du_part[((size_t)(b * H + h) * NT + c) * KD + i];
    }
    part[q][i] = acc;
    __syncthreads();
    if (q == 0) {
        const float tot = (part[0][i] + part[1][i]) + (part[2][i] + part[3][i]);
        if (u_dtype == RWKV6_BF16) reinterpret_cast<uint16_t*>(du)[h * KD + i] = f2bf(tot);
        else reinterpret_cast<float*>(du)[h * KD + i] = tot;
    }
}

// ---------------------------------------------------------------------------
// host side: C ABI
// ---------------------------------------------------------------------------
namespace {

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int64_t nchunks(int64_t T) { return (T + CL - 1) / CL; }
inline size_t round_up(size_t x) { return (x + 255) & ~(size_t)255; }

int check_shape(int64_t B, int64_t H, int64_t T, int64_t K, int64_t V) {
    if (B < 1 || H < 1 || T < 0 || K < 1 || V < 1) return RWKV6_ERR_INVALID_ARG;
    if (K != KD || V != KD) return RWKV6_ERR_UNSUPPORTED;
    if (B * H > 65535) return RWKV6_ERR_UNSUPPORTED;                  // grid.y limit
    if (T > ((int64_t)1 << 30)) return RWKV6_ERR_UNSUPPORTED;
    return RWKV6_OK;
}

int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? RWKV6_OK : RWKV6_ERR_LAUNCH;
}

// Records phase_events[i] (a hipEvent_t) on the stream when the caller asked for timing.
inline void mark(void* const* ev, int i, hipStream_t s) {
    if (ev && ev[i]) (void)hipEventRecord(reinterpret_cast<hipEvent_t>(ev[i]), s);
}

}  // namespace

extern "C" {

size_t rwkv6_wkv_saved_bytes(int64_t B, int64_t H, int64_t T, int64_t K, int64_t V) {
    if (check_shape(B, H, T, K, V) != RWKV6_OK) return 0;
    const int64_t NT = nchunks(T);
    return round_up((size_t)(B * H) * (NT + 1) * KD * KD * 2) +
           round_up((size_t)(B * H) * (NT > 0 ? NT : 1) * KD * 4);
}

size_t rwkv6_wkv_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                                 int for_bwd) {
    if (check_shape(B, H, T, K, V) != RWKV6_OK) return 0;
    const size_t BH = (size_t)(B * H), NT = (size_t)(nchunks(T) > 0 ? nchunks(T) : 1);
    size_t sz = round_up(BH * NT * KD * KD * 4);                       // S_loc / dS_loc (fp32)
    if (for_bwd) sz += round_up(BH * NT * KD * KD * 2) + round_up(BH * NT * KD * 4);   // dHs, du_part
    return sz;
}

int rwkv6_wkv_fwd_ex(const void* r, const void* k, const void* v, const void* w, const void* u,
                     int u_dtype, const float* h0, void* o, float* hT, void* saved,
                     void* workspace, int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                     float scale, void* stream, void* const* phase_events) {
    int st = check_shape(B, H, T, K, V);
    if (st != RWKV6_OK) return st;
    if (u_dtype != RWKV6_F32 && u_dtype != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    if (!u || !saved || (T > 0 && (!r || !k || !v || !w || !o || !workspace)))
        return RWKV6_ERR_INVALID_ARG;
    if (!al16(r) || !al16(k) || !al16(v) || !al16(w) || !al16(o) || !al16(saved) ||
        !al16(workspace) || (h0 && !al16(h0)) || (hT && !al16(hT)))
        return RWKV6_ERR_ALIGNMENT;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t NT = nchunks(T);
    const int BH = (int)(B * H);
    uint16_t* Hs = reinterpret_cast<uint16_t*>(saved);
    float* decay = reinterpret_cast<float*>(reinterpret_cast<char*>(saved) +
                                            round_up((size_t)BH * (NT + 1) * KD * KD * 2));
    float* Sloc = reinterpret_cast<float*>(workspace);
    mark(phase_events, 0, s);
    if (NT > 0) {
        dim3 grid((unsigned)NT, (unsigned)BH);
        hipLaunchKernelGGL(wkv6_fwd_chunk_state, grid, dim3(NTHR), 0, s,
                           (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)w, Sloc, decay,
                           (int)T, (int)NT);
    }
    mark(phase_events, 1, s);
    mark(phase_events, 2, s);
    hipLaunchKernelGGL(wkv6_state_scan_fwd, dim3((unsigned)BH * 16), dim3(NTHR), 0, s, Sloc, decay,
                       h0, Hs, hT, (int)NT);
    mark(phase_events, 3, s);
    mark(phase_events, 4, s);
    if (NT > 0) {
        dim3 grid((unsigned)NT, (unsigned)BH);
        hipLaunchKernelGGL(wkv6_fwd_chunk_output, grid, dim3(NTHR), 0, s, (const uint16_t*)r,
                           (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)w, u, u_dtype,
                           (const uint16_t*)Hs, (uint16_t*)o, scale, (int)H, (int)T, (int)NT);
    }
    mark(phase_events, 5, s);
    return launch_status();
}

int rwkv6_wkv_bwd_ex(const void* r, const void* k, const void* v, const void* w, const void* u,
                     int u_dtype, const void* dO, const float* dhT, const void* saved, void* dr,
                     void* dk, void* dv, void* dw, void* du, float* dh0, void* workspace,
                     int64_t B, int64_t H, int64_t T, int64_t K, int64_t V, float scale,
                     void* stream, void* const* phase_events) {
    int st = check_shape(B, H, T, K, V);
    if (st != RWKV6_OK) return st;
    if (u_dtype != RWKV6_F32 && u_dtype != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    if (!u || !du || !saved || !workspace ||
        (T > 0 && (!r || !k || !v || !w || !dO || !dr || !dk || !dv || !dw)))
        return RWKV6_ERR_INVALID_ARG;
    if (!al16(r) || !al16(k) || !al16(v) || !al16(w) || !al16(dO) || !al16(saved) ||
        !al16(dr) || !al16(dk) || !al16(dv) || !al16(dw) || !al16(workspace) ||
        (dhT && !al16(dhT)) || (dh0 && !al16(dh0)))
        return RWKV6_ERR_ALIGNMENT;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t NT = nchunks(T);
    const int BH = (int)(B * H);
    const uint16_t* Hs = reinterpret_cast<const uint16_t*>(saved);
    const float* decay = reinterpret_cast<const float*>(
        reinterpret_cast<const char*>(saved) + round_up((size_t)BH * (NT + 1) * KD * KD * 2));
    const size_t NTa = (size_t)(NT > 0 ? NT : 1);
    float* dSloc = reinterpret_cast<float*>(workspace);
    uint16_t* dHs = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(workspace) +
                                                round_up((size_t)BH * NTa * KD * KD * 4));
    float* du_part = reinterpret_cast<float*>(reinterpret_cast<char*>(dHs) +
                                              round_up((size_t)BH * NTa * KD * KD * 2));
    mark(phase_events, 0, s);
    if (NT > 0) {
        dim3 grid((unsigned)NT, (unsigned)BH);
        hipLaunchKernelGGL(wkv6_bwd_chunk_dstate, grid, dim3(NTHR), 0, s, (const uint16_t*)r,
                           (const uint16_t*)w, (const uint16_t*)dO, dSloc, scale, (int)T, (int)NT);
    }
    mark(phase_events, 1, s);
    mark(phase_events, 2, s);
    hipLaunchKernelGGL(wkv6_state_scan_bwd, dim3((unsigned)BH * 16), dim3(NTHR), 0, s, dSloc,
                       decay, dhT, dHs, dh0, (int)NT);
    mark(phase_events, 3, s);
    if (NT > 0) {
        dim3 grid((unsigned)NT, (unsigned)BH);
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(wkv6_bwd_chunk_grads),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)sizeof(BwdSmem)) != hipSuccess)
            return RWKV6_ERR_LAUNCH;
        mark(phase_events, 4, s);
        hipLaunchKernelGGL(wkv6_bwd_chunk_grads, grid, dim3(NTHR), sizeof(BwdSmem), s,
                           (const uint16_t*)r, (const uint16_t*)k, (const uint16_t*)v,
                           (const uint16_t*)w, u, u_dtype, (const uint16_t*)dO, Hs,
                           (const uint16_t*)dHs, (uint16_t*)dr, (uint16_t*)dk, (uint16_t*)dv,
                           (uint16_t*)dw, du_part, scale, (int)H, (int)T, (int)NT);
        mark(phase_events, 5, s);
        mark(phase_events, 6, s);
        hipLaunchKernelGGL(wkv6_du_reduce, dim3((unsigned)H), dim3(NTHR), 0, s, du_part, du, u_dtype,
                           (int)B, (int)H, (int)NT);
        mark(phase_events, 7, s);
    } else {
        if (hipMemsetAsync(du, 0, (size_t)H * KD * (u_dtype == RWKV6_BF16 ? 2 : 4), s) != hipSuccess)
            return RWKV6_ERR_LAUNCH;
    }
    return launch_status();
}

int rwkv6_wkv_fwd(const void* r, const void* k, const void* v, const void* w, const void* u,
                  int u_dtype, const float* h0, void* o, float* hT, void* saved,
                  void* workspace, int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                  float scale, void* stream) {
    return rwkv6_wkv_fwd_ex(r, k, v, w, u, u_dtype, h0, o, hT, saved, workspace, B, H, T, K, V,
                            scale, stream, nullptr);
}

int rwkv6_wkv_bwd(const void* r, const void* k, const void* v, const void* w, const void* u,
                  int u_dtype, const void* dO, const float* dhT, const void* saved, void* dr,
                  void* dk, void* dv, void* dw, void* du, float* dh0, void* workspace,
                  int64_t B, int64_t H, int64_t T, int64_t K, int64_t V, float scale,
                  void* stream) {
    return rwkv6_wkv_bwd_ex(r, k, v, w, u, u_dtype, dO, dhT, saved, dr, dk, dv, dw, du, dh0,
                            workspace, B, H, T, K, V, scale, stream, nullptr);
}

}  // extern "C"
