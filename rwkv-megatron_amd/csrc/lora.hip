// The LoRA bottlenecks of RWKV6TimeMix fused with what consumes their output, for MI355X
// (gfx950).  Sequence-first [T,B,C] bf16, N = T*B tokens.
//
// Reference (/root/reference/rwkv_megatron/rwkv6_layer_specs.py):
//   bottleneck(x) = tanh(x W_down) W_up + bias          :177-195 (W_up [E,R,C], bias [E,C])
//   token shift:  E = 5, R = 32, m = bottleneck(xxx)     :364-369, :446
//                 mixed_e = x + (shift(x) - x) * m_e     :447-452
//   decay:        E = 1, R = 64, decay = bottleneck(mixed_w)  :370-375, :454
// The down-projection and tanh stay a hipBLASLt GEMM (N x C x E*R, output ~5 MB).  The
// up-projection is a K = R contraction whose [E,N,C] output is the big tensor, so it is
// computed here on MFMA and consumed in registers:
//   rwkv6_ddlerp_lora_fwd  writes the five mixes directly (no m round trip through HBM);
//   rwkv6_lora_bias_fwd    writes m + bias, the bottleneck's own output [N,E,C] (for E = 1
//                          the decay of :454);
//   rwkv6_ddlerp_lora_bwd  recomputes m and writes d_mexp = d_mixed * delta (the LoRA GEMMs'
//                          input), d_delta_part = sum_e d_mixed_e (m_e + bias_e),
//                          d_sum = sum_e d_mixed_e (both summed in fp32, stored bf16) and
//                          d_bias partials;
//   rwkv6_shift_lerp_bwd   finishes dx and d_maa from those and d_xxx.
//
// Up-projection tile: a wave owns 16 tokens x 64 channels.  MFMA 16x16x32 with
//   A = W_up^T rows (channels, k = rank), B = neck rows (tokens, k = rank),
// so D[channel][token]; the A rows are permuted (tile_channel) so that lane (q, L) ends up
// holding two runs of 8 channels, c0 + 8q + (0..7) and c0 + 32 + 8q + (0..7), of token L.
// That layout goes through a wave-private LDS tile (fp32) to the row layout of the global
// loads and stores, lane (rw, cg) = (lane >> 3, lane & 7) holding channels c0 + 8 cg + (0..7)
// of tokens rw and rw + 8, so every 16-byte access instruction covers 128 contiguous bytes of
// 8 token rows (at 64 bytes of 16 rows, as the MFMA layout would store, the same loads and
// stores stream 1.3-1.4x slower).  W_up^T is staged in LDS once per block.
#include "common.h"
#include "../../include/rwkv6_amd.h"

#define LORA_THR 256      // 4 waves, each 16 tokens x 64 channels at a time
#define LORA_TT 128       // tokens per block (64-token groups walked in turn)
#define LORA_NE 5
#ifndef LORA_BWD_AHEAD
#define LORA_BWD_AHEAD 2
#endif
#define LORA_MT_RS 68                  // row stride (floats) of a wave's m tile

namespace {

// channel (relative to c0) of MFMA tile tc, row 4q' + rr' = L': the run layout above
__device__ __forceinline__ int tile_channel(int tc, int L) {
    const int qq = L >> 2, rr = L & 3;
    return tc < 2 ? 8 * qq + 4 * tc + rr : 32 + 8 * qq + 4 * (tc - 2) + rr;
}

// Blocks are dispatched round-robin over the 8 XCDs: XCD x gets the token blocks
// [x*per, (x+1)*per) (all channel blocks of each, consecutively), so its L2 holds one
// eighth of neck.  The grid is 8 * per * nCB; blocks past the last token block exit.
__device__ __forceinline__ bool lora_tile(int64_t nTB, int64_t nCB, int64_t per, int64_t& tb,
                                          int64_t& cb) {
    const int64_t id = blockIdx.x, xcd = id & 7, j = id >> 3;
    tb = xcd * per + j / nCB;
    cb = j - (j / nCB) * nCB;
    return tb < nTB;
}

// Block operand staging: the 64 channel rows of W_up^T (all E mixes), shared by every token
// of the block, go to LDS once per block, rows padded by 8 elements so the 16 rows a wave
// reads with 16-byte loads fall on distinct banks.  The neck operand is per token (one lane's
// own row) and is read straight from global memory.
__device__ __forceinline__ int lds_rs(int R) { return R + 8; }
__host__ __device__ __forceinline__ size_t lora_lds_bytes(int E, int R) {
    return (size_t)E * 64 * (R + 8) * 2;
}

__device__ __forceinline__ void lora_stage(uint16_t* sw, const uint16_t* __restrict__ wut, int E,
                                           int64_t C, int R, int64_t c0) {
    const int rs = lds_rs(R), R8 = R / 8;
    for (int idx = threadIdx.x; idx < E * 64 * R8; idx += LORA_THR) {
        const int row = idx / R8, k8 = idx - row * R8;          // row = e*64 + channel
        const int e = row >> 6, ch = row & 63;
        *reinterpret_cast<uint4*>(sw + row * rs + 8 * k8) =
            *reinterpret_cast<const uint4*>(wut + ((int64_t)e * C + c0 + ch) * R + 8 * k8);
    }
}

}  // namespace

// LERP: out_e = x + (shift(x) - x) * (m_e + bias_e)  (E = 5);  else out_e = m_e + bias_e.
// Token n of output e starts at out.p[e] + n * ors (ors = C for separate [N,C] tensors, E * C
// for one [N,E,C] tensor).  A block takes REP consecutive 128-token tiles of its channel block
// (the single-mix decay output stages the block's W_up for four tiles instead of one).
// Wave wv takes the tokens 64 g + 16 wv + (0..15) of group g of the block (2 REP groups), all
// 64 channels.  m comes out of the MFMA one token per lane column and goes through the wave's
// LDS tile to the row layout of every global access, lane (rw, cg) = (lane >> 3, lane & 7)
// holding channels 8 cg + (0..7) of tokens rw and rw + 8: a load or store instruction covers
// 128 contiguous bytes of 8 token rows (16 rows at 64 bytes each stream ~1.3x slower).
// The stages s = E g + e are one straight run; each issues the neck pieces of stage
// s + AH (and, for LERP, x and x[t-B] of the group that stage opens) before its own
// stores.  Loads and stores are unconditional: a token past the end works on the last token
// and stores its values again (same values, same place).
// KS = R / 32, or 0: from R at run time (ranks past the first 32 are then loaded in the stage).
template <int E, bool LERP, int REP, int KS>
__global__ void __launch_bounds__(LORA_THR)
rwkv6_lora_up_kernel(const uint16_t* __restrict__ neck, const uint16_t* __restrict__ wut,
                     const void* __restrict__ bias, int pdt, const uint16_t* __restrict__ x,
                     OutPtrs<E> out, int64_t ors, int64_t N, int64_t B, int64_t C, int R,
                     int64_t per) {
    constexpr int NG = 2 * REP, NS = NG * E, KP = KS > 0 ? KS : 1;
    // prefetch depth: two stages for five mixes, one for the single decay output (measured
    // best at the config-3 shape: 61.5 against 63.1 and 62.2 us at depths 1 and 3, and 19.5
    // against 20.0 us)
    constexpr int AH = E > 1 ? 2 : 1;
    __shared__ __attribute__((aligned(16))) float mt[4][16 * LORA_MT_RS];   // per wave: m [token][channel]
    __shared__ __attribute__((aligned(16))) float bsm[E][64];          // bias of the block's channels
    int64_t tb, cb;
    if (!lora_tile((N + LORA_TT * REP - 1) / (LORA_TT * REP), C / 64, per, tb, cb)) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, L = lane & 15, q = lane >> 4;
    const int rw = lane >> 3, cg = lane & 7;
    const int64_t c0 = cb * 64, cl = c0 + 8 * cg;
    extern __shared__ __attribute__((aligned(16))) uint16_t lora_sm[];
    lora_stage(lora_sm, wut, E, C, R, c0);
    if (threadIdx.x < E * 8) {
        const int e = threadIdx.x >> 3, c8 = (threadIdx.x & 7) * 8;
        float bb[8];
        load_param8(bias, pdt, (int64_t)e * C + c0 + c8, bb);
#pragma unroll
        for (int j = 0; j < 8; ++j) bsm[e][c8 + j] = bb[j];
    }
    static_assert(LORA_TT == 128, "two 64-token groups per 128-token tile");
    const int64_t tblk = tb * REP * LORA_TT + 16 * wv;
    // group g: the MFMA column token (L) and the lane's row tokens (rw, rw + 8), clamped
    auto tok_m = [&](int g) { const int64_t t = tblk + 64 * g + L; return t < N ? t : N - 1; };
    auto tok_r = [&](int g, int k) { const int64_t t = tblk + 64 * g + rw + 8 * k; return t < N ? t : N - 1; };
    uint4 xr[2], pr[2], nkb[AH][KP];
    auto load_x = [&](int g) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int64_t t = tok_r(g, k);
            xr[k] = *reinterpret_cast<const uint4*>(x + t * C + cl);
            pr[k] = *reinterpret_cast<const uint4*>(x + (t >= B ? t - B : t) * C + cl);
        }
    };
    auto load_stage = [&](int st) {
        const int g = st / E, e = st - g * E;
        const uint16_t* nrow = neck + tok_m(g) * E * R + e * R + 8 * q;
#pragma unroll
        for (int ks = 0; ks < KP; ++ks)
            nkb[st % AH][ks] = *reinterpret_cast<const uint4*>(nrow + 32 * ks);
    };
    if (LERP) load_x(0);
#pragma unroll
    for (int st = 0; st < AH; ++st) load_stage(st);
    __syncthreads();
    const int rs = lds_rs(R);
    float* mtw = mt[wv];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        uint4 xc[2], pc[2];
        if (LERP) {
            xc[0] = xr[0]; xc[1] = xr[1]; pc[0] = pr[0]; pc[1] = pr[1];
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int st = E * g + e;
            const uint16_t* swe = lora_sm + e * 64 * rs;
            f32x4 acc[4] = {};
#pragma unroll
            for (int ks = 0; ks < KP; ++ks) {
                const bf16x8 bq = __builtin_bit_cast(bf16x8, nkb[st % AH][ks]);
#pragma unroll
                for (int tcn = 0; tcn < 4; ++tcn)
                    acc[tcn] = mfma32(ld_bf16x8(swe + tile_channel(tcn, L) * rs + 32 * ks + 8 * q), bq,
                                      acc[tcn]);
            }
            if (KS == 0) {
                const uint16_t* nrow = neck + tok_m(g) * E * R + e * R + 8 * q;
                for (int ks = 1; ks < R / 32; ++ks) {
                    const bf16x8 bq = ld_bf16x8(nrow + 32 * ks);
#pragma unroll
                    for (int tcn = 0; tcn < 4; ++tcn)
                        acc[tcn] = mfma32(ld_bf16x8(swe + tile_channel(tcn, L) * rs + 32 * ks + 8 * q), bq,
                                          acc[tcn]);
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                float* d = mtw + L * LORA_MT_RS + 32 * hh + 8 * q;
                *reinterpret_cast<float4*>(d) = make_float4(acc[2 * hh][0], acc[2 * hh][1], acc[2 * hh][2], acc[2 * hh][3]);
                *reinterpret_cast<float4*>(d + 4) =
                    make_float4(acc[2 * hh + 1][0], acc[2 * hh + 1][1], acc[2 * hh + 1][2], acc[2 * hh + 1][3]);
            }
            // the wave's own LDS writes and reads run in issue order; the compiler must not
            // move the reads above the writes
            asm volatile("" ::: "memory");
            float m[2][8];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const float* sp = mtw + (rw + 8 * k) * LORA_MT_RS + 8 * cg;
                const float4 m0 = *reinterpret_cast<const float4*>(sp);
                const float4 m1 = *reinterpret_cast<const float4*>(sp + 4);
                m[k][0] = m0.x; m[k][1] = m0.y; m[k][2] = m0.z; m[k][3] = m0.w;
                m[k][4] = m1.x; m[k][5] = m1.y; m[k][6] = m1.z; m[k][7] = m1.w;
            }
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            if (st + AH < NS) {
                if (LERP && (st + AH) % E == 0) load_x((st + AH) / E);
                load_stage(st + AH);
            }
            __builtin_amdgcn_sched_barrier(0);
            const float4 b0 = *reinterpret_cast<const float4*>(&bsm[e][8 * cg]);
            const float4 b1 = *reinterpret_cast<const float4*>(&bsm[e][8 * cg + 4]);
            const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int64_t t = tok_r(g, k);
                float o[8];
                if (LERP) {
                    float xv[8], xp[8];
                    unpack8(xc[k], xv);
                    unpack8(pc[k], xp);
                    const float keep = t >= B ? 1.f : 0.f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] = xv[j] + (xp[j] * keep - xv[j]) * (m[k][j] + bb[j]);
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] = m[k][j] + bb[j];
                }
                // nontemporal for the five mixes (the single decay output measured slower so)
                if (E > 1) store8_nt(out.p[e] + t * ors + cl, o);
                else store8(out.p[e] + t * ors + cl, o);
            }
        }
    }
}

// Backward of the token-shift LoRA's up-projection + ddlerp (E = 5), per token:
//   d_mexp_e = d_mixed_e * delta;  dd = sum_e d_mixed_e (m_e + bias_e);  ds = sum_e d_mixed_e
// and the d_bias partial of this block's tokens: part[blockIdx.x][e][C].
// Wave wv takes the 32 tokens 32 wv + (0..31) of the block, 16 at a time (pass P), all 64
// channels.  m comes out of the MFMA one token per lane column (lane (q, L): channel runs
// 8q + (0..7) and 32 + 8q + (0..7) of token L) and goes through a wave-private LDS tile to
// the row layout every global access uses: lane (rw, cg) = (lane >> 3, lane & 7) holds
// channels 8 cg + (0..7) of tokens rw and rw + 8, so a load or store instruction covers
// 128 contiguous bytes of 8 token rows.  (An instruction spanning 16 rows at 64 bytes each
// streams ~1.35x slower on MI355X, measured with the same loads and stores and no
// arithmetic: 276 against 201 us at N = 16384, C = 2048.)
// The wave's ten stages s = 5 P + e (pass P, mix e) are one straight run; each stage issues
// the loads of stage s + LORA_BWD_AHEAD before its own stores (the vector-memory counter
// retires loads and stores in issue order).  No load or store sits under a branch: a token
// past the end works on the last token and stores its values again (same values, same
// place), and only its d_bias contribution is masked.
// KS = R / 32 (1 or 2; the launch picks it).
template <int KS>
__global__ void __launch_bounds__(LORA_THR)
rwkv6_ddlerp_lora_bwd_kernel(const uint16_t* __restrict__ neck, const uint16_t* __restrict__ wut,
                             const void* __restrict__ bias, int pdt,
                             const uint16_t* __restrict__ x, InPtrs<LORA_NE> dmix,
                             uint16_t* __restrict__ dmexp, uint16_t* __restrict__ dd_out,
                             uint16_t* __restrict__ ds_out, float* __restrict__ part, int64_t N,
                             int64_t B, int64_t C, int R, int64_t per) {
    __shared__ __attribute__((aligned(16))) float mt[4][16 * LORA_MT_RS];   // per wave: m [token][channel]
    __shared__ float red[LORA_NE][4][64];          // [mix][wave][channel]
    __shared__ __attribute__((aligned(16))) float bsm[LORA_NE][64];   // bias of the block's channels
    int64_t tb, cb;
    if (!lora_tile((N + LORA_TT - 1) / LORA_TT, C / 64, per, tb, cb)) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, L = lane & 15, q = lane >> 4;
    const int rw = lane >> 3, cg = lane & 7;
    const int64_t c0 = cb * 64, cl = c0 + 8 * cg;
    extern __shared__ __attribute__((aligned(16))) uint16_t lora_sm[];
    lora_stage(lora_sm, wut, LORA_NE, C, R, c0);
    if (threadIdx.x < LORA_NE * 8) {
        const int e = threadIdx.x >> 3, c8 = (threadIdx.x & 7) * 8;
        float bb[8];
        load_param8(bias, pdt, (int64_t)e * C + c0 + c8, bb);
#pragma unroll
        for (int j = 0; j < 8; ++j) bsm[e][c8 + j] = bb[j];
    }
    static_assert(LORA_TT == 128, "four waves of 32 tokens per block");
    // pass P: the MFMA column token (L) and the lane's two row tokens (rw, rw + 8), clamped
    int64_t tm[2], tr[2][2];
    float keep[2][2];
#pragma unroll
    for (int P = 0; P < 2; ++P) {
        const int64_t t0 = tb * LORA_TT + 32 * wv + 16 * P;
        tm[P] = t0 + L < N ? t0 + L : N - 1;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int64_t t = t0 + rw + 8 * k;
            tr[P][k] = t < N ? t : N - 1;
            keep[P][k] = t < N ? 1.f : 0.f;
        }
    }
    // stage loads: the neck piece (MFMA layout) and d_mixed (row layout), LORA_BWD_AHEAD
    // stages ahead in a ring; x and x[t-B] of a pass (packed) with its first stage's loads
    uint4 xr[2], pr[2], nkb[LORA_BWD_AHEAD][KS], dqb[LORA_BWD_AHEAD][2];
    auto load_x = [&](int P) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int64_t t = tr[P][k];
            xr[k] = *reinterpret_cast<const uint4*>(x + t * C + cl);
            pr[k] = *reinterpret_cast<const uint4*>(x + (t >= B ? t - B : t) * C + cl);
        }
    };
    auto load_stage = [&](int st) {
        const int P = st / LORA_NE, e = st - P * LORA_NE;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            nkb[st % LORA_BWD_AHEAD][ks] =
                *reinterpret_cast<const uint4*>(neck + tm[P] * LORA_NE * R + e * R + 32 * ks + 8 * q);
#pragma unroll
        for (int k = 0; k < 2; ++k)
            dqb[st % LORA_BWD_AHEAD][k] = *reinterpret_cast<const uint4*>(dmix.p[e] + tr[P][k] * C + cl);
    };
    load_x(0);
#pragma unroll
    for (int st = 0; st < LORA_BWD_AHEAD; ++st) load_stage(st);
    __syncthreads();
    const int rs = lds_rs(R);
    float* mtw = mt[wv];
    float bsum[LORA_NE];                           // d_bias of channel 8 cg + 4 b3 + 2 b4 + b5
#pragma unroll
    for (int P = 0; P < 2; ++P) {
        const uint4 xc[2] = {xr[0], xr[1]}, pc[2] = {pr[0], pr[1]};
        float dd[2][8], ds[2][8];
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
            for (int j = 0; j < 8; ++j) dd[k][j] = ds[k][j] = 0.f;
#pragma unroll
        for (int e = 0; e < LORA_NE; ++e) {
            const int st = LORA_NE * P + e;
            const uint16_t* swe = lora_sm + e * 64 * rs;
            // m = neck_e W_up_e, 16 tokens x 64 channels, to the wave's tile
            f32x4 acc[4] = {};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const bf16x8 bq = __builtin_bit_cast(bf16x8, nkb[st % LORA_BWD_AHEAD][ks]);
#pragma unroll
                for (int tcn = 0; tcn < 4; ++tcn)
                    acc[tcn] = mfma32(ld_bf16x8(swe + tile_channel(tcn, L) * rs + 32 * ks + 8 * q), bq,
                                      acc[tcn]);
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                float* d = mtw + L * LORA_MT_RS + 32 * hh + 8 * q;
                *reinterpret_cast<float4*>(d) = make_float4(acc[2 * hh][0], acc[2 * hh][1], acc[2 * hh][2], acc[2 * hh][3]);
                *reinterpret_cast<float4*>(d + 4) =
                    make_float4(acc[2 * hh + 1][0], acc[2 * hh + 1][1], acc[2 * hh + 1][2], acc[2 * hh + 1][3]);
            }
            // the wave's own LDS writes and reads run in issue order; the compiler must not
            // move the reads above the writes
            asm volatile("" ::: "memory");
            float m[2][8];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const float* sp = mtw + (rw + 8 * k) * LORA_MT_RS + 8 * cg;
                const float4 m0 = *reinterpret_cast<const float4*>(sp);
                const float4 m1 = *reinterpret_cast<const float4*>(sp + 4);
                m[k][0] = m0.x; m[k][1] = m0.y; m[k][2] = m0.z; m[k][3] = m0.w;
                m[k][4] = m1.x; m[k][5] = m1.y; m[k][6] = m1.z; m[k][7] = m1.w;
            }
            asm volatile("" ::: "memory");
            float v[2][8];
            unpack8(dqb[st % LORA_BWD_AHEAD][0], v[0]);
            unpack8(dqb[st % LORA_BWD_AHEAD][1], v[1]);
            // later stages' loads go out before this stage's stores (the scheduling barriers
            // keep them here: hoisted to the top, the ten stages' loads would hold far more
            // registers)
            __builtin_amdgcn_sched_barrier(0);
            if (st + LORA_BWD_AHEAD < 2 * LORA_NE) {
                if (st + LORA_BWD_AHEAD == LORA_NE) load_x(1);
                load_stage(st + LORA_BWD_AHEAD);
            }
            __builtin_amdgcn_sched_barrier(0);
            const float4 b0 = *reinterpret_cast<const float4*>(&bsm[e][8 * cg]);
            const float4 b1 = *reinterpret_cast<const float4*>(&bsm[e][8 * cg + 4]);
            const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
            float vs[8];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                float xv[8], dl[8];
                unpack8(xc[k], xv);
                unpack8(pc[k], dl);
                const float keep_p = tr[P][k] >= B ? 1.f : 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    dl[j] = dl[j] * keep_p - xv[j];
                    dd[k][j] += v[k][j] * (m[k][j] + bb[j]);
                    ds[k][j] += v[k][j];
                    v[k][j] *= dl[j];                               // d_mexp
                    vs[j] = k == 0 ? keep[P][0] * v[0][j] : vs[j] + keep[P][1] * v[1][j];
                }
                store8(dmexp + ((int64_t)e * N + tr[P][k]) * C + cl, v[k]);
            }
            // d_bias: sum over the wave's 16 tokens (lane bits 3-5).  Transposing butterfly:
            // each step keeps one half of a lane's values and adds the partner's copy of that
            // half; row_ror:8 for bit 3, then the row swaps for bits 4 and 5, whose two
            // results sum to the even row's (half's) A value plus the odd one's in the even
            // lanes and to the B values in the odd ones.  Lane (rw, cg) ends with channel
            // 8 cg + 4 b3 + 2 b4 + b5, in a fixed order.
            {
                const bool up = lane & 8;
#pragma unroll
                for (int i = 0; i < 4; ++i) vs[i] = (up ? vs[i + 4] : vs[i]) + lane_xor8(up ? vs[i] : vs[i + 4]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(vs[i]), __float_as_uint(vs[i + 2]),
                                                                false, false);
                vs[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
            }
            {
                const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(vs[0]), __float_as_uint(vs[1]),
                                                                false, false);
                vs[0] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
            }
            bsum[e] = P == 0 ? vs[0] : bsum[e] + vs[0];
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            store8(dd_out + tr[P][k] * C + cl, dd[k]);
            store8(ds_out + tr[P][k] * C + cl, ds[k]);
        }
    }
    {
        const int ch = 8 * cg + 4 * ((lane >> 3) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 5) & 1);
#pragma unroll
        for (int e = 0; e < LORA_NE; ++e) red[e][wv][ch] = bsum[e];
    }
    __syncthreads();
    for (int j = threadIdx.x; j < LORA_NE * 64; j += LORA_THR) {
        const int e = j >> 6, c = j & 63;
        part[(tb * LORA_NE + e) * C + c0 + c] = ((red[e][0][c] + red[e][1][c]) + red[e][2][c]) + red[e][3][c];
    }
}

// Backward of xxx = x + (shift(x) - x) * maa together with the rest of the input gradient:
//   d_delta[t] = dd[t] + d_xxx[t] maa,   dx[t] = ds[t] + d_xxx[t] - d_delta[t] + d_delta[t+1]
//   d_maa partial = sum_t d_xxx[t] (x[t-1] - x[t])  -> part[tblk * B + b][C]
// Block = 8 token slots x 32 channel groups (8 channels each) over SLB_TB tokens of one batch
// row; thread (ts, cgl) takes the tokens ts + 8j.  Every token is independent: d_delta[t+1] is
// formed again from the next token's dd and d_xxx (re-read, mostly from L2) rather than carried
// along a walk, so all of a thread's loads can be in flight together.  Loads clamp the token
// (no branch); a token past the end stores nothing and adds nothing.
#define SLB_TB 32
#define SLB_SS 8
#define SLB_NJ (SLB_TB / SLB_SS)
__global__ void __launch_bounds__(LORA_THR)
rwkv6_shift_lerp_bwd_kernel(const uint16_t* __restrict__ x, const void* __restrict__ maa, int pdt,
                            const uint16_t* __restrict__ dd, const uint16_t* __restrict__ ds,
                            const uint16_t* __restrict__ dxxx, uint16_t* __restrict__ dx,
                            float* __restrict__ part, int64_t T, int64_t B, int64_t C) {
    __shared__ float red[SLB_SS][32 * 8 + 4];
    const int ts = threadIdx.x >> 5, cgl = threadIdx.x & 31;
    const int64_t C8 = C / 8, cg = (int64_t)blockIdx.y * 32 + cgl;
    const int64_t b = blockIdx.z;
    float acc[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[s] = 0.f;
    if (cg < C8) {
        float mv[8];
        load_param8(maa, pdt, 8 * cg, mv);
#pragma unroll
        for (int j = 0; j < SLB_NJ; ++j) {
            const int64_t t = (int64_t)blockIdx.x * SLB_TB + ts + SLB_SS * j;
            const int64_t tc = t < T ? t : T - 1;
            const int64_t tp = tc > 0 ? tc - 1 : 0, tn = tc + 1 < T ? tc + 1 : tc;
            const float kv = t < T ? 1.f : 0.f, kp = tc > 0 ? 1.f : 0.f, kn = tc + 1 < T ? 1.f : 0.f;
            const int64_t off = (tc * B + b) * C + 8 * cg;
            const int64_t offp = (tp * B + b) * C + 8 * cg, offn = (tn * B + b) * C + 8 * cg;
            float xv[8], xp[8], dxx[8], ddv[8], dsv[8], dxn[8], ddn[8], out[8];
            load8(x + off, xv);
            load8(x + offp, xp);
            load8(dxxx + off, dxx);
            load8(dd + off, ddv);
            load8(ds + off, dsv);
            load8(dxxx + offn, dxn);
            load8(dd + offn, ddn);
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const float dlt = ddv[s] + dxx[s] * mv[s];
                const float nd = kn * (ddn[s] + dxn[s] * mv[s]);
                out[s] = dsv[s] + dxx[s] - dlt + nd;
                acc[s] += kv * (dxx[s] * (kp * xp[s] - xv[s]));
            }
            if (t < T) store8_nt(dx + off, out);   // streaming: 70 -> 60 us at config 3
        }
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) red[ts][8 * cgl + s] = acc[s];
    __syncthreads();
    const int64_t P_row = (int64_t)blockIdx.x * B + b;
    for (int c = threadIdx.x; c < 256; c += LORA_THR) {
        const int64_t ch = (int64_t)blockIdx.y * 256 + c;
        if (ch >= C) continue;
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < SLB_SS; ++q) sum += red[q][c];
        part[P_row * C + ch] = sum;
    }
}

// The backward of the bottleneck's tanh (rwkv6_layer_specs.py:177-195):
//   d_pre[n][e*R + r] = d_neck(e, n, r) * (1 - neck[n][e*R + r]^2),
// with d_neck(e, n, r) at d_neck + e*sE + n*sN + r (the up-projection's input gradient as the
// batched or per-mix GEMM left it) and d_pre in the [N, E*R] layout of the down-projection's
// GEMMs.  One thread per 8 consecutive r (16-byte accesses).
__global__ void __launch_bounds__(LORA_THR)
rwkv6_lora_tanh_bwd_kernel(const uint16_t* __restrict__ d_neck, int64_t sE, int64_t sN,
                           const uint16_t* __restrict__ neck, uint16_t* __restrict__ d_pre,
                           int64_t N, int E, int R) {
    const int64_t R8 = R / 8, per_n = (int64_t)E * R8;
    const int64_t i = (int64_t)blockIdx.x * LORA_THR + threadIdx.x;
    if (i >= N * per_n) return;
    const int64_t n = i / per_n, rem = i - n * per_n;
    const int64_t e = rem / R8, r8 = rem - e * R8;
    float d[8], t[8], y[8];
    load8(d_neck + e * sE + n * sN + 8 * r8, d);
    load8(neck + n * E * R + e * R + 8 * r8, t);
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = d[j] * (1.f - t[j] * t[j]);
    store8(d_pre + n * E * R + e * R + 8 * r8, y);
}

// Column sums of x [N, M] bf16 (the bias gradient of a bottleneck, summed over the tokens),
// stage 1: block (rb, cb) sums rows [256 rb, 256 rb + 256) of columns [256 cb, 256 cb + 256);
// thread (q, g) takes 8 columns and the rows q, q + 8, ...; the 8 partials of a column are
// combined in LDS in a fixed order into part[rb][M] (partials_reduce_kernel of common.h finishes).
// BATCH rows' loads are issued together: 8 when the grid leaves few waves per CU (17.4 -> 13.0
// us at N = 16384, M = 2048), 1 when it fills the device (M = 4096: 22.8 us, ~5.9 TB/s, where
// batches of 8 measured 27 us).  Same summation order either way.
#define CS_ROWS 256
template <int BATCH>
__global__ void __launch_bounds__(LORA_THR)
rwkv6_col_sum_kernel(const uint16_t* __restrict__ x, int64_t N, int64_t M,
                     float* __restrict__ part) {
    __shared__ float acc[8][256 + 4];
    const int q = threadIdx.x >> 5, g = threadIdx.x & 31;
    const int64_t c0 = (int64_t)blockIdx.y * 256 + 8 * g;
    const int64_t r0 = (int64_t)blockIdx.x * CS_ROWS;
    float a[8] = {};
    if (c0 < M) {
        // rows q, q + 8, ... of the block in order; eight loads in flight (unconditional: a
        // row past the end reads the last row and adds zero)
        const int64_t r1 = min<int64_t>(N, r0 + CS_ROWS);
        static_assert(CS_ROWS % (8 * BATCH) == 0, "rows in whole batches per thread");
        for (int k0 = 0; k0 < CS_ROWS / 8; k0 += BATCH) {
            // the batch's 16-byte loads first, then the sums (left to itself the compiler
            // waited for each load before issuing the next)
            uint4 raw[BATCH];
#pragma unroll
            for (int k = 0; k < BATCH; ++k) {
                const int64_t rw = r0 + q + 8 * (k0 + k);
                raw[k] = *reinterpret_cast<const uint4*>(x + (rw < r1 ? rw : r1 - 1) * M + c0);
            }
#pragma unroll
            for (int k = 0; k < BATCH; ++k) {
                const float keep = r0 + q + 8 * (k0 + k) < r1 ? 1.f : 0.f;
                float f[8];
                unpack8(raw[k], f);
#pragma unroll
                for (int j = 0; j < 8; ++j) a[j] += keep * f[j];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[q][8 * g + j] = a[j];
    __syncthreads();
    const int cl = threadIdx.x;                     // 256 threads, one column each
    const int64_t c = (int64_t)blockIdx.y * 256 + cl;
    if (c < M) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) t += acc[j][cl];
        part[(int64_t)blockIdx.x * M + c] = t;
    }
}

namespace {
inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int launch_status() { return hipGetLastError() == hipSuccess ? RWKV6_OK : RWKV6_ERR_LAUNCH; }
inline int lora_check(int E, int64_t N, int64_t C, int64_t R, int pdt) {
    if (N < 0 || C < 1 || R < 1) return RWKV6_ERR_INVALID_ARG;
    if (C % 64 || R % 32 || R > 256 || lora_lds_bytes(E, (int)R) > 65536) return RWKV6_ERR_UNSUPPORTED;
    if (pdt != RWKV6_F32 && pdt != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    return RWKV6_OK;
}
template <typename P, int NP>
inline int gather(const void* const* src, P& dst) {
    if (!src) return RWKV6_ERR_INVALID_ARG;
    for (int e = 0; e < NP; ++e) {
        if (!src[e]) return RWKV6_ERR_INVALID_ARG;
        if (!al16(src[e])) return RWKV6_ERR_ALIGNMENT;
        dst.p[e] = (decltype(dst.p[0]))src[e];
    }
    return RWKV6_OK;
}
// token blocks (of rep 128-token tiles) per XCD and the padded 1-D grid of lora_tile
inline int64_t up_per(int64_t N, int64_t rep = 1) {
    return ((N + LORA_TT * rep - 1) / (LORA_TT * rep) + 7) / 8;
}
inline dim3 up_grid(int64_t N, int64_t C, int64_t rep = 1) {
    return dim3((unsigned)(8 * up_per(N, rep) * (C / 64)));
}
}  // namespace

extern "C" {

int rwkv6_ddlerp_lora_fwd(const void* x, const void* neck, const void* w_up_t, const void* bias,
                          int param_dtype, void* const* mixed, int64_t T, int64_t B, int64_t C,
                          int64_t R, void* stream) {
    if (T < 0 || B < 1) return RWKV6_ERR_INVALID_ARG;
    int st = lora_check(LORA_NE, T * B, C, R, param_dtype);
    if (st) return st;
    if (T == 0) return RWKV6_OK;
    if (!x || !neck || !w_up_t || !bias) return RWKV6_ERR_INVALID_ARG;
    OutPtrs<LORA_NE> out;
    if ((st = gather<OutPtrs<LORA_NE>, LORA_NE>((const void* const*)mixed, out))) return st;
    if (!al16(x) || !al16(neck) || !al16(w_up_t) || !al16(bias)) return RWKV6_ERR_ALIGNMENT;
    {
        const size_t act = (size_t)(T * B * C) * 2;
        if (any_alias({{out.p[0], act}, {out.p[1], act}, {out.p[2], act}, {out.p[3], act}, {out.p[4], act}},
                      {{x, act}, {neck, (size_t)(T * B * LORA_NE * R) * 2},
                       {w_up_t, (size_t)(LORA_NE * C * R) * 2},
                       {bias, (size_t)(LORA_NE * C) * param_bytes(param_dtype)}}))
            return RWKV6_ERR_INVALID_ARG;
    }
    // five mixes admit R = 32 and 64 (the LDS bound)
    auto kern = R == 64 ? rwkv6_lora_up_kernel<LORA_NE, true, 1, 2> : rwkv6_lora_up_kernel<LORA_NE, true, 1, 1>;
    hipLaunchKernelGGL(kern, up_grid(T * B, C), dim3(LORA_THR),
                       lora_lds_bytes(LORA_NE, (int)R),
                       reinterpret_cast<hipStream_t>(stream), (const uint16_t*)neck,
                       (const uint16_t*)w_up_t, bias, param_dtype, (const uint16_t*)x, out, C,
                       T * B, B, C, (int)R, up_per(T * B));
    return launch_status();
}

int rwkv6_lora_bias_fwd(const void* neck, const void* w_up_t, const void* bias, int param_dtype,
                        void* out, int64_t N, int64_t E, int64_t C, int64_t R, void* stream) {
    if (E != 1 && E != LORA_NE) return E < 1 ? RWKV6_ERR_INVALID_ARG : RWKV6_ERR_UNSUPPORTED;
    int st = lora_check((int)E, N, C, R, param_dtype);
    if (st) return st;
    if (N == 0) return RWKV6_OK;
    if (!neck || !w_up_t || !bias || !out) return RWKV6_ERR_INVALID_ARG;
    if (!al16(neck) || !al16(w_up_t) || !al16(bias) || !al16(out)) return RWKV6_ERR_ALIGNMENT;
    if (any_alias({{out, (size_t)(N * E * C) * 2}},
                  {{neck, (size_t)(N * E * R) * 2}, {w_up_t, (size_t)(E * C * R) * 2},
                   {bias, (size_t)(E * C) * param_bytes(param_dtype)}}))
        return RWKV6_ERR_INVALID_ARG;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (E == 1) {
        OutPtrs<1> o;
        o.p[0] = (uint16_t*)out;
        // ranks 32 and 64 (the decay LoRA's) with a compile-time count, any other from R
        auto kern = R == 64 ? rwkv6_lora_up_kernel<1, false, 4, 2>
                            : R == 32 ? rwkv6_lora_up_kernel<1, false, 4, 1> : rwkv6_lora_up_kernel<1, false, 4, 0>;
        hipLaunchKernelGGL(kern, up_grid(N, C, 4), dim3(LORA_THR),
                           lora_lds_bytes(1, (int)R), s, (const uint16_t*)neck,
                           (const uint16_t*)w_up_t, bias, param_dtype, (const uint16_t*)nullptr, o,
                           C, N, (int64_t)1, C, (int)R, up_per(N, 4));
    } else {
        OutPtrs<LORA_NE> o;
        for (int e = 0; e < LORA_NE; ++e) o.p[e] = (uint16_t*)out + (int64_t)e * C;
        auto kern = R == 64 ? rwkv6_lora_up_kernel<LORA_NE, false, 1, 2> : rwkv6_lora_up_kernel<LORA_NE, false, 1, 1>;
        hipLaunchKernelGGL(kern, up_grid(N, C), dim3(LORA_THR),
                           lora_lds_bytes(LORA_NE, (int)R), s, (const uint16_t*)neck,
                           (const uint16_t*)w_up_t, bias, param_dtype, (const uint16_t*)nullptr, o,
                           (int64_t)LORA_NE * C, N, (int64_t)1, C, (int)R, up_per(N));
    }
    return launch_status();
}

size_t rwkv6_ddlerp_lora_bwd_workspace_bytes(int64_t T, int64_t B, int64_t C) {
    if (T < 0 || B < 1 || C < 1) return 0;
    const int64_t nb = (T * B + LORA_TT - 1) / LORA_TT;
    return (size_t)((nb > 0 ? nb : 1) * LORA_NE * C) * sizeof(float);
}

int rwkv6_ddlerp_lora_bwd(const void* x, const void* neck, const void* w_up_t, const void* bias,
                          int param_dtype, const void* const* d_mixed, void* d_mexp,
                          void* d_delta_part, void* d_sum, void* d_bias, void* workspace,
                          int64_t T, int64_t B, int64_t C, int64_t R, void* stream) {
    if (T < 0 || B < 1) return RWKV6_ERR_INVALID_ARG;
    int st = lora_check(LORA_NE, T * B, C, R, param_dtype);
    if (st) return st;
    // lora_check admits R = 32 and 64 for five mixes (the LDS bound); the kernel is compiled
    // for exactly those two step counts
    if (R != 32 && R != 64) return RWKV6_ERR_UNSUPPORTED;
    if (!bias || !d_bias || !workspace ||
        (T > 0 && (!x || !neck || !w_up_t || !d_mexp || !d_delta_part || !d_sum)))
        return RWKV6_ERR_INVALID_ARG;
    InPtrs<LORA_NE> dm{};
    if (T > 0 && (st = gather<InPtrs<LORA_NE>, LORA_NE>(d_mixed, dm))) return st;
    if (!al16(x) || !al16(neck) || !al16(w_up_t) || !al16(bias) || !al16(d_mexp) ||
        !al16(d_delta_part) || !al16(d_sum) || !al16(workspace))
        return RWKV6_ERR_ALIGNMENT;
    if (T > 0) {
        const size_t act = (size_t)(T * B * C) * 2, par = (size_t)(LORA_NE * C) * param_bytes(param_dtype);
        if (any_alias({{d_mexp, LORA_NE * act}, {d_delta_part, act}, {d_sum, act}, {d_bias, par},
                       {workspace, rwkv6_ddlerp_lora_bwd_workspace_bytes(T, B, C)}},
                      {{x, act}, {neck, (size_t)(T * B * LORA_NE * R) * 2},
                       {w_up_t, (size_t)(LORA_NE * C * R) * 2}, {bias, par}, {dm.p[0], act},
                       {dm.p[1], act}, {dm.p[2], act}, {dm.p[3], act}, {dm.p[4], act}}))
            return RWKV6_ERR_INVALID_ARG;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t N = T * B, nb = (N + LORA_TT - 1) / LORA_TT;
    float* part = reinterpret_cast<float*>(workspace);
    if (N > 0) {
        auto kern = R == 32 ? rwkv6_ddlerp_lora_bwd_kernel<1> : rwkv6_ddlerp_lora_bwd_kernel<2>;
        hipLaunchKernelGGL(kern, up_grid(N, C), dim3(LORA_THR), lora_lds_bytes(LORA_NE, (int)R), s,
                           (const uint16_t*)neck, (const uint16_t*)w_up_t, bias, param_dtype,
                           (const uint16_t*)x, dm, (uint16_t*)d_mexp, (uint16_t*)d_delta_part,
                           (uint16_t*)d_sum, part, N, B, C, (int)R, up_per(N));
    }
    launch_partials_reduce(part, nb, (int64_t)LORA_NE * C, param_dtype, d_bias, nullptr,
                           (int64_t)LORA_NE * C, s);
    return launch_status();
}

size_t rwkv6_shift_lerp_bwd_workspace_bytes(int64_t T, int64_t B, int64_t C) {
    if (T < 0 || B < 1 || C < 1) return 0;
    const int64_t ntb = (T + SLB_TB - 1) / SLB_TB;
    return (size_t)((ntb > 0 ? ntb : 1) * B * C) * sizeof(float);
}

int rwkv6_shift_lerp_bwd(const void* x, const void* maa, int param_dtype, const void* d_delta_part,
                         const void* d_sum, const void* d_xxx, void* dx, void* d_maa,
                         void* workspace, int64_t T, int64_t B, int64_t C, void* stream) {
    if (T < 0 || B < 1 || C < 8) return RWKV6_ERR_INVALID_ARG;
    if (C % 8) return RWKV6_ERR_UNSUPPORTED;
    if (B > 65535) return RWKV6_ERR_UNSUPPORTED;
    if (param_dtype != RWKV6_F32 && param_dtype != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    if (!maa || !d_maa || !workspace || (T > 0 && (!x || !d_delta_part || !d_sum || !d_xxx || !dx)))
        return RWKV6_ERR_INVALID_ARG;
    if (!al16(x) || !al16(maa) || !al16(d_delta_part) || !al16(d_sum) || !al16(d_xxx) ||
        !al16(dx) || !al16(workspace))
        return RWKV6_ERR_ALIGNMENT;
    {
        const size_t act = (size_t)(T * B * C) * 2, par = (size_t)C * param_bytes(param_dtype);
        if (any_alias({{dx, act}, {d_maa, par}, {workspace, rwkv6_shift_lerp_bwd_workspace_bytes(T, B, C)}},
                      {{x, act}, {maa, par}, {d_delta_part, act}, {d_sum, act}, {d_xxx, act}}))
            return RWKV6_ERR_INVALID_ARG;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t ntb = (T + SLB_TB - 1) / SLB_TB;
    float* part = reinterpret_cast<float*>(workspace);
    if (T > 0)
        hipLaunchKernelGGL(rwkv6_shift_lerp_bwd_kernel,
                           dim3((unsigned)ntb, (unsigned)((C / 8 + 31) / 32), (unsigned)B),
                           dim3(LORA_THR), 0, s, (const uint16_t*)x, maa, param_dtype,
                           (const uint16_t*)d_delta_part, (const uint16_t*)d_sum,
                           (const uint16_t*)d_xxx, (uint16_t*)dx, part, T, B, C);
    launch_partials_reduce(part, T > 0 ? ntb * B : (int64_t)0, C, param_dtype, d_maa, nullptr, C, s);
    return launch_status();
}

int rwkv6_lora_tanh_bwd(const void* d_neck, int64_t sE, int64_t sN, const void* neck, void* d_pre,
                        int64_t N, int64_t E, int64_t R, void* stream) {
    if (N < 0 || E < 1 || R < 1 || sE < 0 || sN < 0) return RWKV6_ERR_INVALID_ARG;
    if (R % 8 || sE % 8 || sN % 8 || E > 64) return RWKV6_ERR_UNSUPPORTED;
    if (N == 0) return RWKV6_OK;
    if (!d_neck || !neck || !d_pre) return RWKV6_ERR_INVALID_ARG;
    if (!al16(d_neck) || !al16(neck) || !al16(d_pre)) return RWKV6_ERR_ALIGNMENT;
    const size_t nb = (size_t)(N * E * R) * 2;
    const size_t dnb = (size_t)((E - 1) * sE + (N - 1) * sN + R) * 2;   // extent of d_neck
    if (any_alias({{d_pre, nb}}, {{d_neck, dnb}, {neck, nb}})) return RWKV6_ERR_INVALID_ARG;
    const int64_t items = N * E * (R / 8);
    hipLaunchKernelGGL(rwkv6_lora_tanh_bwd_kernel, dim3((unsigned)((items + LORA_THR - 1) / LORA_THR)),
                       dim3(LORA_THR), 0, reinterpret_cast<hipStream_t>(stream),
                       (const uint16_t*)d_neck, sE, sN, (const uint16_t*)neck, (uint16_t*)d_pre, N,
                       (int)E, (int)R);
    return launch_status();
}

size_t rwkv6_col_sum_workspace_bytes(int64_t N, int64_t M) {
    if (N < 0 || M < 1) return 0;
    const int64_t nb = (N + CS_ROWS - 1) / CS_ROWS;
    return (size_t)((nb > 0 ? nb : 1) * M) * sizeof(float);
}

int rwkv6_col_sum(const void* x, int64_t N, int64_t M, int param_dtype, void* out,
                  void* workspace, void* stream) {
    if (N < 0 || M < 1) return RWKV6_ERR_INVALID_ARG;
    if (M % 8) return RWKV6_ERR_UNSUPPORTED;
    if (param_dtype != RWKV6_F32 && param_dtype != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    if (!out || !workspace || (N > 0 && !x)) return RWKV6_ERR_INVALID_ARG;
    if (!al16(x) || !al16(workspace)) return RWKV6_ERR_ALIGNMENT;
    if (any_alias({{out, (size_t)M * param_bytes(param_dtype)},
                   {workspace, rwkv6_col_sum_workspace_bytes(N, M)}},
                  {{x, (size_t)(N * M) * 2}}))
        return RWKV6_ERR_INVALID_ARG;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t nb = (N + CS_ROWS - 1) / CS_ROWS;
    float* part = reinterpret_cast<float*>(workspace);
    if (N > 0) {
        const dim3 grid((unsigned)nb, (unsigned)((M + 255) / 256));
        auto kern = (int64_t)grid.x * grid.y >= 1024 ? rwkv6_col_sum_kernel<1> : rwkv6_col_sum_kernel<8>;
        hipLaunchKernelGGL(kern, grid, dim3(LORA_THR), 0, s, (const uint16_t*)x, N, M, part);
    }
    launch_partials_reduce(part, N > 0 ? nb : (int64_t)0, M, param_dtype, out, nullptr, M, s);
    return launch_status();
}

}  // extern "C"
