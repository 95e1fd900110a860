// Token shift + static lerp of RWKV6TimeMix.forward (the input of its token-shift LoRA)
// and the channel-mix kernels, for MI355X (gfx950).  Sequence-first [T,B,C] bf16.
//
// Reference (/root/reference/rwkv_megatron/rwkv6_layer_specs.py):
//   shift(x)[t] = x[t-1], shift(x)[0] = 0                        :290-300
//   delta = shift(x) - x ; xxx = x + delta * maa_x                :443-444
// The data-dependent lerp of :447-452 is written by the LoRA up-projection kernel
// (lora.hip), which also holds the backward of both lerps.
//
// Channel mix (RWKV6ChannelMix.forward, :512-536) uses the same shift with static
// coefficients mix_coeffs [2,C]:
//   mixed_e = x + delta * mix_coeffs[e], e in (up, gate)          :515-520
//   h = relu(linear_up(mixed_up))^2                               :522-524
//   y = linear_down(h) * sigmoid(linear_gate(mixed_gate))         :525-536
// so it gets a lerp kernel writing [2,T,B,C] (each half a contiguous GEMM operand),
// its backward, and the relu^2 and sigmoid-gate epilogues with their backwards.
// The kernels compute in fp32 registers and round once to bf16 on store; each
// thread owns 8 consecutive channels (one 16-byte vector) so every global
// access is a coalesced 16-byte load or store.  All parameter-gradient
// reductions are two-stage with a fixed order (deterministic).
#include <initializer_list>

#include "common.h"
#include "../../include/rwkv6_amd.h"

#define MIX_THR 256

// The static lerps, out_e[n] = x[n] + (shift(x)[n] - x[n]) * coef[e] (token rows n = t*B + b,
// shift(x)[n] = x[n - B], zero for n < B): xxx = lerp with maa (NE = 1, rwkv6_shift_lerp_fwd),
// or the channel mix's two mixes with mix_coeffs [2,C] (NE = 2, rwkv6_cmix_lerp_fwd).  Thread = 8 channels of
// LERP_ROWS rows (grid.x over channel groups, grid.y over row blocks, striding when the rows
// outnumber the grid): its coefficients are loaded once and all its row loads are in flight
// together (clamped rows: no branch).  8 rows measured 6-8 % faster than 4 at the config-3
// shape (28.4 against 30.8 us for xxx, 38.8 against 40.8 for the two mixes); 16 was slower.
#define LERP_ROWS 8
template <int NE>
__global__ void __launch_bounds__(MIX_THR)
rwkv6_lerp_rows_kernel(const uint16_t* __restrict__ x, const void* __restrict__ coef, int pdt,
                       OutPtrs<NE> out, int64_t N, int64_t B, int64_t C) {
    const int64_t C8 = C / 8, cg = (int64_t)blockIdx.x * MIX_THR + threadIdx.x;
    if (cg >= C8) return;
    float m[NE][8];
#pragma unroll
    for (int e = 0; e < NE; ++e) load_param8(coef, pdt, e * C + 8 * cg, m[e]);
    for (int64_t r0 = (int64_t)blockIdx.y * LERP_ROWS; r0 < N; r0 += (int64_t)gridDim.y * LERP_ROWS) {
        float xv[LERP_ROWS][8], xp[LERP_ROWS][8];
#pragma unroll
        for (int j = 0; j < LERP_ROWS; ++j) {
            const int64_t r = r0 + j < N ? r0 + j : N - 1;
            load8(x + r * C + 8 * cg, xv[j]);
            load8(x + (r >= B ? r - B : r) * C + 8 * cg, xp[j]);
        }
#pragma unroll
        for (int j = 0; j < LERP_ROWS; ++j) {
            const int64_t r = r0 + j;
            const float keep = (r < N ? r : N - 1) >= B ? 1.f : 0.f;
#pragma unroll
            for (int e = 0; e < NE; ++e) {
                float o[8];
#pragma unroll
                for (int s = 0; s < 8; ++s) o[s] = xv[j][s] + (xp[j][s] * keep - xv[j][s]) * m[e][s];
                if (r < N) store8(out.p[e] + r * C + 8 * cg, o);
            }
        }
    }
}
inline dim3 lerp_grid(int64_t N, int64_t C) {
    const int64_t rb = (N + LERP_ROWS - 1) / LERP_ROWS;
    return dim3((unsigned)((C / 8 + MIX_THR - 1) / MIX_THR), (unsigned)(rb < 65535 ? rb : 65535));
}

// Backward kernel: block = 8 token sub-segments x 32 channel groups (256 threads); the
// block covers tokens [64*blockIdx.x, +64) of batch blockIdx.z and channels
// [256*blockIdx.y, +256).  Thread (ss, cgl) walks 8 tokens of 8 channels.  Parameter
// partial sums are reduced over the 8 sub-segments in LDS (fixed order) and written
// per (token block, batch): part[(tblk*B + b)][rows][C].
#define MIX_TB 64          // tokens per block
#define MIX_SS 8           // tokens per thread

// ---------------------------------------------------------------------------------------
// Channel mix.
#define CMIX_NE 2

// Backward of the channel-mix lerp (walked forward with dx[t] emitted one token late; d_delta
// of each sub-segment's first token is handed to the previous sub-segment through LDS):
//   d_delta[t] = sum_e dmix_e[t] mix_e,  dx[t] = sum_e dmix_e[t] - d_delta[t] + d_delta[t+1],
//   d_mix_e partial = sum_t dmix_e[t] delta[t]  -> part[(tblk*B + b)][2][C].
__device__ __forceinline__ void cmix_token(const float* mv, const InPtrs<CMIX_NE>& dmix,
                                           int64_t off, float* dd, float* dsum, float (*g)[8]) {
#pragma unroll
    for (int s = 0; s < 8; ++s) dd[s] = dsum[s] = 0.f;
#pragma unroll
    for (int e = 0; e < CMIX_NE; ++e) {
        load8(dmix.p[e] + off, g[e]);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            dd[s] += g[e][s] * mv[e * 8 + s];
            dsum[s] += g[e][s];
        }
    }
}

__global__ void __launch_bounds__(MIX_THR)
rwkv6_cmix_lerp_bwd_kernel(const uint16_t* __restrict__ x, const void* __restrict__ mix, int pdt,
                           InPtrs<CMIX_NE> dmix, uint16_t* __restrict__ dx,
                           float* __restrict__ part, int64_t T, int64_t B, int64_t C) {
    __shared__ float first_dd[MIX_SS][32][8];
    __shared__ float red[MIX_SS][CMIX_NE][32 * 8 + 4];
    const int ss = threadIdx.x >> 5, cgl = threadIdx.x & 31;
    const int64_t C8 = C / 8, cg = (int64_t)blockIdx.y * 32 + cgl;
    const int64_t b = blockIdx.z;
    const int64_t t_lo = (int64_t)blockIdx.x * MIX_TB + MIX_SS * ss, t_hi = min(T, t_lo + MIX_SS);
    const bool active = cg < C8 && t_lo < T;
    float acc[CMIX_NE][8], pend[8], mv[CMIX_NE * 8];
#pragma unroll
    for (int e = 0; e < CMIX_NE; ++e)
#pragma unroll
        for (int s = 0; s < 8; ++s) acc[e][s] = 0.f;
    if (active) {
#pragma unroll
        for (int e = 0; e < CMIX_NE; ++e) load_param8(mix, pdt, e * C + 8 * cg, mv + 8 * e);
        float xprev[8];
        if (t_lo > 0) load8(x + ((t_lo - 1) * B + b) * C + 8 * cg, xprev);
        else for (int s = 0; s < 8; ++s) xprev[s] = 0.f;
        // The thread's MIX_SS tokens in a fixed, unrolled walk: x and d_mixed of the token two
        // ahead are loaded (clamped to the last token, unconditionally) before this token's
        // arithmetic, so a load's latency overlaps two tokens of work instead of stalling each
        // one (58.5 -> 54.6 us at the config-3 shape; one ahead 56.0, all eight up front 55.2).
        const int n = (int)(t_hi - t_lo);
        auto ld = [&](int j, uint4* r) {
            const int64_t off = ((t_lo + min(j, n - 1)) * B + b) * C + 8 * cg;
            r[0] = *reinterpret_cast<const uint4*>(x + off);
#pragma unroll
            for (int e = 0; e < CMIX_NE; ++e) r[1 + e] = *reinterpret_cast<const uint4*>(dmix.p[e] + off);
        };
        uint4 nxt[1 + CMIX_NE], nx2[1 + CMIX_NE];
        ld(0, nxt);
        ld(1, nx2);
#pragma unroll
        for (int j = 0; j < MIX_SS; ++j) {
            uint4 cur[1 + CMIX_NE];
#pragma unroll
            for (int q = 0; q <= CMIX_NE; ++q) { cur[q] = nxt[q]; nxt[q] = nx2[q]; }
            if (j + 2 < MIX_SS) ld(j + 2, nx2);
            if (j < n) {
                const int64_t off = ((t_lo + j) * B + b) * C + 8 * cg;
                float xv[8], dd[8], dsum[8], g[CMIX_NE][8], out[8];
                unpack8(cur[0], xv);
#pragma unroll
                for (int s = 0; s < 8; ++s) dd[s] = dsum[s] = 0.f;
#pragma unroll
                for (int e = 0; e < CMIX_NE; ++e) {
                    unpack8(cur[1 + e], g[e]);
#pragma unroll
                    for (int s = 0; s < 8; ++s) {
                        dd[s] += g[e][s] * mv[e * 8 + s];
                        dsum[s] += g[e][s];
                    }
                }
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const float delta = xprev[s] - xv[s];
#pragma unroll
                    for (int e = 0; e < CMIX_NE; ++e) acc[e][s] += g[e][s] * delta;
                    xprev[s] = xv[s];
                }
                if (j > 0) {
#pragma unroll
                    for (int s = 0; s < 8; ++s) out[s] = pend[s] + dd[s];
                    store8(dx + off - B * C, out);
                } else {
#pragma unroll
                    for (int s = 0; s < 8; ++s) first_dd[ss][cgl][s] = dd[s];
                }
#pragma unroll
                for (int s = 0; s < 8; ++s) pend[s] = dsum[s] - dd[s];
            }
        }
    }
    __syncthreads();
    if (active) {
        float nd[8];
        if (t_hi >= T) {
#pragma unroll
            for (int s = 0; s < 8; ++s) nd[s] = 0.f;
        } else if (ss + 1 < MIX_SS) {
#pragma unroll
            for (int s = 0; s < 8; ++s) nd[s] = first_dd[ss + 1][cgl][s];
        } else {
            float dsum[8], g[CMIX_NE][8];
            cmix_token(mv, dmix, (t_hi * B + b) * C + 8 * cg, nd, dsum, g);
        }
        float out[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) out[s] = pend[s] + nd[s];
        store8(dx + ((t_hi - 1) * B + b) * C + 8 * cg, out);
    }
#pragma unroll
    for (int e = 0; e < CMIX_NE; ++e)
#pragma unroll
        for (int s = 0; s < 8; ++s) red[ss][e][8 * cgl + s] = acc[e][s];
    __syncthreads();
    const int64_t P_row = (int64_t)blockIdx.x * B + b;
    for (int j = threadIdx.x; j < CMIX_NE * 256; j += MIX_THR) {
        const int e = j >> 8, c = j & 255;
        const int64_t ch = (int64_t)blockIdx.y * 256 + c;
        if (ch >= C) continue;
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < MIX_SS; ++q) sum += red[q][e][c];
        part[(P_row * CMIX_NE + e) * C + ch] = sum;
    }
}

// out[i] = sum_{j < S} part[j][i] (fp32, j in order), written bf16 or fp32: the partial
// weight gradients of a token-split GEMM summed in one pass (instead of a reduction kernel
// writing fp32 and a cast kernel).  Thread = 8 consecutive elements; all S partial loads are
// issued before the sum.
__global__ void __launch_bounds__(MIX_THR)
rwkv6_sum_partials_kernel(const float* __restrict__ part, int S, int64_t n8, int64_t n, int pdt,
                          void* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * MIX_THR + threadIdx.x;
    if (i >= n8) return;
    const float* p = part + 8 * i;
    float acc[8];
    {
        const float4 a = *reinterpret_cast<const float4*>(p);
        const float4 b = *reinterpret_cast<const float4*>(p + 4);
        acc[0] = a.x; acc[1] = a.y; acc[2] = a.z; acc[3] = a.w;
        acc[4] = b.x; acc[5] = b.y; acc[6] = b.z; acc[7] = b.w;
    }
#pragma unroll 4
    for (int j = 1; j < S; ++j) {
        const float4 a = *reinterpret_cast<const float4*>(p + (int64_t)j * n);
        const float4 b = *reinterpret_cast<const float4*>(p + (int64_t)j * n + 4);
        acc[0] += a.x; acc[1] += a.y; acc[2] += a.z; acc[3] += a.w;
        acc[4] += b.x; acc[5] += b.y; acc[6] += b.z; acc[7] += b.w;
    }
    if (pdt == RWKV6_BF16) {
        store8(reinterpret_cast<uint16_t*>(out) + 8 * i, acc);
    } else {
        float* o = reinterpret_cast<float*>(out) + 8 * i;
        *reinterpret_cast<float4*>(o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        *reinterpret_cast<float4*>(o + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
}

// Elementwise epilogues over n bf16 elements (n % 8 == 0); each thread owns EW_VEC 16-byte
// vectors, all loads issued before any arithmetic.  One vector per thread (more, smaller-
// footprint waves) measured faster than two at the config-3 shapes: sigmoid gate backward 54
// against 68 us, forward 36 against 40, relu^2 78 against 83, its backward 139 against 145;
// four were slower still.
#define EW_VEC 1          // 16-byte pieces per thread.  Loads and stores clamp the index
                          // (no branch, so all of a thread's loads are in flight together);
                          // a piece past the end repeats the last one, same value, same place
__device__ __forceinline__ float sigmoid_(float z) { return 1.f / (1.f + __expf(-z)); }

// h = relu(up)^2
__global__ void __launch_bounds__(MIX_THR)
rwkv6_relu_sq_kernel(const uint16_t* __restrict__ up, uint16_t* __restrict__ h, int64_t n8) {
    const int64_t i0 = ((int64_t)blockIdx.x * MIX_THR + threadIdx.x) * EW_VEC;
    float a[EW_VEC][8];
#pragma unroll
    for (int v = 0; v < EW_VEC; ++v)
        load8(up + 8 * min(i0 + v, n8 - 1), a[v]);
#pragma unroll
    for (int v = 0; v < EW_VEC; ++v) {
        const int64_t jo = min(i0 + v, n8 - 1);         // past the end: last piece again
        float o[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float r = fmaxf(a[v][s], 0.f);
            o[s] = r * r;
        }
        store8_nt(h + 8 * jo, o);        // streaming: 77 -> 70 us at the config-3 shape
    }
}

// d_up = 2 relu(up) dh
__global__ void __launch_bounds__(MIX_THR)
rwkv6_relu_sq_bwd_kernel(const uint16_t* __restrict__ up, const uint16_t* __restrict__ dh,
                         uint16_t* __restrict__ dup, int64_t n8) {
    const int64_t i0 = ((int64_t)blockIdx.x * MIX_THR + threadIdx.x) * EW_VEC;
    float a[EW_VEC][8], g[EW_VEC][8];
#pragma unroll
    for (int v = 0; v < EW_VEC; ++v) {
        const int64_t j = min(i0 + v, n8 - 1);
        load8(up + 8 * j, a[v]);
        load8(dh + 8 * j, g[v]);
    }
#pragma unroll
    for (int v = 0; v < EW_VEC; ++v) {
        const int64_t jo = min(i0 + v, n8 - 1);         // past the end: last piece again
        float o[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) o[s] = 2.f * fmaxf(a[v][s], 0.f) * g[v][s];
        store8(dup + 8 * jo, o);
    }
}

// y = out * sigmoid(gate_pre)
__global__ void __launch_bounds__(MIX_THR)
rwkv6_sigmoid_gate_kernel(const uint16_t* __restrict__ out, const uint16_t* __restrict__ gp,
                          uint16_t* __restrict__ y, int64_t n8) {
    const int64_t i0 = ((int64_t)blockIdx.x * MIX_THR + threadIdx.x) * EW_VEC;
    float a[EW_VEC][8], z[EW_VEC][8];
#pragma unroll
    for (int v = 0; v < EW_VEC; ++v) {
        const int64_t j = min(i0 + v, n8 - 1);
        load8(out + 8 * j, a[v]);
        load8(gp + 8 * j, z[v]);
    }
#pragma unroll
    for (int v = 0; v < EW_VEC; ++v) {
        const int64_t jo = min(i0 + v, n8 - 1);         // past the end: last piece again
        float o[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) o[s] = a[v][s] * sigmoid_(z[v][s]);
        store8(y + 8 * jo, o);
    }
}

// d_out = dy sigmoid(z);  d_gate_pre = dy out sigmoid(z) (1 - sigmoid(z))
__global__ void __launch_bounds__(MIX_THR)
rwkv6_sigmoid_gate_bwd_kernel(const uint16_t* __restrict__ out, const uint16_t* __restrict__ gp,
                              const uint16_t* __restrict__ dy, uint16_t* __restrict__ dout,
                              uint16_t* __restrict__ dgp, int64_t n8) {
    const int64_t i0 = ((int64_t)blockIdx.x * MIX_THR + threadIdx.x) * EW_VEC;
    float a[EW_VEC][8], z[EW_VEC][8], g[EW_VEC][8];
#pragma unroll
    for (int v = 0; v < EW_VEC; ++v) {
        const int64_t j = min(i0 + v, n8 - 1);
        load8(out + 8 * j, a[v]);
        load8(gp + 8 * j, z[v]);
        load8(dy + 8 * j, g[v]);
    }
#pragma unroll
    for (int v = 0; v < EW_VEC; ++v) {
        const int64_t jo = min(i0 + v, n8 - 1);         // past the end: last piece again
        float o1[8], o2[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float sg = sigmoid_(z[v][s]);
            o1[s] = g[v][s] * sg;
            o2[s] = g[v][s] * a[v][s] * sg * (1.f - sg);
        }
        store8(dout + 8 * jo, o1);
        store8(dgp + 8 * jo, o2);
    }
}

namespace {
inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int mix_check(int64_t T, int64_t B, int64_t C, int pdt) {
    if (T < 0 || B < 1 || C < 8) return RWKV6_ERR_INVALID_ARG;
    if (C % 8) return RWKV6_ERR_UNSUPPORTED;
    if (pdt != RWKV6_F32 && pdt != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    return RWKV6_OK;
}
inline unsigned nblocks(int64_t n) { return (unsigned)((n + MIX_THR - 1) / MIX_THR); }
// Gathers an array of N device pointers; 0 if one is null, RWKV6_ERR_ALIGNMENT if misaligned.
template <typename P, int N>
inline int gather(const void* const* src, P& dst) {
    if (!src) return RWKV6_ERR_INVALID_ARG;
    for (int e = 0; e < N; ++e) {
        if (!src[e]) return RWKV6_ERR_INVALID_ARG;
        if (!al16(src[e])) return RWKV6_ERR_ALIGNMENT;
        dst.p[e] = (decltype(dst.p[0]))src[e];
    }
    return RWKV6_OK;
}
inline int launch_status() { return hipGetLastError() == hipSuccess ? RWKV6_OK : RWKV6_ERR_LAUNCH; }
}  // namespace

extern "C" {

int rwkv6_shift_lerp_fwd(const void* x, const void* maa, int param_dtype, void* xxx, int64_t T,
                         int64_t B, int64_t C, void* stream) {
    int st = mix_check(T, B, C, param_dtype);
    if (st) return st;
    if (T == 0) return RWKV6_OK;
    if (!x || !maa || !xxx) return RWKV6_ERR_INVALID_ARG;
    if (!al16(x) || !al16(maa) || !al16(xxx)) return RWKV6_ERR_ALIGNMENT;
    const size_t act = (size_t)(T * B * C) * 2;
    if (any_alias({{xxx, act}}, {{x, act}, {maa, (size_t)C * param_bytes(param_dtype)}}))
        return RWKV6_ERR_INVALID_ARG;
    OutPtrs<1> out;
    out.p[0] = (uint16_t*)xxx;
    hipLaunchKernelGGL(rwkv6_lerp_rows_kernel<1>, lerp_grid(T * B, C), dim3(MIX_THR), 0,
                       reinterpret_cast<hipStream_t>(stream), (const uint16_t*)x, maa, param_dtype,
                       out, T * B, B, C);
    return launch_status();
}

static dim3 bwd_grid(int64_t T, int64_t B, int64_t C) {
    return dim3((unsigned)((T + MIX_TB - 1) / MIX_TB), (unsigned)((C / 8 + 31) / 32), (unsigned)B);
}
int rwkv6_cmix_lerp_fwd(const void* x, const void* mix, int param_dtype, void* const* mixed,
                        int64_t T, int64_t B, int64_t C, void* stream) {
    int st = mix_check(T, B, C, param_dtype);
    if (st) return st;
    if (T == 0) return RWKV6_OK;
    if (!x || !mix) return RWKV6_ERR_INVALID_ARG;
    OutPtrs<CMIX_NE> out;
    if ((st = gather<OutPtrs<CMIX_NE>, CMIX_NE>((const void* const*)mixed, out))) return st;
    if (!al16(x) || !al16(mix)) return RWKV6_ERR_ALIGNMENT;
    const size_t act = (size_t)(T * B * C) * 2;
    if (any_alias({{out.p[0], act}, {out.p[1], act}},
                  {{x, act}, {mix, (size_t)CMIX_NE * C * param_bytes(param_dtype)}}))
        return RWKV6_ERR_INVALID_ARG;
    hipLaunchKernelGGL(rwkv6_lerp_rows_kernel<CMIX_NE>, lerp_grid(T * B, C), dim3(MIX_THR), 0,
                       reinterpret_cast<hipStream_t>(stream), (const uint16_t*)x, mix, param_dtype,
                       out, T * B, B, C);
    return launch_status();
}

size_t rwkv6_cmix_lerp_bwd_workspace_bytes(int64_t T, int64_t B, int64_t C) {
    if (T < 0 || B < 1 || C < 8) return 0;
    const int64_t ntb = (T + MIX_TB - 1) / MIX_TB;
    return (size_t)((ntb > 0 ? ntb : 1) * B * CMIX_NE * C) * sizeof(float);
}

int rwkv6_cmix_lerp_bwd(const void* x, const void* mix, int param_dtype,
                        const void* const* d_mixed, void* dx, void* d_mix, void* workspace,
                        int64_t T, int64_t B, int64_t C, void* stream) {
    int st = mix_check(T, B, C, param_dtype);
    if (st) return st;
    if (B > 65535) return RWKV6_ERR_UNSUPPORTED;
    if (!mix || !d_mix || !workspace || (T > 0 && (!x || !dx))) return RWKV6_ERR_INVALID_ARG;
    InPtrs<CMIX_NE> dm{};
    if (T > 0 && (st = gather<InPtrs<CMIX_NE>, CMIX_NE>(d_mixed, dm))) return st;
    if (!al16(x) || !al16(mix) || !al16(dx) || !al16(workspace)) return RWKV6_ERR_ALIGNMENT;
    {
        const size_t act = (size_t)(T * B * C) * 2, par = (size_t)CMIX_NE * C * param_bytes(param_dtype);
        if (any_alias({{dx, act}, {d_mix, par}, {workspace, rwkv6_cmix_lerp_bwd_workspace_bytes(T, B, C)}},
                      {{x, act}, {mix, par}, {dm.p[0], act}, {dm.p[1], act}}))
            return RWKV6_ERR_INVALID_ARG;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t ntb = (T + MIX_TB - 1) / MIX_TB;
    float* part = reinterpret_cast<float*>(workspace);
    if (T > 0)
        hipLaunchKernelGGL(rwkv6_cmix_lerp_bwd_kernel, bwd_grid(T, B, C), dim3(MIX_THR), 0, s,
                           (const uint16_t*)x, mix, param_dtype, dm, (uint16_t*)dx, part, T, B,
                           C);
    launch_partials_reduce(part, T > 0 ? ntb * B : (int64_t)0, (int64_t)CMIX_NE * C, param_dtype,
                           d_mix, nullptr, (int64_t)CMIX_NE * C, s);
    return launch_status();
}

static int ew_check(int64_t n, std::initializer_list<const void*> ptrs) {
    if (n < 0) return RWKV6_ERR_INVALID_ARG;
    if (n % 8) return RWKV6_ERR_UNSUPPORTED;
    if (n == 0) return RWKV6_OK;
    for (const void* p : ptrs) {
        if (!p) return RWKV6_ERR_INVALID_ARG;
        if (!al16(p)) return RWKV6_ERR_ALIGNMENT;
    }
    return RWKV6_OK;
}
static unsigned ew_blocks(int64_t n8) {
    return (unsigned)((n8 + (int64_t)MIX_THR * EW_VEC - 1) / ((int64_t)MIX_THR * EW_VEC));
}

int rwkv6_relu_sq_fwd(const void* up, void* h, int64_t n, void* stream) {
    int st = ew_check(n, {up, h});
    if (st || n == 0) return st;
    if (any_alias({{h, (size_t)n * 2}}, {{up, (size_t)n * 2}})) return RWKV6_ERR_INVALID_ARG;
    hipLaunchKernelGGL(rwkv6_relu_sq_kernel, dim3(ew_blocks(n / 8)), dim3(MIX_THR), 0,
                       reinterpret_cast<hipStream_t>(stream), (const uint16_t*)up, (uint16_t*)h,
                       n / 8);
    return launch_status();
}

int rwkv6_relu_sq_bwd(const void* up, const void* dh, void* d_up, int64_t n, void* stream) {
    int st = ew_check(n, {up, dh, d_up});
    if (st || n == 0) return st;
    const size_t nb = (size_t)n * 2;
    if (any_alias({{d_up, nb}}, {{up, nb}, {dh, nb}})) return RWKV6_ERR_INVALID_ARG;
    hipLaunchKernelGGL(rwkv6_relu_sq_bwd_kernel, dim3(ew_blocks(n / 8)), dim3(MIX_THR), 0,
                       reinterpret_cast<hipStream_t>(stream), (const uint16_t*)up,
                       (const uint16_t*)dh, (uint16_t*)d_up, n / 8);
    return launch_status();
}

int rwkv6_sigmoid_gate_fwd(const void* out, const void* gate_pre, void* y, int64_t n,
                           void* stream) {
    int st = ew_check(n, {out, gate_pre, y});
    if (st || n == 0) return st;
    const size_t nb = (size_t)n * 2;
    if (any_alias({{y, nb}}, {{out, nb}, {gate_pre, nb}})) return RWKV6_ERR_INVALID_ARG;
    hipLaunchKernelGGL(rwkv6_sigmoid_gate_kernel, dim3(ew_blocks(n / 8)), dim3(MIX_THR), 0,
                       reinterpret_cast<hipStream_t>(stream), (const uint16_t*)out,
                       (const uint16_t*)gate_pre, (uint16_t*)y, n / 8);
    return launch_status();
}

int rwkv6_sigmoid_gate_bwd(const void* out, const void* gate_pre, const void* dy, void* d_out,
                           void* d_gate_pre, int64_t n, void* stream) {
    int st = ew_check(n, {out, gate_pre, dy, d_out, d_gate_pre});
    if (st || n == 0) return st;
    const size_t nb = (size_t)n * 2;
    if (any_alias({{d_out, nb}, {d_gate_pre, nb}}, {{out, nb}, {gate_pre, nb}, {dy, nb}}))
        return RWKV6_ERR_INVALID_ARG;
    hipLaunchKernelGGL(rwkv6_sigmoid_gate_bwd_kernel, dim3(ew_blocks(n / 8)), dim3(MIX_THR), 0,
                       reinterpret_cast<hipStream_t>(stream), (const uint16_t*)out,
                       (const uint16_t*)gate_pre, (const uint16_t*)dy, (uint16_t*)d_out,
                       (uint16_t*)d_gate_pre, n / 8);
    return launch_status();
}

int rwkv6_sum_partials(const float* part, int64_t S, int64_t n, int out_dtype, void* out,
                       void* stream) {
    if (S < 1 || S > 64 || n < 0) return RWKV6_ERR_INVALID_ARG;
    if (out_dtype != RWKV6_F32 && out_dtype != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    int st = ew_check(n, {part, out});
    if (st || n == 0) return st;
    if (any_alias({{out, (size_t)n * param_bytes(out_dtype)}}, {{part, (size_t)(S * n) * 4}}))
        return RWKV6_ERR_INVALID_ARG;
    hipLaunchKernelGGL(rwkv6_sum_partials_kernel, dim3(nblocks(n / 8)), dim3(MIX_THR), 0,
                       reinterpret_cast<hipStream_t>(stream), part, (int)S, n / 8, n, out_dtype,
                       out);
    return launch_status();
}

}  // extern "C"
