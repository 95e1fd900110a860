// Fused token shift + lerp + data-dependent lerp of RWKV6TimeMix.forward, and
// the fused backward of both, for MI355X (gfx950).  Sequence-first [T,B,C] bf16.
//
// Reference (/root/reference/rwkv_megatron/rwkv6_layer_specs.py):
//   shift(x)[t] = x[t-1], shift(x)[0] = 0                        :290-300
//   delta = shift(x) - x ; xxx = x + delta * maa_x                :443-444
//   m = bottleneck_token_shift(xxx) (LoRA; its bias is :195)      :446
//   mixed_e = x + delta * m_e, e in (w,k,v,r,g)                   :447-452
// The LoRA output m is laid out e-outer ([5,T,B,C]) so batched GEMMs produce and
// consume it without copies.
// The kernels compute in fp32 registers and round once to bf16 on store; each
// thread owns 8 consecutive channels (one 16-byte vector) so every global
// access is a coalesced 16-byte load or store.  All parameter-gradient
// reductions are two-stage with a fixed order (deterministic).
#include "common.h"
#include "../../include/rwkv6_amd.h"

#define MIX_NE 5          // number of data-dependent mixes (w,k,v,r,g)
#define MIX_SEG 64        // tokens walked per thread in the backward
#define MIX_THR 256

namespace {

__device__ __forceinline__ void load8(const uint16_t* p, float* f) {
    unpack8(*reinterpret_cast<const uint4*>(p), f);
}
__device__ __forceinline__ void store8(uint16_t* p, const float* f) {
    uint4 q;
    q.x = (uint32_t)f2bf(f[0]) | ((uint32_t)f2bf(f[1]) << 16);
    q.y = (uint32_t)f2bf(f[2]) | ((uint32_t)f2bf(f[3]) << 16);
    q.z = (uint32_t)f2bf(f[4]) | ((uint32_t)f2bf(f[5]) << 16);
    q.w = (uint32_t)f2bf(f[6]) | ((uint32_t)f2bf(f[7]) << 16);
    *reinterpret_cast<uint4*>(p) = q;
}
__device__ __forceinline__ void load_param8(const void* p, int dtype, int64_t off, float* f) {
    if (dtype == RWKV6_BF16) {
        load8(reinterpret_cast<const uint16_t*>(p) + off, f);
    } else {
        const float4* q = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + off);
        float4 a = q[0], b = q[1];
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    }
}

}  // namespace

// xxx = x + (shift(x) - x) * maa
__global__ void __launch_bounds__(MIX_THR)
rwkv6_shift_lerp_kernel(const uint16_t* __restrict__ x, const void* __restrict__ maa, int pdt,
                        uint16_t* __restrict__ xxx, int64_t T, int64_t B, int64_t C) {
    const int64_t C8 = C / 8;
    const int64_t idx = (int64_t)blockIdx.x * MIX_THR + threadIdx.x;
    if (idx >= T * B * C8) return;
    const int64_t cg = idx % C8, tb = idx / C8;
    const int64_t off = tb * C + 8 * cg;
    float xv[8], xp[8], m[8], out[8];
    load8(x + off, xv);
    if (tb >= B) load8(x + off - B * C, xp);
    else for (int s = 0; s < 8; ++s) xp[s] = 0.f;
    load_param8(maa, pdt, 8 * cg, m);
#pragma unroll
    for (int s = 0; s < 8; ++s) out[s] = xv[s] + (xp[s] - xv[s]) * m[s];
    store8(xxx + off, out);
}

// mixed[e] = x + (shift(x) - x) * (mexp[e] + bias[e]);  mexp, mixed: [5,T,B,C]
__global__ void __launch_bounds__(MIX_THR)
rwkv6_ddlerp_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ mexp,
                    const void* __restrict__ bias, int pdt, uint16_t* __restrict__ mixed,
                    int64_t T, int64_t B, int64_t C) {
    const int64_t C8 = C / 8;
    const int64_t idx = (int64_t)blockIdx.x * MIX_THR + threadIdx.x;
    const int64_t N = T * B;
    if (idx >= N * C8) return;
    const int64_t cg = idx % C8, tb = idx / C8;
    const int64_t off = tb * C + 8 * cg;
    float xv[8], d[8];
    load8(x + off, xv);
    if (tb >= B) {
        load8(x + off - B * C, d);
#pragma unroll
        for (int s = 0; s < 8; ++s) d[s] -= xv[s];
    } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) d[s] = -xv[s];
    }
#pragma unroll
    for (int e = 0; e < MIX_NE; ++e) {
        float m[8], bb[8], out[8];
        load8(mexp + e * N * C + off, m);
        load_param8(bias, pdt, e * C + 8 * cg, bb);
#pragma unroll
        for (int s = 0; s < 8; ++s) out[s] = xv[s] + d[s] * (m[s] + bb[s]);
        store8(mixed + e * N * C + off, out);
    }
}

// d_mexp[e][t] = d_mixed[e][t] * delta[t]; part[(seg*B + b)][e][C] = sum over the
// segment's tokens (thread = (segment of MIX_SEG tokens, batch b, 8 channels)).
__global__ void __launch_bounds__(MIX_THR)
rwkv6_ddlerp_bwd_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ dmix,
                        uint16_t* __restrict__ dmexp, float* __restrict__ part, int64_t T,
                        int64_t B, int64_t C) {
    const int64_t C8 = C / 8;
    const int64_t nseg = (T + MIX_SEG - 1) / MIX_SEG;
    const int64_t idx = (int64_t)blockIdx.x * MIX_THR + threadIdx.x;
    if (idx >= nseg * B * C8) return;
    const int64_t cg = idx % C8, rest = idx / C8;
    const int64_t b = rest % B, seg = rest / B;
    const int64_t N = T * B;
    const int64_t t_lo = seg * MIX_SEG, t_hi = min(T, t_lo + MIX_SEG);
    float acc[MIX_NE][8];
#pragma unroll
    for (int e = 0; e < MIX_NE; ++e)
#pragma unroll
        for (int s = 0; s < 8; ++s) acc[e][s] = 0.f;
    float xprev[8];
    if (t_lo > 0) load8(x + ((t_lo - 1) * B + b) * C + 8 * cg, xprev);
    else for (int s = 0; s < 8; ++s) xprev[s] = 0.f;
    for (int64_t t = t_lo; t < t_hi; ++t) {
        const int64_t off = (t * B + b) * C + 8 * cg;
        float xv[8], delta[8];
        load8(x + off, xv);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            delta[s] = xprev[s] - xv[s];
            xprev[s] = xv[s];
        }
#pragma unroll
        for (int e = 0; e < MIX_NE; ++e) {
            float g[8], out[8];
            load8(dmix + e * N * C + off, g);
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                out[s] = g[s] * delta[s];
                acc[e][s] += out[s];
            }
            store8(dmexp + e * N * C + off, out);
        }
    }
    float* pp = part + (seg * B + b) * MIX_NE * C + 8 * cg;
#pragma unroll
    for (int e = 0; e < MIX_NE; ++e) {
        float4* q = reinterpret_cast<float4*>(pp + e * C);
        q[0] = make_float4(acc[e][0], acc[e][1], acc[e][2], acc[e][3]);
        q[1] = make_float4(acc[e][4], acc[e][5], acc[e][6], acc[e][7]);
    }
}

// Input gradient of both lerps.  Thread = (segment, batch b, 8 channels), walking
// its tokens from last to first and carrying d_delta[t+1]:
//   d_delta[t] = sum_e dmix_e[t] m_e[t] + dxxx[t] maa,   m_e = mexp_e + bias_e
//   dx[t]      = sum_e dmix_e[t] + dxxx[t] - d_delta[t] + d_delta[t+1]
//   part[(seg*B + b)][C] = sum over the segment of dxxx[t] delta[t]   (d_maa)
__device__ __forceinline__ void mix_token(const uint16_t* __restrict__ mexp, const float* bb,
                                          const float* mv, const uint16_t* __restrict__ dmix,
                                          const uint16_t* __restrict__ dxxx, int64_t off,
                                          int64_t NC, float* dd, float* dsum, float* dxv) {
    if (dxxx) load8(dxxx + off, dxv);
    else for (int s = 0; s < 8; ++s) dxv[s] = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        dd[s] = dxv[s] * mv[s];
        dsum[s] = dxv[s];
    }
#pragma unroll
    for (int e = 0; e < MIX_NE; ++e) {
        float m[8], g[8];
        load8(mexp + e * NC + off, m);
        load8(dmix + e * NC + off, g);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            dd[s] += g[s] * (m[s] + bb[e * 8 + s]);
            dsum[s] += g[s];
        }
    }
}

__global__ void __launch_bounds__(MIX_THR)
rwkv6_mix_bwd_kernel(const uint16_t* __restrict__ x, const void* __restrict__ maa,
                     const uint16_t* __restrict__ mexp, const void* __restrict__ bias, int pdt,
                     const uint16_t* __restrict__ dmix, const uint16_t* __restrict__ dxxx,
                     uint16_t* __restrict__ dx, float* __restrict__ part, int64_t T, int64_t B,
                     int64_t C) {
    const int64_t C8 = C / 8;
    const int64_t nseg = (T + MIX_SEG - 1) / MIX_SEG;
    const int64_t idx = (int64_t)blockIdx.x * MIX_THR + threadIdx.x;
    if (idx >= nseg * B * C8) return;
    const int64_t cg = idx % C8, rest = idx / C8;
    const int64_t b = rest % B, seg = rest / B;
    const int64_t NC = T * B * C;
    const int64_t t_lo = seg * MIX_SEG, t_hi = min(T, t_lo + MIX_SEG);
    float mv[8], bb[MIX_NE * 8];
    load_param8(maa, pdt, 8 * cg, mv);
#pragma unroll
    for (int e = 0; e < MIX_NE; ++e) load_param8(bias, pdt, e * C + 8 * cg, bb + 8 * e);
    float dnext[8], acc[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[s] = 0.f;
    if (t_hi < T) {
        float dsum[8], dxv[8];
        mix_token(mexp, bb, mv, dmix, dxxx, (t_hi * B + b) * C + 8 * cg, NC, dnext, dsum, dxv);
    } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) dnext[s] = 0.f;
    }
    float xcur[8];
    load8(x + ((t_hi - 1) * B + b) * C + 8 * cg, xcur);
    for (int64_t t = t_hi - 1; t >= t_lo; --t) {
        const int64_t off = (t * B + b) * C + 8 * cg;
        float xprev[8], dd[8], dsum[8], dxv[8], out[8];
        if (t > 0) load8(x + off - B * C, xprev);
        else for (int s = 0; s < 8; ++s) xprev[s] = 0.f;
        mix_token(mexp, bb, mv, dmix, dxxx, off, NC, dd, dsum, dxv);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            out[s] = dsum[s] - dd[s] + dnext[s];
            acc[s] += dxv[s] * (xprev[s] - xcur[s]);
            dnext[s] = dd[s];
            xcur[s] = xprev[s];
        }
        store8(dx + off, out);
    }
    float4* q = reinterpret_cast<float4*>(part + (seg * B + b) * C + 8 * cg);
    q[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    q[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

// out[n] = sum_p part[p][n] for n < Nn, in param dtype; fixed order.
__global__ void __launch_bounds__(MIX_THR)
rwkv6_col_reduce(const float* __restrict__ part, int64_t P, int64_t Nn, int pdt,
                 void* __restrict__ out) {
    const int64_t n = (int64_t)blockIdx.x * MIX_THR + threadIdx.x;
    if (n >= Nn) return;
    float acc = 0.f;
    for (int64_t p = 0; p < P; ++p) acc += part[p * Nn + n];
    if (pdt == RWKV6_BF16) reinterpret_cast<uint16_t*>(out)[n] = f2bf(acc);
    else reinterpret_cast<float*>(out)[n] = acc;
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
    const int64_t n = T * B * (C / 8);
    hipLaunchKernelGGL(rwkv6_shift_lerp_kernel, dim3(nblocks(n)), dim3(MIX_THR), 0,
                       reinterpret_cast<hipStream_t>(stream), (const uint16_t*)x, maa, param_dtype,
                       (uint16_t*)xxx, T, B, C);
    return launch_status();
}

int rwkv6_ddlerp_fwd(const void* x, const void* mexp, const void* bias, int param_dtype,
                     void* mixed, int64_t T, int64_t B, int64_t C, void* stream) {
    int st = mix_check(T, B, C, param_dtype);
    if (st) return st;
    if (T == 0) return RWKV6_OK;
    if (!x || !mexp || !bias || !mixed) return RWKV6_ERR_INVALID_ARG;
    if (!al16(x) || !al16(mexp) || !al16(bias) || !al16(mixed)) return RWKV6_ERR_ALIGNMENT;
    const int64_t n = T * B * (C / 8);
    hipLaunchKernelGGL(rwkv6_ddlerp_kernel, dim3(nblocks(n)), dim3(MIX_THR), 0,
                       reinterpret_cast<hipStream_t>(stream), (const uint16_t*)x,
                       (const uint16_t*)mexp, bias, param_dtype, (uint16_t*)mixed, T, B, C);
    return launch_status();
}

size_t rwkv6_ddlerp_bwd_workspace_bytes(int64_t T, int64_t B, int64_t C) {
    if (T < 0 || B < 1 || C < 8) return 0;
    const int64_t nseg = (T + MIX_SEG - 1) / MIX_SEG;
    return (size_t)((nseg > 0 ? nseg : 1) * B * MIX_NE * C) * sizeof(float);
}

int rwkv6_ddlerp_bwd(const void* x, const void* d_mixed, int param_dtype, void* d_mexp,
                     void* d_bias, void* workspace, int64_t T, int64_t B, int64_t C,
                     void* stream) {
    int st = mix_check(T, B, C, param_dtype);
    if (st) return st;
    if (!d_bias || !workspace || (T > 0 && (!x || !d_mixed || !d_mexp))) return RWKV6_ERR_INVALID_ARG;
    if (!al16(x) || !al16(d_mixed) || !al16(d_mexp) || !al16(workspace)) return RWKV6_ERR_ALIGNMENT;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t nseg = (T + MIX_SEG - 1) / MIX_SEG;
    float* part = reinterpret_cast<float*>(workspace);
    if (T > 0)
        hipLaunchKernelGGL(rwkv6_ddlerp_bwd_kernel, dim3(nblocks(nseg * B * (C / 8))), dim3(MIX_THR),
                           0, s, (const uint16_t*)x, (const uint16_t*)d_mixed, (uint16_t*)d_mexp,
                           part, T, B, C);
    hipLaunchKernelGGL(rwkv6_col_reduce, dim3(nblocks(MIX_NE * C)), dim3(MIX_THR), 0, s, part,
                       T > 0 ? nseg * B : (int64_t)0, (int64_t)MIX_NE * C, param_dtype, d_bias);
    return launch_status();
}

size_t rwkv6_mix_bwd_workspace_bytes(int64_t T, int64_t B, int64_t C) {
    if (T < 0 || B < 1 || C < 8) return 0;
    const int64_t nseg = (T + MIX_SEG - 1) / MIX_SEG;
    return (size_t)((nseg > 0 ? nseg : 1) * B * C) * sizeof(float);
}

int rwkv6_mix_bwd(const void* x, const void* maa, const void* mexp, const void* bias,
                  int param_dtype, const void* d_mixed, const void* d_xxx, void* dx,
                  void* d_maa, void* workspace, int64_t T, int64_t B, int64_t C,
                  void* stream) {
    int st = mix_check(T, B, C, param_dtype);
    if (st) return st;
    if (!maa || !bias || !d_maa || !workspace || (T > 0 && (!x || !mexp || !d_mixed || !dx)))
        return RWKV6_ERR_INVALID_ARG;
    if (!al16(x) || !al16(maa) || !al16(mexp) || !al16(bias) || !al16(d_mixed) ||
        (d_xxx && !al16(d_xxx)) || !al16(dx) || !al16(workspace))
        return RWKV6_ERR_ALIGNMENT;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t nseg = (T + MIX_SEG - 1) / MIX_SEG;
    float* part = reinterpret_cast<float*>(workspace);
    if (T > 0)
        hipLaunchKernelGGL(rwkv6_mix_bwd_kernel, dim3(nblocks(nseg * B * (C / 8))), dim3(MIX_THR), 0,
                           s, (const uint16_t*)x, maa, (const uint16_t*)mexp, bias, param_dtype,
                           (const uint16_t*)d_mixed, (const uint16_t*)d_xxx, (uint16_t*)dx, part,
                           T, B, C);
    hipLaunchKernelGGL(rwkv6_col_reduce, dim3(nblocks(C)), dim3(MIX_THR), 0, s, part,
                       T > 0 ? nseg * B : (int64_t)0, C, param_dtype, d_maa);
    return launch_status();
}

}  // extern "C"
