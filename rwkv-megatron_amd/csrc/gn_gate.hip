// Fused per-head GroupNorm * silu(gate) for MI355X (gfx950), forward and backward.
//
// Reference (/root/reference/rwkv_megatron/rwkv6_layer_specs.py):
//   o = rearrange(wkv_out, "b h t n -> t b (h n)")                     :341
//   y = group_norm(o as [(t b), c], groups = heads, weight, bias, eps)  :90-97, :461-465
//   y = y * silu(linear_gate(mixed_gate))                               :458, :466
// eps is config.layernorm_epsilon (:68).  Without a gate (g_pre = NULL) the kernels are the
// plain GroupNorm of the reference's GroupNorm.forward over [N, C] (:90-97).  One group is
// the 64 channels of one (token, batch, head); 8 lanes own a group, 8 channels (16 bytes)
// each, and reduce with cross-lane shuffles.  The WKV output may be read head-first, which
// fuses away the layout copy of :341.  Parameter-gradient sums are two-stage with a fixed
// order (deterministic).
#include "common.h"
#include "../../include/rwkv6_amd.h"

#define GN_D 64           // channels per group (head size)
#define GN_THR 256        // 32 groups per block pass
#define GN_TT 64          // tokens per block (one (b,h) per block row)

namespace {

__device__ __forceinline__ float sigmoidf_(float z) { return 1.f / (1.f + __expf(-z)); }

// element offset of (t, b, h, channel c0) in o
__device__ __forceinline__ int64_t o_off(int head_first, int64_t t, int64_t b, int64_t h,
                                         int64_t c0, int64_t T, int64_t B, int64_t H) {
    return head_first ? ((b * H + h) * T + t) * GN_D + c0 : ((t * B + b) * H + h) * GN_D + c0;
}

}  // namespace

// grid: (ceil(T / GN_TT), B*H); thread = (group slot gs = tid/8, lane8 = tid%8)
template <bool GATE>
__global__ void __launch_bounds__(GN_THR)
rwkv6_gn_gate_fwd_kernel(const uint16_t* __restrict__ o, int head_first,
                         const uint16_t* __restrict__ g_pre, const void* __restrict__ gamma,
                         const void* __restrict__ beta, int pdt, float eps,
                         uint16_t* __restrict__ y, float* __restrict__ mean_out,
                         float* __restrict__ rstd_out, int64_t T, int64_t B, int64_t H) {
    const int64_t bh = blockIdx.y, b = bh / H, h = bh % H;
    const int gs = threadIdx.x >> 3, l8 = threadIdx.x & 7;
    const int64_t c0 = 8 * l8;
    float ga[8], be[8];
    load_param8(gamma, pdt, h * GN_D + c0, ga);
    load_param8(beta, pdt, h * GN_D + c0, be);
    const int64_t C = H * GN_D;
    for (int p = 0; p < GN_TT / 32; ++p) {
        const int64_t t = (int64_t)blockIdx.x * GN_TT + p * 32 + gs;
        if (t >= T) break;
        float x[8], z[8], out[8];
        load8(o + o_off(head_first, t, b, h, c0, T, B, H), x);
        const int64_t yo = (t * B + b) * C + h * GN_D + c0;
        if (GATE) load8(g_pre + yo, z);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s += x[i];
        const float mean = sum8lanes(s) * (1.f / GN_D);
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) v += (x[i] - mean) * (x[i] - mean);
        const float rstd = rsqrtf(sum8lanes(v) * (1.f / GN_D) + eps);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            out[i] = ((x[i] - mean) * rstd * ga[i] + be[i]) * (GATE ? z[i] * sigmoidf_(z[i]) : 1.f);
        store8(y + yo, out);
        if (l8 == 0) {
            mean_out[(t * B + b) * H + h] = mean;
            rstd_out[(t * B + b) * H + h] = rstd;
        }
    }
}

// Backward.  Partial sums of dgamma/dbeta per block: part[b*nTB + tb][which][h][64].
template <bool GATE>
__global__ void __launch_bounds__(GN_THR)
rwkv6_gn_gate_bwd_kernel(const uint16_t* __restrict__ o, int head_first,
                         const uint16_t* __restrict__ g_pre, const void* __restrict__ gamma,
                         const void* __restrict__ beta, int pdt,
                         const float* __restrict__ mean_in, const float* __restrict__ rstd_in,
                         const uint16_t* __restrict__ dy, uint16_t* __restrict__ d_o,
                         uint16_t* __restrict__ d_g, float* __restrict__ part, int64_t T,
                         int64_t B, int64_t H) {
    __shared__ float red[2][32][GN_D + 1];
    const int64_t bh = blockIdx.y, b = bh / H, h = bh % H;
    const int gs = threadIdx.x >> 3, l8 = threadIdx.x & 7;
    const int64_t c0 = 8 * l8;
    const int64_t C = H * GN_D;
    float ga[8], be[8], accg[8], accb[8];
    load_param8(gamma, pdt, h * GN_D + c0, ga);
    load_param8(beta, pdt, h * GN_D + c0, be);
#pragma unroll
    for (int i = 0; i < 8; ++i) accg[i] = accb[i] = 0.f;
    for (int p = 0; p < GN_TT / 32; ++p) {
        const int64_t t = (int64_t)blockIdx.x * GN_TT + p * 32 + gs;
        if (t >= T) break;
        float x[8], z[8], g[8], xh[8], dxh[8], outo[8], outg[8];
        const int64_t oo = o_off(head_first, t, b, h, c0, T, B, H);
        const int64_t yo = (t * B + b) * C + h * GN_D + c0;
        load8(o + oo, x);
        if (GATE) load8(g_pre + yo, z);
        load8(dy + yo, g);
        const float mean = mean_in[(t * B + b) * H + h], rstd = rstd_in[(t * B + b) * H + h];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            xh[i] = (x[i] - mean) * rstd;
            float dn = g[i];
            if (GATE) {
                const float sg = sigmoidf_(z[i]);
                const float n = xh[i] * ga[i] + be[i];
                outg[i] = g[i] * n * sg * (1.f + z[i] * (1.f - sg));
                dn = g[i] * (z[i] * sg);
            }
            accg[i] += dn * xh[i];
            accb[i] += dn;
            dxh[i] = dn * ga[i];
            s1 += dxh[i];
            s2 += dxh[i] * xh[i];
        }
        s1 = sum8lanes(s1) * (1.f / GN_D);
        s2 = sum8lanes(s2) * (1.f / GN_D);
#pragma unroll
        for (int i = 0; i < 8; ++i) outo[i] = rstd * (dxh[i] - s1 - xh[i] * s2);
        store8(d_o + oo, outo);
        if (GATE) store8(d_g + yo, outg);
    }
    // reduce the 32 group slots of this block (fixed order)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        red[0][gs][c0 + i] = accg[i];
        red[1][gs][c0 + i] = accb[i];
    }
    __syncthreads();
    if (threadIdx.x < 2 * GN_D) {
        const int which = threadIdx.x / GN_D, c = threadIdx.x % GN_D;
        float acc = 0.f;
        for (int j = 0; j < 32; ++j) acc += red[which][j][c];
        const int64_t nTB = gridDim.x;
        part[(((b * nTB + blockIdx.x) * 2 + which) * H + h) * GN_D + c] = acc;
    }
}

namespace {
inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int gn_check(int64_t T, int64_t B, int64_t H, int64_t K, int pdt) {
    if (T < 0 || B < 1 || H < 1 || K < 1) return RWKV6_ERR_INVALID_ARG;
    if (K != GN_D) return RWKV6_ERR_UNSUPPORTED;
    if (B * H > 65535) return RWKV6_ERR_UNSUPPORTED;
    if (pdt != RWKV6_F32 && pdt != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    return RWKV6_OK;
}
inline int launch_status() { return hipGetLastError() == hipSuccess ? RWKV6_OK : RWKV6_ERR_LAUNCH; }
}  // namespace

extern "C" {

int rwkv6_gn_gate_fwd(const void* o, int head_first, const void* g_pre, const void* gamma,
                      const void* beta, int param_dtype, float eps, void* y, float* mean,
                      float* rstd, int64_t T, int64_t B, int64_t H, int64_t K, void* stream) {
    int st = gn_check(T, B, H, K, param_dtype);
    if (st) return st;
    if (T == 0) return RWKV6_OK;
    if (!o || !gamma || !beta || !y || !mean || !rstd) return RWKV6_ERR_INVALID_ARG;
    if (!al16(o) || !al16(g_pre) || !al16(gamma) || !al16(beta) || !al16(y))
        return RWKV6_ERR_ALIGNMENT;
    const size_t act = (size_t)(T * B * H * GN_D) * 2, st4 = (size_t)(T * B * H) * 4,
                 par = (size_t)(H * GN_D) * param_bytes(param_dtype);
    if (any_alias({{y, act}, {mean, st4}, {rstd, st4}},
                  {{o, act}, {g_pre, act}, {gamma, par}, {beta, par}}))
        return RWKV6_ERR_INVALID_ARG;
    dim3 grid((unsigned)((T + GN_TT - 1) / GN_TT), (unsigned)(B * H));
    hipLaunchKernelGGL(g_pre ? rwkv6_gn_gate_fwd_kernel<true> : rwkv6_gn_gate_fwd_kernel<false>,
                       grid, dim3(GN_THR), 0, reinterpret_cast<hipStream_t>(stream),
                       (const uint16_t*)o, head_first, (const uint16_t*)g_pre, gamma, beta,
                       param_dtype, eps, (uint16_t*)y, mean, rstd, T, B, H);
    return launch_status();
}

size_t rwkv6_gn_gate_bwd_workspace_bytes(int64_t T, int64_t B, int64_t H, int64_t K) {
    if (T < 0 || B < 1 || H < 1 || K != GN_D) return 0;
    const int64_t nTB = (T + GN_TT - 1) / GN_TT;
    return (size_t)((nTB > 0 ? nTB : 1) * B * H * 2 * GN_D) * sizeof(float);
}

int rwkv6_gn_gate_bwd(const void* o, int head_first, const void* g_pre, const void* gamma,
                      const void* beta, int param_dtype, const float* mean, const float* rstd,
                      const void* dy, void* d_o, void* d_g_pre, void* dgamma, void* dbeta,
                      void* workspace, int64_t T, int64_t B, int64_t H, int64_t K,
                      void* stream) {
    int st = gn_check(T, B, H, K, param_dtype);
    if (st) return st;
    if (!gamma || !beta || !dgamma || !dbeta || !workspace || (!g_pre != !d_g_pre) ||
        (T > 0 && (!o || !mean || !rstd || !dy || !d_o)))
        return RWKV6_ERR_INVALID_ARG;
    if (!al16(o) || !al16(g_pre) || !al16(gamma) || !al16(beta) || !al16(dy) || !al16(d_o) ||
        !al16(d_g_pre) || !al16(workspace))
        return RWKV6_ERR_ALIGNMENT;
    {
        const size_t act = (size_t)(T * B * H * GN_D) * 2, st4 = (size_t)(T * B * H) * 4,
                     par = (size_t)(H * GN_D) * param_bytes(param_dtype);
        if (any_alias({{d_o, act}, {d_g_pre, act}, {dgamma, par}, {dbeta, par},
                       {workspace, rwkv6_gn_gate_bwd_workspace_bytes(T, B, H, K)}},
                      {{o, act}, {g_pre, act}, {gamma, par}, {beta, par}, {mean, st4}, {rstd, st4},
                       {dy, act}}))
            return RWKV6_ERR_INVALID_ARG;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t nTB = (T + GN_TT - 1) / GN_TT;
    if (T > 0) {
        dim3 grid((unsigned)nTB, (unsigned)(B * H));
        hipLaunchKernelGGL(g_pre ? rwkv6_gn_gate_bwd_kernel<true> : rwkv6_gn_gate_bwd_kernel<false>,
                           grid, dim3(GN_THR), 0, s, (const uint16_t*)o, head_first,
                           (const uint16_t*)g_pre, gamma, beta, param_dtype, mean, rstd,
                           (const uint16_t*)dy, (uint16_t*)d_o, (uint16_t*)d_g_pre,
                           (float*)workspace, T, B, H);
    }
    // partials [P][2 C]: dgamma columns, then dbeta
    launch_partials_reduce((const float*)workspace, T > 0 ? B * nTB : (int64_t)0, 2 * H * GN_D,
                           param_dtype, dgamma, dbeta, H * GN_D, s);
    return launch_status();
}

}  // extern "C"
