// Shared device helpers for the gfx950 (CDNA4) kernels of the RWKV-6 time-mix path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// log2(e): decays are kept in base-2 log units so every exponential is one v_exp_f32.
#define RW_L2E 1.4426950408889634f

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// two fp32 -> two bf16 (a in the low half), the same rounding as f2bf, in one
// v_cvt_pk_bf16_f32 instead of two conversions, a shift and an or
__device__ __forceinline__ uint32_t pk2(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ uint4 pack8(const float* f) {
    return make_uint4(pk2(f[0], f[1]), pk2(f[2], f[3]), pk2(f[4], f[5]), pk2(f[6], f[7]));
}
__device__ __forceinline__ bf16x4 cvt4(float a, float b, float c, float d) {
    return __builtin_bit_cast(bf16x4, make_uint2(pk2(a, b), pk2(c, d)));
}
// 2^x with the hardware base-2 exponential (v_exp_f32).
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }
// a.x*b.x + a.y*b.y + a.z*b.z + a.w*b.w of two packed bf16x4 (uint2), fp32 sums (v_dot2).
__device__ __forceinline__ float dot4_bf16(uint2 a, uint2 b) {
    const float lo = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.x),
                                                     __builtin_bit_cast(bf16x2, b.x), 0.f, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.y),
                                           __builtin_bit_cast(bf16x2, b.y), lo, false);
}

__device__ __forceinline__ f32x4 mfma32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(bf16x4 a, bf16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld_bf16x8(const uint16_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ bf16x4 ld_bf16x4(const uint16_t* p) {
    return __builtin_bit_cast(bf16x4, *reinterpret_cast<const uint2*>(p));
}
__device__ __forceinline__ void unpack8(uint4 q, float* f) {
    f[0] = __uint_as_float(q.x << 16); f[1] = __uint_as_float(q.x & 0xffff0000u);
    f[2] = __uint_as_float(q.y << 16); f[3] = __uint_as_float(q.y & 0xffff0000u);
    f[4] = __uint_as_float(q.z << 16); f[5] = __uint_as_float(q.z & 0xffff0000u);
    f[6] = __uint_as_float(q.w << 16); f[7] = __uint_as_float(q.w & 0xffff0000u);
}
__device__ __forceinline__ void unpack4(uint2 q, float* f) {
    f[0] = __uint_as_float(q.x << 16); f[1] = __uint_as_float(q.x & 0xffff0000u);
    f[2] = __uint_as_float(q.y << 16); f[3] = __uint_as_float(q.y & 0xffff0000u);
}

// The mixes are separate [T,B,C] tensors (each one the input or input-gradient of its own
// projection); kernels receive their addresses by value.
template <int N> struct OutPtrs { uint16_t* p[N]; };
template <int N> struct InPtrs { const uint16_t* p[N]; };

// 8 consecutive bf16 <-> fp32 through one 16-byte access.
__device__ __forceinline__ void load8(const uint16_t* p, float* f) {
    unpack8(*reinterpret_cast<const uint4*>(p), f);
}
__device__ __forceinline__ void store8(uint16_t* p, const float* f) {
    *reinterpret_cast<uint4*>(p) = pack8(f);
}
// The same as a nontemporal (streaming) store: for large outputs written once and not read
// back by the same kernel; it measured much faster for the LoRA up-projection's five mixes
// and slower for some other outputs, so each call site chooses.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store8_nt(uint16_t* p, const float* f) {
    const uint4 q = pack8(f);
    const u32x4_t v = {q.x, q.y, q.z, q.w};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(p));
}
// 8 consecutive parameters (RWKV6_BF16 or RWKV6_F32, the codes of rwkv6_amd.h) as fp32.
// Branch-free: both forms issue two 16-byte loads from in-bounds addresses (the bf16 form
// reads its one piece twice) and select the converted values, so the caller's other loads
// stay in flight (a load under a branch makes the merge wait for every outstanding load).
__device__ __forceinline__ void load_param8(const void* p, int dtype, int64_t off, float* f) {
    const bool h = dtype == 1;
    const char* b = reinterpret_cast<const char*>(p) + (h ? off * 2 : off * 4);
    const uint4 x = *reinterpret_cast<const uint4*>(b);
    const uint4 y = *reinterpret_cast<const uint4*>(b + (h ? 0 : 16));
    float hf[8];
    unpack8(x, hf);
    const unsigned w[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
#pragma unroll
    for (int s = 0; s < 8; ++s) f[s] = h ? hf[s] : __builtin_bit_cast(float, w[s]);
}

// Lane exchanges without an address operand: DPP (a modifier of the consuming VALU op)
// within rows of 16 lanes, ds_swizzle within 32 lanes; only the exchange across the two
// 32-lane halves goes through ds_bpermute.
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_xor1(float v) { return dpp_mov<0xB1>(v); }   // quad_perm 1,0,3,2
__device__ __forceinline__ float lane_xor2(float v) { return dpp_mov<0x4E>(v); }   // quad_perm 2,3,0,1
__device__ __forceinline__ float lane_xor8(float v) { return dpp_mov<0x128>(v); }  // row_ror:8
template <int M> __device__ __forceinline__ float lane_xor_swz(float v) {          // M < 32
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v),
                                                                 0x1F | (M << 10)));
}
__device__ __forceinline__ float lane_xor32(float v) { return __shfl_xor(v, 32); }
// Sums across the four 16-lane rows of a wave (lane = 16 lq + lr) on the VALU, with gfx950's
// row swaps instead of LDS-pipe shuffles.  With both operands x, v_permlane16_swap leaves the
// even row of each row pair in the first result and the odd row in the second (rows 0,1 ->
// x_0, x_1; rows 2,3 -> x_2, x_3, in every lane of the pair), and v_permlane32_swap leaves
// rows {0,1} in the first and rows {2,3} in the second (probed on the device).
struct RowSums {
    float pair;        // x_0 + x_1 in rows 0 and 1, x_2 + x_3 in rows 2 and 3
    float lo, hi;      // x_0 + x_1 and x_2 + x_3, in every lane
};
__device__ __forceinline__ RowSums row_sums(float x) {
    const unsigned b = __float_as_uint(x);
    const auto r16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    RowSums r;
    r.pair = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const unsigned pb = __float_as_uint(r.pair);
    const auto r32 = __builtin_amdgcn_permlane32_swap(pb, pb, false, false);
    r.lo = __uint_as_float(r32[0]);
    r.hi = __uint_as_float(r32[1]);
    return r;
}

// Sum over aligned groups of 8 lanes; all 8 lanes get the same bits.  The last step adds
// the other quad through row_half_mirror (lane i <-> lane 7 - i of the group).
__device__ __forceinline__ float sum8lanes(float v) {
    v += lane_xor1(v);
    v += lane_xor2(v);
    v += dpp_mov<0x141>(v);
    return v;
}

// Host side: a device buffer as (address, bytes).  Entry points reject calls where an output
// overlaps an input or another output: several kernels re-load a clamped last piece after
// other threads have stored theirs, and the walks read chunk c + 1 before storing chunk c, so
// an aliased output would be read back as an input.  Null pointers and empty spans never
// overlap.
struct Span {
    const void* p;
    size_t n;
};
inline bool spans_overlap(const Span& a, const Span& b) {
    if (!a.p || !b.p || !a.n || !b.n) return false;
    const char* x = static_cast<const char*>(a.p);
    const char* y = static_cast<const char*>(b.p);
    return x < y + b.n && y < x + a.n;
}
// bytes of one parameter element (RWKV6_BF16 = 1 -> 2, RWKV6_F32 = 0 -> 4)
inline size_t param_bytes(int dtype) { return dtype == 1 ? 2 : 4; }
inline bool any_alias(std::initializer_list<Span> outs, std::initializer_list<Span> ins) {
    for (const Span* o = outs.begin(); o != outs.end(); ++o) {
        for (const Span& i : ins)
            if (spans_overlap(*o, i)) return true;
        for (const Span* o2 = o + 1; o2 != outs.end(); ++o2)
            if (spans_overlap(*o, *o2)) return true;
    }
    return false;
}

// Second stage of every fixed-order reduction over token blocks: out[n] = sum_p part[p][n]
// for fp32 partials part[P][Nn], written bf16 or fp32 (pdt); columns n >= split go to
// out2[n - split] (split = Nn: all to out).  Thread (q, nl) of a 256-thread block sums the
// rows q, q + 8, ... of column 32 blockIdx.x + nl in order, eight loads in flight (clamped:
// a row past the end reads the last row and adds zero), then the eight row-lane sums are
// added in order: deterministic, and the same at every launch.  P = 0 writes zeros.
#define PR_THR 256
#define PR_BATCH 8
namespace {
__global__ void __launch_bounds__(PR_THR)
partials_reduce_kernel(const float* __restrict__ part, int64_t P, int64_t Nn, int pdt,
                       void* __restrict__ out, void* __restrict__ out2, int64_t split) {
    __shared__ float acc8[8][32];
    const int q = threadIdx.x >> 5, nl = threadIdx.x & 31;
    const int64_t n = (int64_t)blockIdx.x * 32 + nl, nc = n < Nn ? n : Nn - 1;
    float acc = 0.f;
    for (int64_t p0 = q; p0 < P; p0 += 8 * PR_BATCH) {
        float v[PR_BATCH];
#pragma unroll
        for (int k = 0; k < PR_BATCH; ++k) {
            const int64_t p = p0 + 8 * k;
            v[k] = part[(p < P ? p : P - 1) * Nn + nc];
        }
#pragma unroll
        for (int k = 0; k < PR_BATCH; ++k) acc += p0 + 8 * k < P ? v[k] : 0.f;
    }
    acc8[q][nl] = acc;
    __syncthreads();
    if (q == 0 && n < Nn) {
        float tot = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) tot += acc8[j][nl];
        void* dst = n < split ? out : out2;
        const int64_t i = n < split ? n : n - split;
        if (pdt == 1) reinterpret_cast<uint16_t*>(dst)[i] = f2bf(tot);   // RWKV6_BF16
        else reinterpret_cast<float*>(dst)[i] = tot;
    }
}
inline void launch_partials_reduce(const float* part, int64_t P, int64_t Nn, int pdt, void* out,
                                   void* out2, int64_t split, hipStream_t s) {
    hipLaunchKernelGGL(partials_reduce_kernel, dim3((unsigned)((Nn + 31) / 32)), dim3(PR_THR), 0, s,
                       part, P, Nn, pdt, out, out2, split);
}
}  // namespace
