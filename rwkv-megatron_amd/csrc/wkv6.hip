// WKV6 forward / backward for MI355X (gfx950), K = V = 64.
//
// Replaces fla's fused_recurrent_rwkv6 / chunk_rwkv6 as called at
// /root/reference/rwkv_megatron/rwkv6_layer_specs.py:339.  The recurrence is
//   o_t = s * r_t^T (S_{t-1} + diag(u) k_t v_t^T),   S_t = diag(exp(w_t)) S_{t-1} + k_t v_t^T.
//
// Decomposition (all deterministic):
//   wkv6_fwd_pieces  only when B*H gives fewer than 256 workgroups: per (b,h, piece of segments
//                    0..P-2), the piece's end state from a zero start and its total decay
//                    (k, v, w read once more)
//   wkv6_fwd_fold    chains the pieces from h0 into each segment's start state
//   wkv6_fwd_walk    per (b,h, segment): walks the chunks in order with the fp32 state in
//                    registers: o = (r e^{G_{t-1}}) S_in + intra-chunk attention, then
//                    S_out = e^{G_63} S_in + sum_tau (k_tau e^{G_63 - G_tau}) v_tau^T  [MFMA];
//                    writes o and the bf16 S_in of every chunk for the backward
//   wkv6_bwd_pieces  segmented backward only: per (b,h, piece of segments 1..P-1), the state
//                    gradient the piece hands to the left from a zero one, and its decay
//   wkv6_bwd_fold    chains them from dhT into each segment's starting state gradient
//   wkv6_bwd_loop    per (b,h, segment): the reverse walk, all gradients of each chunk with
//                    dS_out(c-1) = e^{G_63} dS_out(c) + s sum_t (r_t e^{G_{t-1}}) dO_t^T  [MFMA]
//                    carried in registers; dh0 and the du partials
//   chunk-parallel backward, when even the segments cannot fill the device (few, short
//   sequences):
//     wkv6_bwd_chunk_dstate  per (b,h, chunk): dS_loc and the chunk decay                [MFMA]
//     wkv6_state_scan_bwd    per (b,h, element): dS_out(c-1) = e^{G_63(c)} dS_out(c) + dS_loc(c)
//     wkv6_bwd_chunk_grads   per (b,h, chunk): dr, dk, dv, dw, du partials               [MFMA]
//   wkv6_du_reduce   per (h, channel): fixed-order sum of the du partials
//
// Inside a 64-token chunk G is the inclusive cumulative log-decay (base-2 units, so
// every exponential is one v_exp_f32) and a chunk is four 16-token sub-blocks with
// midpoints mu_I = G[16I+7].  Each chunk kernel first builds, once, the operand tiles
//   Rm[t] = r_t e^{G_{t-1} - mu_I(t)},      Km[tau] = k_tau e^{mu_J(tau) - G_tau}
// (bounded by the decay of 8 tokens either way; with w floored at W_MIN the factors stay
// inside e^{+-80}).  The intra-chunk attention is then, on bf16 MFMA,
//   I == J:  A[t][tau] = sum_i Rm[t][i] Km[tau][i]
//   I >  J:  A[t][tau] = sum_i (Rm[t][i] e^{mu_I - b_J}) (Km[tau][i] e^{b_J - mu_J}),
// b_J = G[16J+15] the end of block J: each factor spans at most 8 tokens next to a block
// boundary, so neither underflows unless the pair's own decay is already below e^-23
// (f = e^{mu_I - mu_J} as one factor spans 16+ tokens and would underflow for pairs that
// still matter).  The cross-block factors are per-channel scalars applied to operands or
// to accumulator columns, never per-element exponentials.
//
// Operands that reduce over tokens are read from the same token-major LDS tile with
// the gfx950 LDS transpose read (ds_read_b64_tr_b16), so no tile is stored twice.
// Every MFMA accumulates in fp32 and the carried states are fp32.  dw is a cancelling suffix
// sum of Rm*acc_r - Km*acc_k: its terms cancel exactly only if the epilogue multiplies the
// accumulators by the very bf16 Rm, Km the products used, so it does (single bf16 operands,
// no hi + lo split).
#include <algorithm>
#include <atomic>
#include <mutex>

#include "common.h"
#include "../../include/rwkv6_amd.h"

#define KD 64            // head size (K == V)
#define CL 64            // chunk length (tokens)
#define TS 72            // LDS row stride of a bf16 64x64 tile (elements): 144 B rows
#define GS 72            // LDS row stride of an fp32 64x64 tile (elements)
#define GSG 68           // row stride of the fp32 cumulative-decay view: 16-byte aligned rows, so a
                         // thread reads 8 consecutive values with two 16-byte loads (8 rows x 8
                         // threads of a wave hit distinct banks), and reads of rows 4 apart by 16
                         // consecutive lanes fall 16 banks apart
#define NTHR 256
#define NTHR_G 512       // threads of the gradient kernel (8 waves)
// Per-token log-decay floor.  The midpoint-referenced operand tiles scale by the decay of up
// to 8 tokens either way, which must stay inside the bf16/fp32 exponent range (8 * 10 < 88);
// a token below the floor keeps a decay factor e^-10 = 4.5e-5 instead of a smaller one
// (relative change of the state below that); its dw (d decay in the sequence-first entry) is
// 0, the derivative of the floored forward, within e^-10 of the exact one.
#define W_MIN (-10.0f)
#define FLOOR_FF 21807.29f    // e^{-W_MIN - 0.01}: Fm Fk above it marks a floored token

typedef uint16_t tile_t[CL][TS];
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ---------------------------------------------------------------------------
// operand fragments
// ---------------------------------------------------------------------------
// Fragment convention (16x16 MFMA tiles): lane = 16*q + L.  An A operand supplies
// row L, a B operand column L; the k-slot s of the operand maps to one reduction
// index, identically for both operands of a product.

// Transposed read of a token-major tile X (row stride TS): the lane receives
// X[r0 + 4q + s][c0 + L], s = 0..3 -- one column, four consecutive rows.
__device__ __forceinline__ bf16x4 ld_tr4(const uint16_t* X, int r0, int c0, int lane = threadIdx.x & 63) {
    const int L = lane & 15, q = lane >> 4;
    const uint16_t* p = X + (r0 + 4 * q + (L >> 2)) * TS + c0 + 4 * (L & 3);
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
}
// 32-row version for the 16x16x32 MFMA: slots 0-3 rows r0+4q+s, slots 4-7 rows r0+16+4q+s.
__device__ __forceinline__ bf16x8 ld_tr8(const uint16_t* X, int r0, int c0, int lane = threadIdx.x & 63) {
    const bf16x4 a = ld_tr4(X, r0, c0, lane), b = ld_tr4(X, r0 + 16, c0, lane);
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}
// Lane l receives X[r0 + s][l], s = 0..3: 16-lane row group q reads columns 16q..16q+15 of
// rows r0..r0+3 (lanes 4s..4s+3 of the group read row s), so a wave reads 4 rows x 64
// columns and each lane gets 4 consecutive rows of its own column.
__device__ __forceinline__ bf16x4 ld_col4(const uint16_t* X, int r0) {
    const int lane = threadIdx.x & 63, L = lane & 15, q = lane >> 4;
    const uint16_t* p = X + (r0 + (L >> 2)) * TS + 16 * q + 4 * (L & 3);
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
}
// Lane (q, L) receives X[r0 + 8q + s][c0 + L], s = 0..3: the 16 lanes of row group q read
// rows r0 + 8q + (0..3) (lanes 4s..4s+3 read row s as 16 consecutive columns).
__device__ __forceinline__ bf16x4 ld_tr4_g8(const uint16_t* X, int r0, int c0, int lane = threadIdx.x & 63) {
    const int L = lane & 15, q = lane >> 4;
    const uint16_t* p = X + (r0 + 8 * q + (L >> 2)) * TS + c0 + 4 * (L & 3);
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
}
// 8 consecutive rows r0 + 8q + (0..7) of column c0 + L.
__device__ __forceinline__ bf16x8 ld_tr8_g8(const uint16_t* X, int r0, int c0, int lane = threadIdx.x & 63) {
    const bf16x4 a = ld_tr4_g8(X, r0, c0, lane), b = ld_tr4_g8(X, r0 + 4, c0, lane);
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Direct read of row `row` with the slot order of ld_tr8: columns c0+4q+(0..3), c0+16+4q+(0..3).
__device__ __forceinline__ bf16x8 ld_dir8(const uint16_t* X, int row, int c0, int lane = threadIdx.x & 63) {
    const int q = lane >> 4;
    const uint2 a = *reinterpret_cast<const uint2*>(X + row * TS + c0 + 4 * q);
    const uint2 b = *reinterpret_cast<const uint2*>(X + row * TS + c0 + 16 + 4 * q);
    return __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
}
// Direct 16-byte read of row `row`, columns c0 + 8q .. +7 (products whose operands are both direct).
__device__ __forceinline__ bf16x8 ld_row8(const uint16_t* X, int row, int c0, int lane = threadIdx.x & 63) {
    const int q = lane >> 4;
    return ld_bf16x8(X + row * TS + c0 + 8 * q);
}
// Per-slot fp32 factors in ld_dir8 order from a 64-vector.
__device__ __forceinline__ void dir8_vec(const float* v, int c0, float* f, int lane = threadIdx.x & 63) {
    const int q = lane >> 4;
    const float4 a = *reinterpret_cast<const float4*>(v + c0 + 4 * q);
    const float4 b = *reinterpret_cast<const float4*>(v + c0 + 16 + 4 * q);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ void row8_vec(const float* v, int c0, float* f, int lane = threadIdx.x & 63) {
    const int q = lane >> 4;
    const float4 a = *reinterpret_cast<const float4*>(v + c0 + 8 * q);
    const float4 b = *reinterpret_cast<const float4*>(v + c0 + 8 * q + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ bf16x8 scale8(bf16x8 x, const float* f) {
    float y[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) y[s] = (float)x[s] * f[s];
    return __builtin_bit_cast(bf16x8, pack8(y));
}

// ---------------------------------------------------------------------------
// tile movement and the chunk cumulative decay
// ---------------------------------------------------------------------------

// One 16-byte piece of a token-major tile: row, columns c8 .. c8 + 7.
__device__ __forceinline__ void sstore16(uint16_t (*X)[TS], int row, int c8, uint4 v) {
    *reinterpret_cast<uint4*>(&X[row][c8]) = v;
}


// Token tensors come in two layouts:
//   head-first  [B,H,T,64]   (fla's contract)                 SEQ = false
//   seq-first   [T,B,H*64]   (the linear-layer outputs, :454-457) SEQ = true
// tok_base gives the element offset of (b*H + h, token t0); tok_rs the token stride.
template <bool SEQ>
__device__ __forceinline__ size_t tok_base(int bh, int t0, int B, int H, int T) {
    if (SEQ) {
        const int b = bh / H, h = bh - b * H;
        return (((size_t)t0 * B + b) * H + h) * KD;
    }
    return ((size_t)bh * T + t0) * KD;
}
template <bool SEQ>
__device__ __forceinline__ size_t tok_rs(int B, int H) {
    return SEQ ? (size_t)B * H * KD : (size_t)KD;
}

// Token-major LDS tile -> global (rows < nvalid, token stride rs), NT_ threads.
template <int NT_>
__device__ __forceinline__ void store_tile(uint16_t* __restrict__ dst, uint16_t (*tok)[TS],
                                           int nvalid, size_t rs = KD) {
#pragma unroll
    for (int p = 0; p < 512 / NT_; ++p) {
        int idx = p * NT_ + threadIdx.x;
        int row = idx >> 3, c8 = (idx & 7) * 8;
        if (row < nvalid)
            *reinterpret_cast<uint4*>(dst + (size_t)row * rs + c8) =
                *reinterpret_cast<const uint4*>(&tok[row][c8]);
    }
}

// Inclusive cumulative log2-decay over the 64 tokens of a chunk (token-major fp32
// Gm[t][i]) from a token-major bf16 tile, NT_ threads (NT_/64 token parts).  The tile
// holds the log-decay w, or (DEC) the pre-activation `decay` with w = -exp(decay)
// (rwkv6_layer_specs.py:336) evaluated here in fp32; w is floored at W_MIN.  Padding rows
// must read as w = 0: callers zero-fill them (DEC: the kernel masks rows >= nvalid).
// `tot` holds NT_ floats.  Ends with a barrier.
template <int NT_, bool DEC = false>
__device__ __forceinline__ void build_G(uint16_t (*Wm)[TS], float (*Gm)[GSG], float* tot,
                                        int nvalid = CL) {
    constexpr int NP = NT_ / 64, PL = CL / NP;
    const int i = threadIdx.x & 63, part = threadIdx.x >> 6;
    float loc[PL];
    float run = 0.f;
#pragma unroll
    for (int s4 = 0; s4 < PL; s4 += 4) {
        const bf16x4 x4 = ld_col4(&Wm[0][0], PL * part + s4);       // column i = lane
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int s = s4 + j;
            const float x = (float)x4[j];
            const float wn = DEC ? ((PL * part + s < nvalid) ? -ex2(x * RW_L2E) : 0.f) : x;
            run += fmaxf(wn, W_MIN) * RW_L2E;
            loc[s] = run;
        }
    }
    tot[part * 64 + i] = run;
    __syncthreads();
    float off = 0.f;                       // same order as a loop over p < part
#pragma unroll
    for (int p = 0; p < NP - 1; ++p) off += p < part ? tot[p * 64 + i] : 0.f;
#pragma unroll
    for (int s = 0; s < PL; ++s) Gm[PL * part + s][i] = loc[s] + off;
    __syncthreads();
}

// G[row][c8 .. c8+7] with two 16-byte LDS reads.
__device__ __forceinline__ void g8(const float (*Gm)[GSG], int row, int c8, float* f) {
    const float4 a = *reinterpret_cast<const float4*>(&Gm[row][c8]);
    const float4 b = *reinterpret_cast<const float4*>(&Gm[row][c8 + 4]);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
// G[row - 1][c8 .. c8+7], zero for row 0 (G before the chunk's first token).
__device__ __forceinline__ void g8m1(const float (*Gm)[GSG], int row, int c8, float* f) {
    g8(Gm, row > 0 ? row - 1 : 0, c8, f);
#pragma unroll
    for (int s = 0; s < 8; ++s) f[s] = row > 0 ? f[s] : 0.f;
}

__device__ __forceinline__ float load_u(const void* u, int u_dtype, int idx) {
    return u_dtype == RWKV6_BF16 ? bf2f(reinterpret_cast<const uint16_t*>(u)[idx])
                                 : reinterpret_cast<const float*>(u)[idx];
}

// Index of the cross-block pair (I, J), I > J, in the 6-entry tables.
__host__ __device__ constexpr int pair_index(int I, int J) { return I * (I - 1) / 2 + J; }

// ---------------------------------------------------------------------------
// forward as a walk: one workgroup per (b,h, segment) carries the fp32 state in registers
// ---------------------------------------------------------------------------
// A segment is a run of consecutive chunks of one sequence.  Per chunk the workgroup reads
// r, k, v, w once (prefetched into registers one chunk ahead), writes o and the bf16 S_in the
// backward consumes, and advances its state
//   S_out = diag(e^{G_63}) S_in + sum_tau (k_tau e^{G_63 - G_tau}) v_tau^T      [MFMA]
// in the accumulator registers.  When B*H alone gives too few workgroups for the device,
// each sequence is cut into P segments: the pre-pass pieces (wkv6_fwd_pieces) give each of
// segments 0..P-2 its local end state and total log-decay (reading k, v, w), wkv6_fwd_fold
// chains them, and each output walk starts from
//   S_start(p) = A(p-1) S_start(p-1) + S_seg(p-1),  S_start(0) = h0.
// 8 waves: wave (W, hh) owns target tokens [16W, 16W+16) x value columns [32hh, 32hh+32)
// of o, and state rows [16W, 16W+16) x columns [32hh, 32hh+32): lane (lq, lr) holds
// S[16W + lr][32hh + 16tp + 4lq + rr] in acc[tp][rr] (the products are computed transposed,
// value side as the A operand, so a lane's four values are adjacent columns of one row).
#define NTHR_W 512
#ifndef WALK_TARGET_ITEMS
#define WALK_TARGET_ITEMS 256   // workgroups a forward should offer (one per CU of an MI355X)
#endif
#define WALK_MIN_CHUNKS 8       // shortest segment worth a pre-pass
#ifndef DSTATE_TARGET_ITEMS
#define DSTATE_TARGET_ITEMS 256 // the same for the backward's walk
#endif
#ifndef WALK_WPE
#define WALK_WPE 2              // waves per SIMD the walk is compiled for (1 block of 8 waves / CU)
#endif

struct WalkSmem {
    // the small members and the decay view first: within the 16-bit offset of the LDS
    // instructions
    float emu[4][KD];                 // e^{mu_I}
    float c1[4][KD];                  // e^{mu_I - b_{I-1}}            (I >= 1)
    float c3[4][KD];                  // e^{G_63 - mu_J}
    float c6[6][KD];                  // e^{b_{I-1} - mu_J}, pair (I, J), J < I
    float dec[2][KD];                 // e^{G_63} of chunk c in dec[c & 1]
    float tot[2][NTHR_W];             // per-part log2-decay sums of chunk c in tot[c & 1]
    float bonus[CL];
    float uh[KD];                     // u of this head
    float G[(CL + 1) * GSG];          // row 0 zero (G before the chunk), row t + 1 = G_t:
                                      // cumulative log2-decay
    tile_t Rm, Km;                    // diagonal-block operands (midpoint-referenced)
    tile_t Ri, Rp;                    // r e^{G_{t-1}} (inter-chunk), r e^{G_{t-1} - b_{I-1}} (cross)
    tile_t Kt, Vm, Ot;                // state-update operand k e^{G_63 - G}, v, o staging
    tile_t Sin[2];                    // bf16 S_in of chunk c in Sin[c & 1]
    uint16_t Kc[6 * 16][TS];          // cross-block sources k e^{b_{I-1} - G}, rows 16 pair(I, J)
    tile_t Wr;                        // raw w of chunk c + 2 (scanned during chunk c)
};
static_assert(sizeof(WalkSmem) <= 160 * 1024, "walk block LDS");

// The decay scan of the output walk runs two chunks ahead, in two halves, so that it shares the
// products' phase of an earlier chunk instead of adding barriers of its own:
//   walk_scan1(c')  (512 threads, part = 8-token run): thread (part, i) scans channel i over
//                   tokens 8 part .. 8 part + 7 of the raw w in Wr, keeps the running sums in
//                   loc and writes the part's total to tot[c' & 1];
//   walk_scan2(c')  one barrier later: the part-end values ge[p] = G[8p + 7] from tot[c' & 1],
//                   the cumulative-decay view G of chunk c' and its per-channel tables (mu_I =
//                   ge[2I], b_{I-1} = ge[2I - 1], G_63 = ge[7]).
// `part` is wave-uniform, so the table branches are scalar.
template <bool DEC, int PB>
__device__ __forceinline__ void walk_scan1(WalkSmem& sm, int nvalid, int tpar, float* loc) {
    // the wave's 8-token part is 2 PB + hh (PB the wave pair, compile-time; hh wave-uniform)
    const int i = threadIdx.x & 63, hh = (threadIdx.x >> 6) & 1, part = 2 * PB + hh;
    float run = 0.f;
#pragma unroll
    for (int s4 = 0; s4 < 8; s4 += 4) {
        const bf16x4 x4 = ld_col4(&sm.Wr[0][0], 8 * part + s4);   // column i = lane
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int s = s4 + j;
            const float x = (float)x4[j];
            const float wn = DEC ? ((8 * part + s < nvalid) ? -ex2(x * RW_L2E) : 0.f) : x;
            run += fmaxf(wn, W_MIN) * RW_L2E;
            loc[s] = run;
        }
    }
    sm.tot[tpar][part * 64 + i] = run;
}
template <int PB>
__device__ __forceinline__ void walk_scan2(WalkSmem& sm, const float* loc, int tpar, int cpar) {
    float (*Gm)[GSG] = reinterpret_cast<float (*)[GSG]>(sm.G + GSG);
    const int i = threadIdx.x & 63, hh = (threadIdx.x >> 6) & 1, part = 2 * PB + hh;
    float ge[8], a = 0.f;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        a += sm.tot[tpar][p * 64 + i];
        ge[p] = a;
    }
    // G before the part: the sum of parts 0 .. part-1
    const float off = hh ? ge[2 * PB] : (PB > 0 ? ge[2 * PB - 1] : 0.f);
#pragma unroll
    for (int s = 0; s < 8; ++s) Gm[8 * part + s][i] = loc[s] + off;
    if constexpr (PB < 2) {
        // parts 0..3: emu, c3 of block `part`, and the c6 pairs (1,0), (2,0), (2,1), (3,0)
        const float mu = hh ? ge[4 * PB + 2] : ge[4 * PB];
        sm.emu[part][i] = ex2(mu);
        sm.c3[part][i] = ex2(ge[7] - mu);
        const float b = PB == 0 ? (hh ? ge[3] : ge[1]) : (hh ? ge[5] : ge[3]);
        const float mj = PB == 0 ? ge[0] : (hh ? ge[0] : ge[2]);
        sm.c6[part][i] = ex2(b - mj);
    } else if constexpr (PB == 2) {
        // parts 4, 5: c1 of blocks I = 1, 2 and the c6 pairs (3,1), (3,2)
        const float mu = hh ? ge[4] : ge[2];
        const float bp = hh ? ge[3] : ge[1];
        sm.c1[1 + hh][i] = ex2(mu - bp);
        sm.c6[part][i] = ex2(ge[5] - (hh ? ge[4] : ge[2]));
    } else {
        // part 6: c1 of block 3; part 7: the chunk decay
        if (hh == 0) {
            sm.c1[3][i] = ex2(ge[6] - ge[5]);
        } else {
            sm.dec[cpar][i] = ex2(ge[7]);
        }
    }
}

// Segments per sequence (shared by the workspace query and the launch): as many (b,h, segment)
// workgroups as fit `target` (one walk per CU) without a second round, no segment shorter
// than WALK_MIN_CHUNKS.  (Rounding up instead, e.g. 3 segments for 96 sequences, put the 288
// walks into two rounds: 30 % slower at B*H = 96, T = 4096.)
inline int walk_segments(int64_t BH, int64_t NT, int64_t target = WALK_TARGET_ITEMS) {
    if (NT <= 0) return 1;
    int64_t P = target / BH > 1 ? target / BH : 1;
    P = std::min<int64_t>(P, std::max<int64_t>(1, NT / WALK_MIN_CHUNKS));
    const int64_t NC = (NT + P - 1) / P;               // chunks per segment
    return (int)((NT + NC - 1) / NC);                   // no empty segment
}

// Pieces of the forward pre-pass (wkv6_fwd_pieces): each of the P-1 earlier segments of a
// sequence is cut into `sub` pieces of at most `ncs` chunks, `sub` the nearest integer to
// PIECE_TARGET / (B*H*(P-1)) (about one piece per CU: with most CUs busy the pre-pass is bound
// by HBM reads, and more, shorter pieces only add states to fold), no piece shorter than
// PIECE_MIN_CHUNKS, and at most max_pieces pieces in all (the workspace they fill).
#ifndef PIECE_TARGET
#define PIECE_TARGET 256
#endif
#define PIECE_MIN_CHUNKS 4
struct Pieces {
    int sub, ncs;
};
inline Pieces prepass_pieces(int64_t BH, int64_t NT, int P, int64_t max_pieces) {
    if (P <= 1 || NT <= 0) return {1, 1};
    const int64_t NC = (NT + P - 1) / P, segs = BH * (P - 1);
    int64_t sub = (2 * PIECE_TARGET + segs) / (2 * segs);          // nearest
    sub = std::max<int64_t>(sub, 1);
    sub = std::min<int64_t>(sub, std::max<int64_t>(1, NC / PIECE_MIN_CHUNKS));
    sub = std::min<int64_t>(sub, std::max<int64_t>(1, max_pieces / segs));
    const int64_t ncs = (NC + sub - 1) / sub;
    return {(int)((NC + ncs - 1) / ncs), (int)ncs};      // no empty piece, sub only shrinks
}

// The backward walks each sequence in one workgroup (wkv6_bwd_loop) when there is one segment;
// with fewer sequences, each is cut into segments like the forward's as long as the (b,h,
// segment) workgroups fill at least 7/8 of the device (a segment walks at ~6 us a chunk
// whatever the occupancy).  Otherwise (few, short segments) the state gradients run
// chunk-parallel.  Returns the segment count of the walk, or 0 for the chunk-parallel form.
inline int bwd_walk_segments(int64_t BH, int64_t NT) {
    const int P = walk_segments(BH, NT, DSTATE_TARGET_ITEMS);
    return (P == 1 || 8 * BH * P >= 7 * DSTATE_TARGET_ITEMS) ? P : 0;
}

struct WalkPrefetch {
    uint4 r, k, v, w;
};

// Rows >= nvalid (>= 1) read row nvalid-1 and return zero: no branch around the load.
__device__ __forceinline__ uint4 gload16c(const uint16_t* __restrict__ src, int row, int c8,
                                          int nvalid, size_t rs) {
    const uint4 x = *reinterpret_cast<const uint4*>(src + (size_t)min(row, nvalid - 1) * rs + c8);
    return row < nvalid ? x : make_uint4(0u, 0u, 0u, 0u);
}

// Raw w of chunk cw for the thread's piece (token row tid >> 3, channels 8 (tid & 7) ..).
template <bool SEQ>
__device__ __forceinline__ uint4 walk_load_w(const uint16_t* __restrict__ w, int bh, int cw, int B,
                                             int H, int T) {
    const int t0 = cw * CL, nvalid = min(CL, T - t0);
    const int row = min((int)(threadIdx.x >> 3), nvalid - 1), c8 = (threadIdx.x & 7) * 8;
    return *reinterpret_cast<const uint4*>(w + tok_base<SEQ>(bh, t0, B, H, T) +
                                           (size_t)row * tok_rs<SEQ>(B, H) + c8);
}

// r, k, v of chunk c and w of chunk cw (the decay scan runs two chunks ahead of the rest).
template <bool SEQ>
__device__ __forceinline__ void walk_issue(WalkPrefetch& f, const uint16_t* __restrict__ r,
                                           const uint16_t* __restrict__ k,
                                           const uint16_t* __restrict__ v,
                                           const uint16_t* __restrict__ w, int bh, int c, int cw,
                                           int B, int H, int T) {
    const size_t rs = tok_rs<SEQ>(B, H);
    // unconditional loads (rows past the end read the last token; the walk zeroes those
    // rows before they reach LDS): a load under a branch makes the next wait a full one
    const int c8 = (threadIdx.x & 7) * 8;
    {
        const int t0 = c * CL, nvalid = min(CL, T - t0);
        const int row = min((int)(threadIdx.x >> 3), nvalid - 1);
        const size_t off = tok_base<SEQ>(bh, t0, B, H, T) + (size_t)row * rs + c8;
        f.r = *reinterpret_cast<const uint4*>(r + off);
        f.k = *reinterpret_cast<const uint4*>(k + off);
        f.v = *reinterpret_cast<const uint4*>(v + off);
    }
    f.w = walk_load_w<SEQ>(w, bh, cw, B, H, T);
}

// Global stores of chunk c (o from Ot, S_in from Sin[c & 1]).  Issued one
// chunk late, before the next prefetch: the wait for a prefetch then never waits on a store.
__device__ __forceinline__ void walk_store(const WalkSmem& sm, uint16_t* __restrict__ o,
                                           uint16_t* __restrict__ Hs, int bh, int c, int T,
                                           int NT) {
    const int row = threadIdx.x >> 3, c8 = (threadIdx.x & 7) * 8;
    const int t0 = c * CL, nvalid = min(CL, T - t0);
    // unconditional (a store under a branch costs the loop a full wait): rows past the end
    // store the last token's own values again
    const int ro = min(row, nvalid - 1);
    // streaming stores (o and the states are read back only by later kernels): 1 % off the
    // walk and 8 us off the next call's pre-pass at config 5
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, *reinterpret_cast<const uint4*>(&sm.Ot[ro][c8])),
                                reinterpret_cast<u32x4_t*>(o + ((size_t)bh * T + t0 + ro) * KD + c8));
    __builtin_nontemporal_store(
        __builtin_bit_cast(u32x4_t, *reinterpret_cast<const uint4*>(&sm.Sin[c & 1][row][c8])),
        reinterpret_cast<u32x4_t*>(Hs + ((size_t)bh * (NT + 1) + c) * KD * KD + row * KD + c8));
}

// The chunk loop of one wave of wkv6_fwd_walk.  Wave wv works on token block I = wv >> 1 of
// the operand tiles and, in the products, on token block W = (0, 0, 1, 1, 3, 3, 2, 2)[wv]:
// both are compile-time here (PB = wv >> 1), so the cross-block loops, the table choices and
// their offsets are resolved statically; all four instantiations pass the same barriers.
template <bool SEQ, int PB>
__device__ __forceinline__ void fwd_walk_chunks(
        WalkSmem& sm, const uint16_t* __restrict__ r, const uint16_t* __restrict__ k,
        const uint16_t* __restrict__ v, const uint16_t* __restrict__ w,
        uint16_t* __restrict__ o, uint16_t* __restrict__ Hs, float scale, int B, int H, int T,
        int NT, int bh, int c_begin, int c_end, int hh, WalkPrefetch& nx, f32x4* acc) {
    constexpr int I = PB;                          // token block of the thread's tile pieces
    constexpr int W = PB < 2 ? PB : 5 - PB;        // token block of the wave's products
    float (*Gm)[GSG] = reinterpret_cast<float (*)[GSG]>(sm.G + GSG);   // Gm[-1] is the zero row
    const int lane = threadIdx.x & 63;
    const int lr = lane & 15, lq = lane >> 4;
    const int row = threadIdx.x >> 3, c8 = (threadIdx.x & 7) * 8;
    // u at the thread's 8 channels, for the bonus of every chunk (constant over the walk)
    float uf[8];
    {
        const float4 ua = *reinterpret_cast<const float4*>(&sm.uh[c8]);
        const float4 ub = *reinterpret_cast<const float4*>(&sm.uh[c8 + 4]);
        uf[0] = ua.x; uf[1] = ua.y; uf[2] = ua.z; uf[3] = ua.w;
        uf[4] = ub.x; uf[5] = ub.y; uf[6] = ub.z; uf[7] = ub.w;
    }
    if (c_begin >= c_end) return;                      // (uniform over the workgroup)
    // The decay scans of the first two chunks (the loop scans chunk c + 2 during chunk c):
    // G and the tables of c_begin, the part sums of c_begin + 1 (tot, loc).  nx holds w of
    // c_begin on entry and w of c_begin + 2 on leaving.
    float loc[8];
    {
        const uint4 w1 = walk_load_w<SEQ>(w, bh, min(c_begin + 1, c_end - 1), B, H, T);
        const uint4 w2 = walk_load_w<SEQ>(w, bh, min(c_begin + 2, c_end - 1), B, H, T);
        int nv = min(CL, T - c_begin * CL);
        sstore16(sm.Wr, row, c8, row < nv ? nx.w : make_uint4(0u, 0u, 0u, 0u));
        __syncthreads();
        walk_scan1<SEQ, PB>(sm, nv, c_begin & 1, loc);
        __syncthreads();
        walk_scan2<PB>(sm, loc, c_begin & 1, c_begin & 1);
        nv = min(CL, T - min(c_begin + 1, c_end - 1) * CL);
        sstore16(sm.Wr, row, c8, row < nv ? w1 : make_uint4(0u, 0u, 0u, 0u));
        __syncthreads();
        walk_scan1<SEQ, PB>(sm, nv, (c_begin + 1) & 1, loc);
        __syncthreads();
        nx.w = w2;
    }
    // first chunk's loads complete here (vmcnt(0)), so the wait at the loop top is set by the
    // loop's own order (the next chunk's loads, then this chunk's two stores) alone
    __builtin_amdgcn_s_waitcnt(0x0F70);
    for (int c = c_begin; c < c_end; ++c) {
        const int nvalid = min(CL, T - c * CL);
        // nx holds r, k, v of chunk c and w of chunk cw = c + 2 (the last chunk of the segment
        // past its end: that scan is never used)
        const int nvw = min(CL, T - min(c + 2, c_end - 1) * CL);
        // Every tile written here was last read before the previous chunk's final barrier
        // (Sin[c & 1] two chunks ago); G and the tables of chunk c were written in the previous
        // chunk's second phase.  The thread's raw r and k stay in registers (rq, kq) for its
        // own operand tiles below.
        // Only a sequence's last chunk can be ragged: a wave-uniform branch around the per-lane
        // zeroing (the empty asm keeps the compiler from turning it into selects on every chunk)
        if (nvalid < CL) {
            asm volatile("");
            if (row >= nvalid) nx.r = nx.k = nx.v = make_uint4(0u, 0u, 0u, 0u);
        }
        if (nvw < CL) {
            asm volatile("");
            if (row >= nvw) nx.w = make_uint4(0u, 0u, 0u, 0u);
        }
        sstore16(sm.Vm, row, c8, nx.v);
        sstore16(sm.Wr, row, c8, nx.w);                       // scanned after the barrier
        const uint4 rq = nx.r, kq = nx.k;
        {
            float rf[8], kf[8], bsum = 0.f;
            unpack8(nx.r, rf);
            unpack8(nx.k, kf);
#pragma unroll
            for (int s = 0; s < 8; ++s) bsum += rf[s] * uf[s] * kf[s];
            bsum = sum8lanes(bsum);
            if ((threadIdx.x & 7) == 0) sm.bonus[row] = bsum;
            // S_in of this chunk, bf16, for the inter-chunk product and the backward: the lane's
            // four values of a state row are adjacent, one 8-byte write per 16 columns
#pragma unroll
            for (int tp = 0; tp < 2; ++tp)
                *reinterpret_cast<uint2*>(&sm.Sin[c & 1][16 * W + lr][32 * hh + 16 * tp + 4 * lq]) =
                    make_uint2(pk2(acc[tp][0], acc[tp][1]), pk2(acc[tp][2], acc[tp][3]));
        }
        // unconditional (the last iterations reload the segment's last chunk): loads under a
        // branch would cost the loop a full wait
        walk_issue<SEQ>(nx, r, k, v, w, bh, min(c + 1, c_end - 1), min(c + 3, c_end - 1), B, H, T);
        {
            // Operand tiles of this thread's piece (token t = row in block I; I is
            // wave-uniform).  Two exponentials per element; every other factor is a
            // per-(block, channel) table entry <= 1 applied to the fp32 value:
            //   Rm = r e^{G_{t-1} - mu_I}     Ri = Rm e^{mu_I}          Rp = Rm e^{mu_I - b_{I-1}}
            //   Km = k e^{mu_I - G_t}         Kt = Km e^{G_63 - mu_I}   Kc(I2) = Km e^{b_{I2-1} - mu_I}
            float rf[8], kf[8], rm[8], km[8], y[8], f[8];
            unpack8(rq, rf);
            unpack8(kq, kf);
            float gm[8], gg[8], gp[8];
            g8(Gm, 16 * I + 7, c8, gm);
            g8(Gm, row, c8, gg);
            g8(Gm, row - 1, c8, gp);                           // the zero row for row 0
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                rm[s] = rf[s] * ex2(gp[s] - gm[s]);
                km[s] = kf[s] * ex2(gm[s] - gg[s]);
            }
            sstore16(sm.Rm, row, c8, pack8(rm));
            sstore16(sm.Km, row, c8, pack8(km));
            auto tab8 = [&](const float* tb) {
                const float4 a = *reinterpret_cast<const float4*>(tb + c8);
                const float4 b = *reinterpret_cast<const float4*>(tb + c8 + 4);
                f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
            };
            tab8(sm.emu[I]);
#pragma unroll
            for (int s = 0; s < 8; ++s) y[s] = rm[s] * f[s];
            sstore16(sm.Ri, row, c8, pack8(y));
            if constexpr (I > 0) {
                tab8(sm.c1[I]);
#pragma unroll
                for (int s = 0; s < 8; ++s) y[s] = rm[s] * f[s];
                sstore16(sm.Rp, row, c8, pack8(y));
            }
            tab8(sm.c3[I]);
#pragma unroll
            for (int s = 0; s < 8; ++s) y[s] = km[s] * f[s];
            sstore16(sm.Kt, row, c8, pack8(y));
#pragma unroll
            for (int I2 = I + 1; I2 < 4; ++I2) {
                const int pi = pair_index(I2, I);
                tab8(sm.c6[pi]);
#pragma unroll
                for (int s = 0; s < 8; ++s) y[s] = km[s] * f[s];
                sstore16(reinterpret_cast<uint16_t (*)[TS]>(sm.Kc[16 * pi]), row & 15, c8, pack8(y));
            }
        }
        __syncthreads();
        bf16x4 vt[4][2];
        {
            const int t = 16 * W + lr;
            // o transposed: every product takes the value side as its A operand and the token
            // side as its B operand, so lane (lq, lr) ends up with o[t = 16W + lr][j0 + 4 lq +
            // rr], four adjacent columns of one token (one 8-byte write into Ot).  The 16x16x32
            // and the 16x16x16 products go to separate accumulators (ao, ab).
            f32x4 ao[2] = {}, ab[2] = {};
            // V^T operands of the wave's 32 columns, token block J in vt[J]: the products below
            // take the blocks they need, and the state update takes all four (ld_tr8 is two
            // ld_tr4 of consecutive blocks), so each is read from LDS once
#pragma unroll
            for (int J = 0; J < 4; ++J)
#pragma unroll
                for (int tp = 0; tp < 2; ++tp) vt[J][tp] = ld_tr4(&sm.Vm[0][0], 16 * J, 32 * hh + 16 * tp);
            // inter-chunk: (r e^{G_{t-1}}) S_in
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const bf16x8 b = ld_dir8(&sm.Ri[0][0], t, 32 * ks);
#pragma unroll
                for (int tp = 0; tp < 2; ++tp)
                    ao[tp] = mfma32(ld_tr8(&sm.Sin[c & 1][0][0], 32 * ks, 32 * hh + 16 * tp), b, ao[tp]);
            }
            // diagonal block: strictly causal part plus the u-bonus diagonal
            {
                f32x4 at = {};
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    at = mfma32(ld_row8(&sm.Km[0][0], 16 * W + lr, 32 * ks), ld_row8(&sm.Rm[0][0], t, 32 * ks), at);
                float xa[4];
                const float bon = sm.bonus[t];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int tl = 4 * lq + rr;
                    xa[rr] = tl < lr ? at[rr] : (tl == lr ? bon : 0.f);
                }
                const bf16x4 aop = cvt4(xa[0], xa[1], xa[2], xa[3]);
#pragma unroll
                for (int tp = 0; tp < 2; ++tp) ab[tp] = mfma16(vt[W][tp], aop, ab[tp]);
            }
            // earlier blocks J < W, both operands referenced at b_{W-1}
#pragma unroll
            for (int J = 0; J < W; ++J) {
                f32x4 at = {};
                const int pr = 16 * pair_index(W, J) + lr;
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    at = mfma32(ld_row8(&sm.Kc[0][0], pr, 32 * ks), ld_row8(&sm.Rp[0][0], t, 32 * ks), at);
                const bf16x4 aop = cvt4(at[0], at[1], at[2], at[3]);
#pragma unroll
                for (int tp = 0; tp < 2; ++tp) ab[tp] = mfma16(vt[J][tp], aop, ab[tp]);
            }
#pragma unroll
            for (int tp = 0; tp < 2; ++tp) {
                float y[4];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) y[rr] = scale * (ao[tp][rr] + ab[tp][rr]);
                *reinterpret_cast<uint2*>(&sm.Ot[t][32 * hh + 16 * tp + 4 * lq]) =
                    make_uint2(pk2(y[0], y[1]), pk2(y[2], y[3]));
            }
        }
        // state update: S = diag(e^{G_63}) S + Kt^T V, computed transposed like o (V^T as the A
        // operand): lane (lq, lr) holds S[16W + lr][j0 + 4 lq + rr], so its row factor is one
        {
            const float d = sm.dec[c & 1][16 * W + lr];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                acc[0][rr] *= d;
                acc[1][rr] *= d;
            }
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 b = ld_tr8(&sm.Kt[0][0], 32 * ks, 16 * W);
#pragma unroll
            for (int tp = 0; tp < 2; ++tp)
                acc[tp] = mfma32(__builtin_shufflevector(vt[2 * ks][tp], vt[2 * ks + 1][tp], 0, 1, 2, 3, 4, 5, 6, 7),
                                 b, acc[tp]);
        }
        // the decay scans ahead: G and the tables of chunk c + 1 from the part sums made during
        // chunk c - 1, then the part sums of chunk c + 2 (in Wr since this chunk's first phase)
        walk_scan2<PB>(sm, loc, (c + 1) & 1, (c + 1) & 1);
        walk_scan1<SEQ, PB>(sm, nvw, c & 1, loc);
        __syncthreads();
        // o and S_in of this chunk, stored after the next chunk's loads were issued: the wait
        // for those at the top of the next iteration leaves these stores in flight (vmcnt
        // counts loads and stores in issue order)
        walk_store(sm, o, Hs, bh, c, T, NT);
    }

}

// Output walk over segment blockIdx.x % P of sequence blockIdx.x / P.  Segment 0 starts from
// h0 (or zero), segment p >= 1 from Sstart[b,h][p-1] (wkv6_fwd_fold).
// SEQ: r, k, v and the pre-activation decay are sequence-first; o is always head-first.
template <bool SEQ>
__global__ void __launch_bounds__(NTHR_W) __attribute__((amdgpu_waves_per_eu(WALK_WPE)))
wkv6_fwd_walk(const uint16_t* __restrict__ r, const uint16_t* __restrict__ k,
              const uint16_t* __restrict__ v, const uint16_t* __restrict__ w,
              const void* __restrict__ u, int u_dtype, const float* __restrict__ h0,
              uint16_t* __restrict__ o, uint16_t* __restrict__ Hs, float* __restrict__ hT,
              const float* __restrict__ Sstart, float scale, int B, int H, int T, int NT, int P) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
    WalkSmem& sm = *reinterpret_cast<WalkSmem*>(smem_raw);
    const int bh = blockIdx.x / P, seg = blockIdx.x - bh * P, h = bh % H;
    const int NC = (NT + P - 1) / P;
    const int c_begin = seg * NC, c_end = min(NT, c_begin + NC);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    // waves 0-3 take token blocks 0,0,1,1 and waves 4-7 blocks 3,3,2,2: with waves dealt
    // round-robin to the 4 SIMDs, each SIMD gets blocks {0,3} or {1,2}, whose cross-block
    // work (W products each) sums to the same 3
    const int W = wv < 4 ? (wv >> 1) : 5 - (wv >> 1), hh = wv & 1;
    const int lr = lane & 15, lq = lane >> 4;
    const size_t sbase = (size_t)bh * KD * KD;

    WalkPrefetch nx;
    if (c_begin < c_end) walk_issue<SEQ>(nx, r, k, v, w, bh, c_begin, c_begin, B, H, T);

    // ---- starting state ----
    f32x4 acc[2];
    {
        const float* s0 = seg > 0 ? Sstart + ((size_t)bh * (P - 1) + seg - 1) * KD * KD
                                  : (h0 ? h0 + sbase : nullptr);
        // one branch around all eight loads (a conditional per element came out ~1 % slower
        // over the whole walk: the register assignment of the loop differed)
        if (s0) {
#pragma unroll
            for (int tp = 0; tp < 2; ++tp) {
                const float4 x = *reinterpret_cast<const float4*>(
                    s0 + (16 * W + lr) * KD + 32 * hh + 16 * tp + 4 * lq);
                acc[tp][0] = x.x; acc[tp][1] = x.y; acc[tp][2] = x.z; acc[tp][3] = x.w;
            }
        } else {
#pragma unroll
            for (int tp = 0; tp < 2; ++tp)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) acc[tp][rr] = 0.f;
        }
        if (threadIdx.x < KD) sm.uh[threadIdx.x] = load_u(u, u_dtype, h * KD + threadIdx.x);
        if (threadIdx.x < GSG) sm.G[threadIdx.x] = 0.f;       // G before the chunk: 0
        __syncthreads();
    }

    switch (__builtin_amdgcn_readfirstlane(wv >> 1)) {
    case 0:
        fwd_walk_chunks<SEQ, 0>(sm, r, k, v, w, o, Hs, scale, B, H, T, NT, bh, c_begin, c_end, hh, nx, acc);
        break;
    case 1:
        fwd_walk_chunks<SEQ, 1>(sm, r, k, v, w, o, Hs, scale, B, H, T, NT, bh, c_begin, c_end, hh, nx, acc);
        break;
    case 2:
        fwd_walk_chunks<SEQ, 2>(sm, r, k, v, w, o, Hs, scale, B, H, T, NT, bh, c_begin, c_end, hh, nx, acc);
        break;
    default:
        fwd_walk_chunks<SEQ, 3>(sm, r, k, v, w, o, Hs, scale, B, H, T, NT, bh, c_begin, c_end, hh, nx, acc);
        break;
    }

    // ---- end of the sequence: the final state ----
    if (seg == P - 1) {
#pragma unroll
        for (int tp = 0; tp < 2; ++tp) {
            const size_t e = (size_t)(16 * W + lr) * KD + 32 * hh + 16 * tp + 4 * lq;
            *reinterpret_cast<uint2*>(Hs + (size_t)bh * (NT + 1) * KD * KD + (size_t)NT * KD * KD + e) =
                make_uint2(pk2(acc[tp][0], acc[tp][1]), pk2(acc[tp][2], acc[tp][3]));
            if (hT)
                *reinterpret_cast<float4*>(hT + sbase + e) =
                    make_float4(acc[tp][0], acc[tp][1], acc[tp][2], acc[tp][3]);
        }
    }
}

// ---------------------------------------------------------------------------
// forward pre-pass: the end states of runs of chunks ("pieces")
// ---------------------------------------------------------------------------
// Segment p of the output walk starts from the state entering its first chunk.  Each of the
// segments 0..P-2 is cut into SUB pieces of at most NCS chunks; one workgroup per (b,h, piece)
// walks its chunks from a zero state, two chunks (PSPAN = 128 tokens) per step,
//   S = diag(e^{G_end}) S + sum_tau (k_tau e^{G_end - G_tau}) v_tau^T        [MFMA]
// with G the cumulative log-decay over the step, and writes the piece's end state S_q (fp32
// [64][64]) and total log2-decay A_q ([64]).  Only k, v and w are read.  Per step, thread
// (part, i) scans the log-decay of channel i over the tokens 16 part .. 16 part + 15 and forms
// those tokens' k e^{G_end - G} itself, written channel-major (two 16-byte stores) as the
// MFMA's A operand: no cumulative-decay tile.  The raw tiles are double-buffered, so a step
// takes two barriers (piece_steps: the next step's scan runs beside this step's state
// update; four before, 78.4 -> 76.8 us at config 5).  The exponents G_end - G_tau are never
// positive, whatever the step's length, so the end state needs none of the walk's 64-token
// references; 128-token steps halve the barriers per token (86.7 against 89.2 us at config 5
// with one 64-token chunk per step; loads two steps ahead measured no faster, and a plain
// read stream of the same shape, one workgroup per CU, takes 59 us).  With 132 KB of LDS a
// piece takes a CU to itself; prepass_pieces caps the pieces at one per CU.
#define PSPAN (2 * CL)     // tokens per step of the pre-pass pieces
#define PETS (PSPAN + 8)   // row stride of the channel-major operand tile (elements)
typedef uint16_t ptile_t[PSPAN][TS];
struct PieceSmem {
    float dec[KD];                    // e^{G_end} of the step
    float tot[2][NTHR_W];             // per-part log2-decay sums of step s in tot[s & 1]
    ptile_t Xm[2], Wt[2], Ym[2];      // the raw tiles of step s in [s & 1] (token-major): k, w,
                                      // v forward; r, w, dO backward
    uint16_t Et[KD][PETS];            // the A operand, channel-major: k e^{G_end - G}
                                      // forward, r e^{G_{t-1}} backward
};
static_assert(sizeof(PieceSmem) <= 160 * 1024, "piece block LDS");

// A step of a pre-pass piece is three parts on raw tiles in LDS (nvalid tokens; the rows past
// them zeroed), spread over two barriers so that the decay scan of the next step shares the
// state update's phase:
//   piece_scan   thread (part, i) scans the log-decay of channel i over the tokens 16 part ..
//                16 part + 15 (running sums kept in loc, the part's total in tot);
//   piece_ebuild one barrier later: G = loc + the earlier parts' totals, the A operand
//                k e^{G_end - G} (forward) or r e^{G_{t-1}} (backward, the exclusive prefix),
//                written channel-major, and the step's decay e^{G_end};
//   piece_update one barrier later: acc = diag(e^{G_end}) acc + E^T Y   (Y = v forward, dO
//                backward).
template <bool SEQ>
__device__ __forceinline__ void piece_scan(PieceSmem& sm, int b, int nvalid, float* loc) {
    const int i = threadIdx.x & 63, part = threadIdx.x >> 6;
    float run = 0.f;
#pragma unroll
    for (int s4 = 0; s4 < 16; s4 += 4) {
        const bf16x4 x4 = ld_col4(&sm.Wt[b][0][0], 16 * part + s4);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int s = s4 + jj;
            const float x = (float)x4[jj];
            const float wn = SEQ ? ((16 * part + s < nvalid) ? -ex2(x * RW_L2E) : 0.f) : x;
            run += fmaxf(wn, W_MIN) * RW_L2E;
            loc[s] = run;
        }
    }
    sm.tot[b][part * 64 + i] = run;
}
template <bool BWD>
__device__ __forceinline__ void piece_ebuild(PieceSmem& sm, int b, const float* loc, float& gsum) {
    const int i = threadIdx.x & 63, part = threadIdx.x >> 6;
    bf16x4 xa[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) xa[s4] = ld_col4(&sm.Xm[b][0][0], 16 * part + 4 * s4);
    // G_t = loc + (sum of the earlier parts); G_end = run_7 + sum of parts 0..6
    float off = 0.f, o7 = 0.f;
#pragma unroll
    for (int p = 0; p < 7; ++p) {
        const float t = sm.tot[b][p * 64 + i];
        off += p < part ? t : 0.f;
        o7 += t;
    }
    const float gend = sm.tot[b][7 * 64 + i] + o7;
    float e[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const float xf = (float)xa[s >> 2][s & 3];
        e[s] = BWD ? xf * ex2(s == 0 ? off : loc[s - 1] + off) : xf * ex2(gend - (loc[s] + off));
    }
    *reinterpret_cast<uint4*>(&sm.Et[i][16 * part]) = pack8(e);
    *reinterpret_cast<uint4*>(&sm.Et[i][16 * part + 8]) = pack8(e + 8);
    if (part == 7) {
        sm.dec[i] = ex2(gend);
        gsum += gend;
    }
}
__device__ __forceinline__ void piece_update(PieceSmem& sm, int b, f32x4* acc) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int W = wv >> 1, hh = wv & 1;   // state rows [16W, +16) x columns [32hh, +32)
    const int lr = lane & 15, lq = lane >> 4;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const float d = sm.dec[16 * W + 4 * lq + rr];
        acc[0][rr] *= d;
        acc[1][rr] *= d;
    }
#pragma unroll
    for (int ks = 0; ks < PSPAN / 32; ++ks) {
        // A: row 16W + lr of Et in the slot order of ld_tr8 (tokens 32ks + 4lq + (0..3) and
        // 32ks + 16 + 4lq + (0..3)), B: the same tokens of Y
        const uint2 a0 = *reinterpret_cast<const uint2*>(&sm.Et[16 * W + lr][32 * ks + 4 * lq]);
        const uint2 a1 = *reinterpret_cast<const uint2*>(&sm.Et[16 * W + lr][32 * ks + 16 + 4 * lq]);
        const bf16x8 a = __builtin_bit_cast(bf16x8, make_uint4(a0.x, a0.y, a1.x, a1.y));
#pragma unroll
        for (int tp = 0; tp < 2; ++tp)
            acc[tp] = mfma32(a, ld_tr8(&sm.Ym[b][0][0], 32 * ks, 32 * hh + 16 * tp), acc[tp]);
    }
}

// The raw 16-byte pieces a thread stores per step: rows (tid >> 3) and (tid >> 3) + 64 of each
// of three tensors (rows past the valid ones read the last valid token and are zeroed before
// the store: unconditional loads).
struct PieceLoads {
    uint4 x[2], w[2], y[2];
};
__device__ __forceinline__ void piece_store(PieceSmem& sm, int b, PieceLoads& f, int nvalid) {
    const int row = threadIdx.x >> 3, c8 = (threadIdx.x & 7) * 8;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (row + 64 * h >= nvalid) f.x[h] = f.w[h] = f.y[h] = make_uint4(0u, 0u, 0u, 0u);
        *reinterpret_cast<uint4*>(&sm.Ym[b][row + 64 * h][c8]) = f.y[h];
        *reinterpret_cast<uint4*>(&sm.Wt[b][row + 64 * h][c8]) = f.w[h];
        *reinterpret_cast<uint4*>(&sm.Xm[b][row + 64 * h][c8]) = f.x[h];
    }
}

// The steps of a piece in the order `step(s)` gives (s = 0 .. nsteps-1; the backward walks its
// steps from the last), two barriers a step: the raw tiles of step s + 1 go into the other
// buffer and the A operand of step s is built (its scan done during step s - 1); then the
// state update of step s and the scan of step s + 1.  `issue(m)` loads step m into nx and
// `nvalid(m)` counts its tokens.  Past the last step the indices stay on it (unconditional
// loads and stores; the extra scan is never used).
template <bool SEQ, bool BWD, class Issue, class Nvalid>
__device__ __forceinline__ void piece_steps(PieceSmem& sm, PieceLoads& nx, int nsteps, Issue issue,
                                            Nvalid nvalid, f32x4* acc, float& gsum) {
    auto step = [&](int s) { return BWD ? nsteps - 1 - min(s, nsteps - 1) : min(s, nsteps - 1); };
    float loc[16];
    issue(step(0));
    piece_store(sm, 0, nx, nvalid(step(0)));
    issue(step(1));
    __syncthreads();
    piece_scan<SEQ>(sm, 0, nvalid(step(0)), loc);
    __syncthreads();
    for (int s = 0; s < nsteps; ++s) {
        const int b = s & 1, nv1 = nvalid(step(s + 1));
        piece_store(sm, b ^ 1, nx, nv1);
        issue(step(s + 2));
        piece_ebuild<BWD>(sm, b, loc, gsum);
        __syncthreads();
        piece_update(sm, b, acc);
        piece_scan<SEQ>(sm, b ^ 1, nv1, loc);
        __syncthreads();
    }
}

template <bool SEQ>
__global__ void __launch_bounds__(NTHR_W)
wkv6_fwd_pieces(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                const uint16_t* __restrict__ w, float* __restrict__ Sseg, float* __restrict__ Aseg,
                int B, int H, int T, int NT, int NC, int SUB, int NCS, int npieces) {
    __shared__ __attribute__((aligned(16))) PieceSmem sm;
    const int bh = blockIdx.x / npieces, q = blockIdx.x - bh * npieces;
    const int sg = q / SUB, j = q - sg * SUB;
    // never empty: SUB = ceil(NC / NCS) puts the last piece's start below the segment's end,
    // and segments 0..P-2 hold NC chunks each
    const int c_begin = sg * NC + j * NCS;
    const int c_end = min(min(c_begin + NCS, (sg + 1) * NC), NT);
    const int t_end = min(c_end * CL, T);
    const int nsteps = (c_end - c_begin + 1) / 2;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int W = wv >> 1, hh = wv & 1;
    const int lr = lane & 15, lq = lane >> 4;
    const int row = threadIdx.x >> 3, c8 = (threadIdx.x & 7) * 8;
    const size_t rs = tok_rs<SEQ>(B, H);
    PieceLoads nx;
    auto issue = [&](int m) {
        const int t0 = (c_begin + 2 * m) * CL, nv = min(PSPAN, t_end - t0);
        const size_t base = tok_base<SEQ>(bh, t0, B, H, T);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const size_t off = base + (size_t)min(row + 64 * h, nv - 1) * rs + c8;
            nx.x[h] = *reinterpret_cast<const uint4*>(k + off);
            nx.y[h] = *reinterpret_cast<const uint4*>(v + off);
            nx.w[h] = *reinterpret_cast<const uint4*>(w + off);
        }
    };
    auto nvalid = [&](int m) { return min(PSPAN, t_end - (c_begin + 2 * m) * CL); };
    f32x4 acc[2] = {};
    float gsum = 0.f;                      // total log2-decay of channel lane (wave 7)
    if (nsteps > 0) piece_steps<SEQ, false>(sm, nx, nsteps, issue, nvalid, acc, gsum);
    const size_t sq = (size_t)bh * npieces + q;
#pragma unroll
    for (int tp = 0; tp < 2; ++tp)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
            Sseg[sq * KD * KD + (16 * W + 4 * lq + rr) * KD + 32 * hh + 16 * tp + lr] = acc[tp][rr];
    if (wv == 7) Aseg[sq * KD + lane] = gsum;
}

// Start states of the output walk's segments 1..P-1: the pieces folded in order onto h0 (or
// zero), S = 2^{A_q} S + S_q, and Sstart[b,h][p-1] = S after the pieces of segments 0..p-1.
// One thread per state element (i, j) of one sequence, 16 blocks of 256 per sequence; the
// pieces are loaded eight at a time (clamped, unconditional loads) ahead of the chain.
#define FOLD_THR 256
__global__ void __launch_bounds__(FOLD_THR)
wkv6_fwd_fold(const float* __restrict__ Sseg, const float* __restrict__ Aseg,
              const float* __restrict__ h0, float* __restrict__ Sstart, int npieces, int SUB,
              int P) {
    constexpr int BPS = KD * KD / FOLD_THR;            // blocks per sequence
    const int bh = blockIdx.x / BPS, e = (blockIdx.x - bh * BPS) * FOLD_THR + threadIdx.x;
    const int i = e / KD;
    float s = h0 ? h0[(size_t)bh * KD * KD + e] : 0.f;
    const size_t qb = (size_t)bh * npieces;
    for (int q0 = 0; q0 < npieces; q0 += 8) {
        float a[8], x[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const size_t q = qb + min(q0 + t, npieces - 1);
            a[t] = Aseg[q * KD + i];
            x[t] = Sseg[q * KD * KD + e];
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int q = q0 + t;
            if (q < npieces) {
                s = ex2(a[t]) * s + x[t];
                if ((q + 1) % SUB == 0) Sstart[((size_t)bh * (P - 1) + (q + 1) / SUB - 1) * KD * KD + e] = s;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// backward pre-pass: the state gradients runs of chunks ("pieces") hand to the left
// ---------------------------------------------------------------------------
// With the reverse walk cut into P segments, segment p starts at its last chunk from the
// state gradient dS_end(p) the later segments hand it.  Each of the segments 1..P-1 is cut into
// SUB pieces of at most NCS chunks (trailing pieces of a short last segment are empty); one
// workgroup per (b,h, piece) walks its chunks from the last to the first from a zero state
// gradient, two chunks (PSPAN = 128 tokens) per step, aligned on the piece's first chunk,
//   dS = diag(e^{G_end}) dS + s sum_t (r_t e^{G_{t-1}}) dO_t^T                  [MFMA]
// (G from the step's start; the exponents are never positive) and writes the piece's dS_q
// (fp32 [64][64]) and total log2-decay A_q ([64]).  Reads r, w (sequence-first for SEQ) and
// dO (head-first); the step body is wkv6_fwd_pieces' with r e^{G_{t-1}} as the A operand.
template <bool SEQ>
__global__ void __launch_bounds__(NTHR_W)
wkv6_bwd_pieces(const uint16_t* __restrict__ r, const uint16_t* __restrict__ w,
                const uint16_t* __restrict__ dO, float* __restrict__ dSp, float* __restrict__ Ap,
                float scale, int B, int H, int T, int NT, int NC, int SUB, int NCS, int npieces) {
    __shared__ __attribute__((aligned(16))) PieceSmem sm;
    const int bh = blockIdx.x / npieces, q = blockIdx.x - bh * npieces;
    const int sg = 1 + q / SUB, j = q - (sg - 1) * SUB;            // segments 1..P-1
    const int c_begin = sg * NC + j * NCS;
    const int c_end = min(min(c_begin + NCS, (sg + 1) * NC), NT);
    const int t_end = min(c_end * CL, T);
    const int nsteps = (c_end - c_begin + 1) / 2;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int W = wv >> 1, hh = wv & 1;
    const int lr = lane & 15, lq = lane >> 4;
    const int row = threadIdx.x >> 3, c8 = (threadIdx.x & 7) * 8;
    const size_t rs = tok_rs<SEQ>(B, H);
    PieceLoads nx;
    auto issue = [&](int m) {
        const int t0 = (c_begin + 2 * m) * CL, nv = min(PSPAN, t_end - t0);
        const size_t base = tok_base<SEQ>(bh, t0, B, H, T);
        const size_t dbase = tok_base<false>(bh, t0, B, H, T);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int rrow = min(row + 64 * h, nv - 1);
            nx.x[h] = *reinterpret_cast<const uint4*>(r + base + (size_t)rrow * rs + c8);
            nx.w[h] = *reinterpret_cast<const uint4*>(w + base + (size_t)rrow * rs + c8);
            nx.y[h] = *reinterpret_cast<const uint4*>(dO + dbase + (size_t)rrow * KD + c8);
        }
    };
    auto nvalid = [&](int m) { return min(PSPAN, t_end - (c_begin + 2 * m) * CL); };
    f32x4 acc[2] = {};
    float gsum = 0.f;                      // total log2-decay of channel lane (wave 7)
    if (nsteps > 0) piece_steps<SEQ, true>(sm, nx, nsteps, issue, nvalid, acc, gsum);
    const size_t sq = (size_t)bh * npieces + q;
#pragma unroll
    for (int tp = 0; tp < 2; ++tp)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
            dSp[sq * KD * KD + (16 * W + 4 * lq + rr) * KD + 32 * hh + 16 * tp + lr] = scale * acc[tp][rr];
    if (wv == 7) Ap[sq * KD + lane] = gsum;
}

// dS_end[b,h][p], p = 0..P-2: the state gradient segment p starts from, the pieces folded from
// the last to the first onto dhT (or zero), dS = 2^{A_q} dS + dS_q, recorded after the first
// piece of each segment p+1.  Thread layout and load batching as wkv6_fwd_fold.
__global__ void __launch_bounds__(FOLD_THR)
wkv6_bwd_fold(const float* __restrict__ dSp, const float* __restrict__ Ap,
              const float* __restrict__ dhT, float* __restrict__ dSend, int npieces, int SUB,
              int P) {
    constexpr int BPS = KD * KD / FOLD_THR;
    const int bh = blockIdx.x / BPS, e = (blockIdx.x - bh * BPS) * FOLD_THR + threadIdx.x;
    const int i = e / KD;
    float s = dhT ? dhT[(size_t)bh * KD * KD + e] : 0.f;
    const size_t qb = (size_t)bh * npieces;
    for (int q0 = npieces - 1; q0 >= 0; q0 -= 8) {
        float a[8], x[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const size_t q = qb + max(q0 - t, 0);
            a[t] = Ap[q * KD + i];
            x[t] = dSp[q * KD * KD + e];
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int q = q0 - t;
            if (q >= 0) {
                s = ex2(a[t]) * s + x[t];
                if (q % SUB == 0) dSend[((size_t)bh * (P - 1) + q / SUB) * KD * KD + e] = s;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// backward state gradients, chunk-parallel form (used when B*H is too small for one
// reverse walk per sequence to fill the device)
// ---------------------------------------------------------------------------
// Per (b,h, chunk): dS_loc = s sum_t (r_t e^{G_{t-1}}) dO_t^T [MFMA] and dec = e^{G_63}; then
// one scan thread per pair of state elements: dS_out(c-1) = dec(c) dS_out(c) + dS_loc(c).
// SEQ: r and w (as pre-activation decay) are sequence-first; dO is head-first.
template <bool SEQ>
__global__ void __launch_bounds__(NTHR)
wkv6_bwd_chunk_dstate(const uint16_t* __restrict__ r, const uint16_t* __restrict__ dO,
                      const uint16_t* __restrict__ w, uint16_t* __restrict__ dSloc,
                      float* __restrict__ dec, float scale, int B, int H, int T, int NT) {
    __shared__ __attribute__((aligned(16))) tile_t Xs, Ys, Wm;
    __shared__ __attribute__((aligned(16))) float Gstore[CL * GSG];
    __shared__ float tot[NTHR];
    float (*Gm)[GSG] = reinterpret_cast<float (*)[GSG]>(Gstore);
    const int c = blockIdx.x, bh = blockIdx.y;
    const int t0 = c * CL, nvalid = min(CL, T - t0);
    const size_t base = tok_base<SEQ>(bh, t0, B, H, T), rs = tok_rs<SEQ>(B, H);
    const size_t dbase = tok_base<false>(bh, t0, B, H, T);
    // all six 16-byte loads in flight before the first LDS store waits on one: the loads are
    // unconditional (rows past the end read the last token) and a ragged last chunk zeroes
    // those rows afterwards (a load under a branch makes the merge wait for it)
    uint4 xr[2], yq[2], wq[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int idx = p * NTHR + threadIdx.x, row = min(idx >> 3, nvalid - 1), c8 = (idx & 7) * 8;
        xr[p] = *reinterpret_cast<const uint4*>(r + base + (size_t)row * rs + c8);
        yq[p] = *reinterpret_cast<const uint4*>(dO + dbase + (size_t)row * KD + c8);
        wq[p] = *reinterpret_cast<const uint4*>(w + base + (size_t)row * rs + c8);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int idx = p * NTHR + threadIdx.x, row = idx >> 3, c8 = (idx & 7) * 8;
        sstore16(Ys, row, c8, yq[p]);
        sstore16(Wm, row, c8, wq[p]);
    }
    if (nvalid < CL) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int idx = p * NTHR + threadIdx.x, row = idx >> 3, c8 = (idx & 7) * 8;
            if (row >= nvalid) {
                sstore16(Ys, row, c8, make_uint4(0u, 0u, 0u, 0u));
                sstore16(Wm, row, c8, make_uint4(0u, 0u, 0u, 0u));
            }
        }
    }
    __syncthreads();
    build_G<NTHR, SEQ>(Wm, Gm, tot, nvalid);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int idx = p * NTHR + threadIdx.x, row = idx >> 3, c8 = (idx & 7) * 8;
        float xf[8], e[8];
        unpack8(xr[p], xf);
        const float keep = row < nvalid ? 1.f : 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) e[s] = xf[s] * keep;
        {
            float gp[8];
            g8m1(Gm, row, c8, gp);
#pragma unroll
            for (int s = 0; s < 8; ++s) e[s] *= ex2(gp[s]);
        }
        sstore16(Xs, row, c8, pack8(e));
    }
    if (threadIdx.x < KD) dec[((size_t)bh * NT + c) * KD + threadIdx.x] = ex2(Gm[CL - 1][threadIdx.x]);
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    f32x4 acc[4] = {};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 a = ld_tr8(&Xs[0][0], 32 * ks, 16 * wv);          // row i = 16wv+lr
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) acc[tj] = mfma32(a, ld_tr8(&Ys[0][0], 32 * ks, 16 * tj), acc[tj]);
    }
    // bf16, staged through LDS (Wm is free since build_G) for 16-byte stores
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) Wm[16 * wv + 4 * lq + rr][16 * tj + lr] = f2bf(scale * acc[tj][rr]);
    __syncthreads();
    store_tile<NTHR>(dSloc + ((size_t)bh * NT + c) * KD * KD, Wm, KD);
}

// A thread carries two adjacent elements of one state row (4-byte bf16 accesses) and issues
// the loads of SCAN_U chunks before it walks them (they do not depend on the carry).
#define SCAN_U 32
#define SCAN_BLK 8                         // blocks per (b,h): 8 x 256 threads x 2 elements

// dHs[c] = bf16(dS_out(c)) (gradient w.r.t. the state after chunk c); dh0 = dS_out(-1).
__global__ void __launch_bounds__(NTHR)
wkv6_state_scan_bwd(const uint16_t* __restrict__ dSloc, const float* __restrict__ decay,
                    const float* __restrict__ dhT, uint16_t* __restrict__ dHs,
                    float* __restrict__ dh0, int NT) {
    const int bh = blockIdx.x / SCAN_BLK;
    const int e = ((blockIdx.x % SCAN_BLK) * NTHR + threadIdx.x) * 2;
    const int i = e >> 6;
    float2 dS = dhT ? *reinterpret_cast<const float2*>(dhT + (size_t)bh * KD * KD + e) : make_float2(0.f, 0.f);
    const uint32_t* sl = reinterpret_cast<const uint32_t*>(dSloc + (size_t)bh * NT * KD * KD + e);
    const float* dc = decay + (size_t)bh * NT * KD + i;
    uint32_t* hs = reinterpret_cast<uint32_t*>(dHs + (size_t)bh * NT * KD * KD + e);
    constexpr size_t ST = KD * KD / 2;
    int c = NT - 1;
    for (; c - (SCAN_U - 1) >= 0; c -= SCAN_U) {
        uint32_t l[SCAN_U];
        float d[SCAN_U];
#pragma unroll
        for (int q = 0; q < SCAN_U; ++q) {
            l[q] = sl[(c - q) * ST];
            d[q] = dc[(c - q) * KD];
        }
#pragma unroll
        for (int q = 0; q < SCAN_U; ++q) {
            hs[(c - q) * ST] = pk2(dS.x, dS.y);
            dS.x = d[q] * dS.x + __uint_as_float(l[q] << 16);
            dS.y = d[q] * dS.y + __uint_as_float(l[q] & 0xffff0000u);
        }
    }
    for (; c >= 0; --c) {
        hs[c * ST] = pk2(dS.x, dS.y);
        const uint32_t l = sl[c * ST];
        const float d = dc[c * KD];
        dS.x = d * dS.x + __uint_as_float(l << 16);
        dS.y = d * dS.y + __uint_as_float(l & 0xffff0000u);
    }
    if (dh0) *reinterpret_cast<float2*>(dh0 + (size_t)bh * KD * KD + e) = dS;
}


// ---------------------------------------------------------------------------
// backward: gradients of one chunk
// ---------------------------------------------------------------------------
// 8 waves: wave (W, hh) owns tokens [16W, 16W+16) (the targets of dr, the sources of dk and
// dv) and channels 32hh .. 32hh+31.  Lane (lq, lr) holds, for tp = 0, 1 and rr = 0..3, the
// positions t = 16W + 4lq + rr, i = 32hh + 16tp + lr: the layout of an MFMA accumulator, so the
// lane that builds an operand element is the lane that finishes that element's gradients.
// G is the cumulative log2-decay, mu_W = G[16W+7], b_W = G[16W+15], Fm = e^{G_{t-1} - mu_W},
// Fk = e^{mu_W - G_t}, s = scale, S_in / S_out the states before / after the chunk, dS the
// gradient of S_out, dA[t][tau] = dO_t . v_tau, and Rm = r Fm, Km = k Fk the bf16 operands:
//   dr = s Fm (e^{mu_W} dO S_in^T + sum_{J<W} p_WJ q_J dA Km + tril(dA) Km)        + s u k dd
//   dk = Fk (e^{G_63-mu_W} v dS^T + s sum_{I>W} q_W p_IW dA^T Rm + s tril(dA)^T Rm) + s u r dd
//   dv = Kt dS + s sum_{I>=W} A_IW^T dO,   Kt = Km e^{G_63-mu_W}
//   dw[t] = D + sum_{m>t} (Rm s acc_r - Km acc_k)[m] - (Km acc_k)[t]
// with acc_r = dr_h / (s Fm), acc_k = dk_h / Fk the bracketed accumulators, cross-block factors
// split at the end of the source block, p_IJ = e^{mu_I - b_J} (table fp), q_J = e^{b_J - mu_J}
// (table kb), applied one after the other to the accumulators (dr, dk) or one to each operand
// (dv), and D = rowsum(S_out * dS) = e^{G_63} rowsum(S_in * dS) + sum_t (Km acc_k^{inter})[t],
// the exact split S_out = e^{G_63} S_in + S_loc written with the dk terms themselves.
// dw is a suffix sum whose terms for pairs (m, tau) both after t cancel; they cancel exactly
// because the epilogue multiplies the accumulators by the very bf16 Rm, Km the products used
// (a rounding the epilogue did not see would survive in dw at the size of the cancelling terms).
// Operand tiles Rm, Km, Kt and Kq = Km q_W are stored channel-major (X^T[i][t]): a lane writes
// its 4 tokens of a channel with one 8-byte store and reads them back the same way.
struct GradSmem {
    // the small, often-read members first: within the 16-bit offset of the LDS instructions
    float emu[4][KD], eg[4][KD], kb[3][KD], fp[6][KD];
    float bonus[CL], Dv[KD];
    float Pk[4][KD];                // per-wave sums of Km acc_k^{inter}, for D
    float red[8][KD];               // block totals and mu of the decay scan, then dw block totals
                                    // [0..3] and du partials [4..7]
    tile_t Vt, Dt;                  // raw v, dO (token-major); output staging at the end
    tile_t RT, KT;                  // raw r, k (token-major), then Rm^T, Km^T (channel-major)
    tile_t KtT, KqT;                // Kt^T, Kq^T (channel-major)
    tile_t Sin, dS;                 // raw w in Sin first, then S_in, dS (bf16 [i][j])
};
static_assert(2 * sizeof(GradSmem) <= 160 * 1024, "two gradient blocks must fit one CU's LDS");

// Channel-major tile X^T (row = channel, stride TS): tokens t0 .. t0 + 3 of channel i in one
// 8-byte access (t0 a multiple of 4).
__device__ __forceinline__ bf16x4 ld_ch4(const uint16_t* XT, int i, int t0) {
    return __builtin_bit_cast(bf16x4, *reinterpret_cast<const uint2*>(XT + i * TS + t0));
}
__device__ __forceinline__ void st_ch4(uint16_t* XT, int i, int t0, const float* f) {
    *reinterpret_cast<uint2*>(XT + i * TS + t0) = make_uint2(pk2(f[0], f[1]), pk2(f[2], f[3]));
}

// What a lane carries from the operand build into the products, and what it hands on to the
// cross-lane and cross-wave part of the epilogue.
struct GradLane {
    bf16x4 rrw[2], krw[2], rmb[2], kmb[2];   // raw r, k and the bf16 operands Rm, Km at its positions
    float Fm[2][4], Fk[2][4], ulane[2];      // epilogue factors; s u of its two channels
};
struct GradOut {
    bf16x4 drb[2], dkb[2];                   // dr, dk (bf16) at the lane's positions
    float dwv[2][4];                         // dw less D and the later lanes / blocks
    float lt[2];                             // the lane's sum of x = Rm s acc_r - Km acc_k
    float dup[2];                            // du partial: sum over the lane's tokens of r k dd
    unsigned floored;                        // head-first: bit 4tp + rr for a floored token
    bool fl[4];                              // the reverse walk's: token rr floored (head-first);
                                             // per-lane flags the compiler keeps as lane masks
                                             // in scalar registers (a bit field costs 3 VALU a
                                             // token to build and test)
    f32x4 av[2];                             // dv
};

// The products of token block W (wave-uniform, in a scalar register) for the NTP 16-channel
// columns c0 + 16tp of the wave, with dr and dk finished as soon as their accumulators are
// complete (their factors, raw r, k and dd are then dead while dv is formed).
template <bool SEQ, int NTP, class Smem>
__device__ __forceinline__ void grads_products(Smem& sm, int W, int c0, float scale,
                                               const GradLane& g, GradOut& out, int lane) {
    const int TW = 16 * W;
    const int lr = lane & 15, lq = lane >> 4;
    const int rowW = TW + lr;
    const uint16_t* Vp = &sm.Vt[0][0];
    const uint16_t* Dp = &sm.Dt[0][0];
    const uint16_t* RTp = &sm.RT[0][0];
    const uint16_t* KTp = &sm.KT[0][0];
    const int cbl[2] = {c0 + lr, c0 + 16 + lr};              // the lane's channel of each tp
    f32x4 ar[2], ak[2];
    float ddv[4], xr[2][4];
    // ---------------- dr (targets t in W) ----------------
    {
        f32x4 tmp[2] = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 a = ld_row8(Dp, rowW, 32 * ks, lane);
#pragma unroll
            for (int tp = 0; tp < NTP; ++tp)
                tmp[tp] = mfma32(a, ld_row8(&sm.Sin[0][0], cbl[tp], 32 * ks, lane), tmp[tp]);
        }
#pragma unroll
        for (int tp = 0; tp < NTP; ++tp) ar[tp] = tmp[tp] * sm.emu[W][cbl[tp]];
    }
    for (int J = 0; J < W; ++J) {          // dA[t = 16W+lr][tau = 16J+4lq+rr], then x Km_J
        f32x4 at = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            at = mfma32(ld_row8(Vp, 16 * J + lr, 32 * ks, lane), ld_row8(Dp, rowW, 32 * ks, lane), at);
        const bf16x4 aop = cvt4(at[0], at[1], at[2], at[3]);
#pragma unroll
        for (int tp = 0; tp < NTP; ++tp) {
            const f32x4 t2 = mfma16(aop, ld_ch4(KTp, cbl[tp], 16 * J + 4 * lq), f32x4{});
            // the two halves of the cross factor one after the other (q_J p_WJ as one number can
            // underflow where the product with t2 is O(1))
            ar[tp] += (t2 * sm.kb[J][cbl[tp]]) * sm.fp[(W * (W - 1)) / 2 + J][cbl[tp]];
        }
    }
    {   // diagonal block: strictly causal part; its diagonal dA[t][t] = dd[t]
        f32x4 at = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            at = mfma32(ld_row8(Vp, rowW, 32 * ks, lane), ld_row8(Dp, rowW, 32 * ks, lane), at);
        // the lane's tokens 16W + 4lq + rr take dd from lane (lq, 4lq + rr), element rr
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) ddv[rr] = __shfl(at[rr], 20 * lq + rr);
        float xa[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) xa[rr] = 4 * lq + rr < lr ? at[rr] : 0.f;
        const bf16x4 aop = cvt4(xa[0], xa[1], xa[2], xa[3]);
#pragma unroll
        for (int tp = 0; tp < NTP; ++tp) ar[tp] = mfma16(aop, ld_ch4(KTp, cbl[tp], TW + 4 * lq), ar[tp]);
    }
    // dr = s Fm acc_r + s u k dd;  Rm s acc_r, the first half of x
#pragma unroll
    for (int tp = 0; tp < NTP; ++tp) {
        float d[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float sar = scale * ar[tp][rr];
            d[rr] = g.Fm[tp][rr] * sar + (g.ulane[tp] * ddv[rr]) * (float)g.krw[tp][rr];
            xr[tp][rr] = (float)g.rmb[tp][rr] * sar;
        }
        out.drb[tp] = cvt4(d[0], d[1], d[2], d[3]);
    }
    // ---------------- dk (sources tau in W) ----------------
    {
        f32x4 tmp[2] = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 a = ld_row8(Vp, rowW, 32 * ks, lane);
#pragma unroll
            for (int tp = 0; tp < NTP; ++tp)
                tmp[tp] = mfma32(a, ld_row8(&sm.dS[0][0], cbl[tp], 32 * ks, lane), tmp[tp]);
        }
        float pk[2];
#pragma unroll
        for (int tp = 0; tp < NTP; ++tp) {
            ak[tp] = tmp[tp] * sm.eg[W][cbl[tp]];
            // this wave's share of sum_tau Km acc_k^{inter}[tau] (the dk terms of D)
            pk[tp] = 0.f;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) pk[tp] += (float)g.kmb[tp][rr] * ak[tp][rr];
        }
        if (NTP == 2) {
            // sum over lq (lane bits 4, 5): lanes of odd lq keep tp = 1, even lq tp = 0
            const bool up = lane & 16;
            float p = (up ? pk[1] : pk[0]) + lane_xor_swz<16>(up ? pk[0] : pk[1]);
            p += lane_xor32(p);
            if (lq < 2) sm.Pk[W][c0 + 16 * lq + lr] = p;
        } else {
            float p = pk[0] + lane_xor_swz<16>(pk[0]);
            p += lane_xor32(p);
            if (lq == 0) sm.Pk[W][c0 + lr] = p;
        }
    }
    {   // diagonal block: dA[t = 16W+4lq+rr][tau = 16W+lr], t > tau
        f32x4 at = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            at = mfma32(ld_row8(Dp, rowW, 32 * ks, lane), ld_row8(Vp, rowW, 32 * ks, lane), at);
        float xa[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) xa[rr] = 4 * lq + rr > lr ? at[rr] * scale : 0.f;
        const bf16x4 aop = cvt4(xa[0], xa[1], xa[2], xa[3]);
#pragma unroll
        for (int tp = 0; tp < NTP; ++tp) ak[tp] = mfma16(aop, ld_ch4(RTp, cbl[tp], TW + 4 * lq), ak[tp]);
    }
    {
        for (int I = W + 1; I < 4; ++I) {  // dA[t = 16I+4lq+rr][tau = 16W+lr], then x Rm_I
            f32x4 at = {};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                at = mfma32(ld_row8(Dp, 16 * I + lr, 32 * ks, lane), ld_row8(Vp, rowW, 32 * ks, lane), at);
            const bf16x4 aop = cvt4(at[0] * scale, at[1] * scale, at[2] * scale, at[3] * scale);
#pragma unroll
            for (int tp = 0; tp < NTP; ++tp) {
                const f32x4 t2 = mfma16(aop, ld_ch4(RTp, cbl[tp], 16 * I + 4 * lq), f32x4{});
                ak[tp] += (t2 * sm.fp[(I * (I - 1)) / 2 + W][cbl[tp]]) * sm.kb[W][cbl[tp]];
            }
        }
    }
    // dk = Fk acc_k + s u r dd;  x = Rm s acc_r - Km acc_k, y = -Km acc_k, summed within the
    // lane over the later tokens; du partial r k dd
    out.floored = 0u;
#pragma unroll
    for (int tp = 0; tp < NTP; ++tp) {
        float d[4], xv[4];
        out.dup[tp] = 0.f;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float rv = (float)g.rrw[tp][rr], kv = (float)g.krw[tp][rr];
            d[rr] = g.Fk[tp][rr] * ak[tp][rr] + (g.ulane[tp] * ddv[rr]) * rv;
            out.dup[tp] += (rv * kv) * ddv[rr];
            const float y = -(float)g.kmb[tp][rr] * ak[tp][rr];
            xv[rr] = xr[tp][rr] + y;
            out.dwv[tp][rr] = y;
            // head-first: Fm Fk = e^{G_{t-1} - G_t} = e^{-max(w_t, W_MIN)} is e^{-W_MIN} exactly
            // at the floor; the test also takes tokens within 1 % of the floor's decay factor
            // (w in [W_MIN, W_MIN + 0.01)), whose exact dw carries a factor below 4.6e-5 too
            if (!SEQ && g.Fm[tp][rr] * g.Fk[tp][rr] > FLOOR_FF) out.floored |= 1u << (4 * tp + rr);
        }
        out.dkb[tp] = cvt4(d[0], d[1], d[2], d[3]);
        out.dwv[tp][2] += xv[3];
        out.dwv[tp][1] += xv[3] + xv[2];
        out.dwv[tp][0] += (xv[3] + xv[2]) + xv[1];
        out.lt[tp] = ((xv[3] + xv[2]) + xv[1]) + xv[0];
    }
    // ---------------- dv (sources tau in W, value columns c0..) ----------------
    f32x4 av[2] = {};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 a = ld_tr8(&sm.KtT[0][0], 32 * ks, TW, lane);           // Kt[tau = 16W+lr][i]
#pragma unroll
        for (int tp = 0; tp < NTP; ++tp)
            av[tp] = mfma32(a, ld_tr8(&sm.dS[0][0], 32 * ks, c0 + 16 * tp, lane), av[tp]);
    }
    // the 16x16x16 products below accumulate onto a VALU copy of the 16x16x32 result, never
    // onto the 16x16x32 result itself (no mixed-shape MFMA accumulation chain)
    {
        float one;
        asm volatile("" : "=v"(one) : "0"(1.0f));
#pragma unroll
        for (int tp = 0; tp < NTP; ++tp) av[tp] = av[tp] * one;
    }
    {   // diagonal block: A[t = 16W+4lq+rr][tau = 16W+lr], t > tau, the u-bonus at t == tau
        f32x4 at = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            at = mfma32(ld_tr8_g8(RTp, 32 * ks, TW, lane), ld_tr8_g8(KTp, 32 * ks, TW, lane), at);
        const float bon = sm.bonus[rowW];
        float xa[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int tl = 4 * lq + rr;
            xa[rr] = (tl > lr ? at[rr] : (tl == lr ? bon : 0.f)) * scale;
        }
        const bf16x4 aop = cvt4(xa[0], xa[1], xa[2], xa[3]);
#pragma unroll
        for (int tp = 0; tp < NTP; ++tp) av[tp] = mfma16(aop, ld_tr4(Dp, TW, c0 + 16 * tp, lane), av[tp]);
    }
    {
        for (int I = W + 1; I < 4; ++I) {  // A[t = 16I+4lq+rr][tau = 16W+lr] = (Rm_I p_IW) Kq_W
            f32x4 at = {};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                float f[8];
                row8_vec(sm.fp[(I * (I - 1)) / 2 + W], 32 * ks, f, lane);
                at = mfma32(scale8(ld_tr8_g8(RTp, 32 * ks, 16 * I, lane), f),
                            ld_tr8_g8(&sm.KqT[0][0], 32 * ks, TW, lane), at);    // Kq[tau = 16W+lr][i]
            }
            const bf16x4 aop = cvt4(at[0] * scale, at[1] * scale, at[2] * scale, at[3] * scale);
#pragma unroll
            for (int tp = 0; tp < NTP; ++tp)
                av[tp] = mfma16(aop, ld_tr4(Dp, 16 * I, c0 + 16 * tp, lane), av[tp]);
        }
    }
#pragma unroll
    for (int tp = 0; tp < NTP; ++tp) out.av[tp] = av[tp];
}

// SEQ: r, k, v, the pre-activation decay and dr, dk, dv, d_decay are sequence-first (dO is
// head-first); the decay gradient is dw * w with w = -exp(decay).
template <bool SEQ>
__global__ void __launch_bounds__(NTHR_G) __attribute__((amdgpu_waves_per_eu(4)))
wkv6_bwd_chunk_grads(const uint16_t* __restrict__ r, const uint16_t* __restrict__ k,
                     const uint16_t* __restrict__ v, const uint16_t* __restrict__ w,
                     const void* __restrict__ u, int u_dtype, const uint16_t* __restrict__ dO,
                     const uint16_t* __restrict__ Hs, const uint16_t* __restrict__ dHs,
                     uint16_t* __restrict__ dr, uint16_t* __restrict__ dk,
                     uint16_t* __restrict__ dv, uint16_t* __restrict__ dw,
                     float* __restrict__ du_part, float scale, int B, int H, int T, int NT) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
    GradSmem& sm = *reinterpret_cast<GradSmem*>(smem_raw);
    const int c = blockIdx.x, bh = blockIdx.y, h = bh % H;
    const int t0 = c * CL, nvalid = min(CL, T - t0);
    const size_t base = tok_base<SEQ>(bh, t0, B, H, T), rs = tok_rs<SEQ>(B, H);
    const size_t dbase = ((size_t)bh * T + t0) * KD;           // dO: head-first
    const int row = threadIdx.x >> 3, c8 = (threadIdx.x & 7) * 8;

    // ---- P0: one 16-byte piece of every tile per thread, all loads in flight together (rows
    // past a ragged end read the last token and are zeroed below) ----
    const int lrow = min(row, nvalid - 1);
    uint4 rq = *reinterpret_cast<const uint4*>(r + base + (size_t)lrow * rs + c8);
    uint4 kq = *reinterpret_cast<const uint4*>(k + base + (size_t)lrow * rs + c8);
    uint4 vq = *reinterpret_cast<const uint4*>(v + base + (size_t)lrow * rs + c8);
    uint4 wq = *reinterpret_cast<const uint4*>(w + base + (size_t)lrow * rs + c8);
    uint4 dq = *reinterpret_cast<const uint4*>(dO + dbase + (size_t)lrow * KD + c8);
    // states: S_in and dS rows (thread row = channel i), into LDS once the w scratch is consumed
    const uint4 sq = *reinterpret_cast<const uint4*>(Hs + ((size_t)bh * (NT + 1) + c) * KD * KD + row * KD + c8);
    const uint4 dsq = *reinterpret_cast<const uint4*>(dHs + ((size_t)bh * NT + c) * KD * KD + row * KD + c8);
    float uf[8];
    load_param8(u, u_dtype, h * KD + c8, uf);
    if (nvalid < CL) {
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        if (row >= nvalid) rq = kq = vq = wq = dq = z;
    }
    sstore16(sm.Vt, row, c8, vq);
    sstore16(sm.Dt, row, c8, dq);
    sstore16(sm.RT, row, c8, rq);
    sstore16(sm.KT, row, c8, kq);
    sstore16(sm.Sin, row, c8, wq);                       // w scratch until the scan has read it
    {
        // bonus[t] = sum_i r u k (token t = row);  Dv[i] = sum_j S_in dS (channel i = row)
        float rf[8], kf[8], a8[8], b8[8], b = 0.f, d = 0.f;
        unpack8(rq, rf);
        unpack8(kq, kf);
        unpack8(sq, a8);
        unpack8(dsq, b8);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            b += (rf[s] * uf[s]) * kf[s];
            d += a8[s] * b8[s];
        }
        b = sum8lanes(b);
        d = sum8lanes(d);
        if ((threadIdx.x & 7) == 0) {
            sm.bonus[row] = b;
            sm.Dv[row] = d;
        }
    }
    __syncthreads();

    // ---- P1: raw r, k, w at the lane's positions; the decay scan in registers; Fm, Fk; Rm, Km ----
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int W = wv >> 1, hh = wv & 1;
    const int lr = lane & 15, lq = lane >> 4;
    const int t4 = 16 * W + 4 * lq;                       // the lane's first token
    GradLane gl;
    bf16x4 wrw[2];
    float kmf[2][4], qloc[2];
#pragma unroll
    for (int tp = 0; tp < 2; ++tp) {
        const int cb = 32 * hh + 16 * tp;
        gl.rrw[tp] = ld_tr4(&sm.RT[0][0], 16 * W, cb);      // x[16W + 4lq + s][cb + lr]
        gl.krw[tp] = ld_tr4(&sm.KT[0][0], 16 * W, cb);
        wrw[tp] = ld_tr4(&sm.Sin[0][0], 16 * W, cb);
        gl.ulane[tp] = scale * load_u(u, u_dtype, h * KD + cb + lr);
        // cumulative log2-decay within the block: the lane's 4 tokens, then the lanes before
        // it in the block (lanes lr + 16 lq' of the same wave)
        float cs[4], run = 0.f;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            float x = (float)wrw[tp][rr];
            if (SEQ) x = t4 + rr < nvalid ? -ex2(x * RW_L2E) : 0.f;   // w = -exp(decay), :336
            run += fmaxf(x, W_MIN) * RW_L2E;
            cs[rr] = run;
        }
        float xi = run, y = __shfl_up(xi, 16);
        xi += lq >= 1 ? y : 0.f;
        y = __shfl_up(xi, 32);
        xi += lq >= 2 ? y : 0.f;                            // inclusive over lq
        const float excl = xi - run;
        const float tot = __shfl(xi, 48 + lr);              // the block's total
        const float m7 = __shfl(excl + cs[3], 16 + lr);     // G at token 16W+7 (lane lq = 1, rr = 3)
        qloc[tp] = tot - m7;                                // b_W - mu_W
        if (lq == 0) {
            sm.red[W][cb + lr] = tot;
            sm.red[4 + W][cb + lr] = m7;
        }
        float rm[4], km[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            gl.Fm[tp][rr] = ex2(excl + (rr ? cs[rr - 1] : 0.f) - m7);
            gl.Fk[tp][rr] = ex2(m7 - (excl + cs[rr]));
            rm[rr] = (float)gl.rrw[tp][rr] * gl.Fm[tp][rr];
            km[rr] = (float)gl.krw[tp][rr] * gl.Fk[tp][rr];
            kmf[tp][rr] = km[rr];
        }
        gl.rmb[tp] = cvt4(rm[0], rm[1], rm[2], rm[3]);
        gl.kmb[tp] = cvt4(km[0], km[1], km[2], km[3]);
    }
    __syncthreads();                       // raw r, k, w read; block totals and mu in `red`

    // ---- P2: operand tiles (channel-major), S_in / dS, the per-block factor tables ----
#pragma unroll
    for (int tp = 0; tp < 2; ++tp) {
        const int i = 32 * hh + 16 * tp + lr;
        *reinterpret_cast<bf16x4*>(&sm.RT[i][t4]) = gl.rmb[tp];
        *reinterpret_cast<bf16x4*>(&sm.KT[i][t4]) = gl.kmb[tp];
        float after = 0.f;                                  // G_63 - b_W
        for (int J = W + 1; J < 4; ++J) after += sm.red[J][i];
        const float eg = ex2(after + qloc[tp]), kq = ex2(qloc[tp]);
        float x[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) x[rr] = kmf[tp][rr] * eg;
        st_ch4(&sm.KtT[0][0], i, t4, x);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) x[rr] = kmf[tp][rr] * kq;
        st_ch4(&sm.KqT[0][0], i, t4, x);
    }
    sstore16(sm.Sin, row, c8, sq);
    sstore16(sm.dS, row, c8, dsq);
    {
        // tables per channel i = lane from the block totals and mu: b_J = G[16J+15],
        // mu_J = b_{J-1} + m7_J; wave wv fills its share (the branches are wave-uniform)
        const int i = lane;
        float bnd[4], mu[4], a = 0.f;
#pragma unroll
        for (int J = 0; J < 4; ++J) {
            mu[J] = a + sm.red[4 + J][i];
            a += sm.red[J][i];
            bnd[J] = a;
        }
        if (wv < 4) {
            const float m = wv == 0 ? mu[0] : wv == 1 ? mu[1] : wv == 2 ? mu[2] : mu[3];
            sm.emu[wv][i] = ex2(m);
            sm.eg[wv][i] = ex2(bnd[3] - m);
            if (wv < 3) sm.kb[wv][i] = ex2((wv == 0 ? bnd[0] : wv == 1 ? bnd[1] : bnd[2]) - m);
            else sm.Dv[i] *= ex2(bnd[3]);
        } else if (wv == 4) {
            sm.fp[0][i] = ex2(mu[1] - bnd[0]);              // (1, 0)
            sm.fp[1][i] = ex2(mu[2] - bnd[0]);              // (2, 0)
        } else if (wv == 5) {
            sm.fp[2][i] = ex2(mu[2] - bnd[1]);              // (2, 1)
            sm.fp[3][i] = ex2(mu[3] - bnd[0]);              // (3, 0)
        } else if (wv == 6) {
            sm.fp[4][i] = ex2(mu[3] - bnd[1]);              // (3, 1)
            sm.fp[5][i] = ex2(mu[3] - bnd[2]);              // (3, 2)
        }
    }
    __syncthreads();

    // ---- P3: the products, dr and dk finished on the way ----
    GradOut go;
    grads_products<SEQ, 2>(sm, __builtin_amdgcn_readfirstlane(W), 32 * hh, scale, gl, go, lane);

    // ---------------- epilogue ----------------
    // dw[t] = D + sum_{m > t} x[m] + y[t]: the suffix sums within the lane are in go.dwv; here
    // across the four lane rows (shuffles) and across the token blocks W (per-wave totals in
    // `red`).
    float wtot[2];
#pragma unroll
    for (int tp = 0; tp < 2; ++tp) {
        // sum over lq' > lq (lanes lr + 16 lq').  The shuffles run on all lanes (a lane outside
        // the exec mask would read as zero).
        const float lt = go.lt[tp];
        const float d16 = __shfl_down(lt, 16);
        float vsum = lt + (lq <= 2 ? d16 : 0.f);
        const float d32 = __shfl_down(vsum, 32);
        vsum += lq <= 1 ? d32 : 0.f;                                // sum over lq' >= lq
        const float later = vsum - lt;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) go.dwv[tp][rr] += later;
        wtot[tp] = vsum;                                            // the wave's total at lq == 0
    }
    // du partial over the wave's 16 tokens: sum over lq (lanes of odd lq keep tp = 1, even
    // lq tp = 0, as for Pk), then over the four token blocks in fixed order below
    {
        const bool up = lane & 16;
        float p = (up ? go.dup[1] : go.dup[0]) + lane_xor_swz<16>(up ? go.dup[0] : go.dup[1]);
        p += lane_xor32(p);
        if (lq < 2) sm.red[4 + W][32 * hh + 16 * lq + lr] = p;
    }
    if (lq == 0) {
        sm.red[W][32 * hh + lr] = wtot[0];
        sm.red[W][32 * hh + 16 + lr] = wtot[1];
    }
    __syncthreads();                       // all products done; red, Pk in
    if (threadIdx.x < KD) {
        const float acc = (sm.red[4][threadIdx.x] + sm.red[5][threadIdx.x]) +
                          (sm.red[6][threadIdx.x] + sm.red[7][threadIdx.x]);
        // head-major [h][b][c][i]: each head's partials are contiguous for the du reduction
        du_part[(((size_t)h * B + bh / H) * NT + c) * KD + threadIdx.x] = scale * acc;
    }
    // dr, dk, dv, dw staged channel-major (X^T[i][t], 8-byte writes of 4 tokens) in tiles the
    // products no longer read, read back token-major by transpose reads for 16-byte stores
    uint16_t (*Ts[4])[TS] = {sm.Vt, sm.Dt, sm.RT, sm.KT};
#pragma unroll
    for (int tp = 0; tp < 2; ++tp) {
        const int i = 32 * hh + 16 * tp + lr;
        float later = sm.Dv[i] + ((sm.Pk[0][i] + sm.Pk[1][i]) + (sm.Pk[2][i] + sm.Pk[3][i]));
        for (int W2 = W + 1; W2 < 4; ++W2) later += sm.red[W2][i];
        float g[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            g[rr] = go.dwv[tp][rr] + later;
            // A floored token's gradient is 0: the derivative of the floored forward, within
            // e^W_MIN of the exact one (which carries the token's own decay factor).  The
            // sequence-first entry returns d decay = dw * w, w = -exp(decay).
            if (SEQ && t4 + rr < nvalid) {
                const float wn = -ex2((float)wrw[tp][rr] * RW_L2E);
                g[rr] = wn < W_MIN ? 0.f : g[rr] * wn;
            }
            if (!SEQ && ((go.floored >> (4 * tp + rr)) & 1u)) g[rr] = 0.f;
        }
        *reinterpret_cast<bf16x4*>(&Ts[0][i][t4]) = go.drb[tp];
        *reinterpret_cast<bf16x4*>(&Ts[1][i][t4]) = go.dkb[tp];
        const float avf[4] = {go.av[tp][0], go.av[tp][1], go.av[tp][2], go.av[tp][3]};
        st_ch4(&Ts[2][0][0], i, t4, avf);
        st_ch4(&Ts[3][0][0], i, t4, g);
    }
    __syncthreads();
    {
        // wave wv stores tokens 16 (wv & 3) + L, channels 32 (wv >> 2) + 8q .. +7 of each tensor
        const int tk = 16 * (wv & 3) + lr, ch = 32 * (wv >> 2) + 8 * lq;
        uint16_t* outs[4] = {dr, dk, dv, dw};
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const uint4 x = __builtin_bit_cast(uint4, ld_tr8_g8(&Ts[n][0][0], 32 * (wv >> 2), 16 * (wv & 3)));
            if (tk < nvalid) *reinterpret_cast<uint4*>(outs[n] + base + (size_t)tk * rs + ch) = x;
        }
    }
}

// ---------------------------------------------------------------------------
// backward as one reverse walk per sequence (B*H large enough to fill the device)
// ---------------------------------------------------------------------------
// One 1024-thread workgroup per (b,h) walks the chunks from the last to the first.  It carries
// the state gradient dS_out(c) (the gradient w.r.t. the state after chunk c, dS_out(NT-1) =
// dhT) in fp32 MFMA accumulators and does, per chunk, what wkv6_bwd_chunk_grads does for one
// chunk (the same factors and rounding points) followed by the state-gradient step
//   dS_out(c-1) = diag(e^{G_63}) dS_out(c) + s sum_t (r_t e^{G_{t-1}})^T dO_t          [MFMA]
// so no dstate pass runs, r, w, dO are read once and dS never goes through HBM; dh0 =
// dS_out(-1) and du are summed over the whole sequence in registers.  The next chunk's raw
// pieces are loaded into registers while the current one is computed.
// 16 waves: wave (W, col) = (wv >> 2, wv & 3) owns tokens [16W, 16W+16) and the one channel
// column [16col, 16col+16); lane (lq, lr) holds t = 16W + 4lq + rr (rr = 0..3), i = 16col + lr,
// and, in the state-gradient accumulator, dS[i = 16col + lr][j = 16W + 4lq + rr].
#define NTHR_L 1024

// Row stride of the 16x16 dA blocks: 20 elements (40 bytes).  With 32-byte rows the direct
// 8-byte reads (row L, columns 4q) of a wave hit the same banks four lanes at a time: 14 clocks
// per instruction against 4 measured on MI355X.
#define DAB_RS 20

struct LoopSmem {
    // Members in the first 64 KB are reached with the 16-bit offset of the LDS instructions;
    // past it every access costs an address add.  The small, often-read members come first,
    // then the tiles in decreasing order of accesses per chunk.
    float emu[4][KD], eg[4][KD], kb[3][KD], fp[6][KD], eG63[KD];
    float bonus[CL], Dv[KD], dd[CL];  // dd[t] = dO_t . v_t
    float uh[KD];                   // u of the head (fp32), for the bonus
    float Pk[4][KD];                // per-wave sums of Km acc_k^{inter}, for D
    float red[8][KD];               // block totals and mu of the decay scan, then dw block
                                    // totals [0..3] and du partials [4..7]
    // the 16x16 blocks of the chunk, once per chunk for all four channel columns:
    // dAb[W(W+1)/2 + J] = dA[t in W][tau in J] (W >= J; the diagonal block strictly lower),
    // bf16 row-major [t][tau]; Ab[I(I+1)/2 + W] = s A[t in I][tau in W] (I >= W; the diagonal
    // block with the u-bonus on its diagonal), bf16 in MFMA-operand order (8 bytes per lane)
    uint16_t dAb[10][16][DAB_RS];
    uint16_t Ab[10][64][4];
    tile_t Dt, dS;                  // raw dO (token-major); dS_out (bf16 [i][j])
    tile_t KT, RT;                  // raw k, r (token-major), then Km^T, Rm^T (channel-major)
    tile_t KtT;                     // raw w first; then Kt^T (channel-major)
    tile_t Vt;                      // raw v (token-major)
    tile_t KqT, RiT;                // Kq^T; (s r e^{G_{t-1}})^T, the state-gradient step's operand
    tile_t RpT[2];                  // (s Rm_I p_IW)^T of the six cross pairs I > W (dv)
    tile_t Sin;                     // S_in (bf16 [i][j])
    tile_t Out[4];                  // dr, dk, dv, dw staged channel-major (token-major for SEQ)
};
static_assert(sizeof(LoopSmem) <= 160 * 1024, "one loop workgroup per CU");

// (J, W) of block b in the order b = W(W+1)/2 + J, J <= W (wave-uniform).
__device__ __forceinline__ void tri_pair(int b, int& hi, int& lo) {
    hi = (b >= 1) + (b >= 3) + (b >= 6);
    lo = b - (hi * (hi + 1)) / 2;
}

// Per-lane LDS byte offsets of the loop kernel's access patterns (lane = 16q + L).  They are
// formed once per launch and passed through an empty asm at the top of every chunk, which
// the compiler must assume changes them: an address of the chunk is then one add (its
// wave-uniform part, or a constant folded into the instruction) from one of them.  Derived
// from the thread id inside the chunk, the addresses cost several instructions each; hoisted
// out of the walk, they do not fit the registers.
struct LaneOfs {
    int tr;      // ((4q + L/4) TS + 4 (L%4)) * 2: ds_read_b64_tr_b16 over rows r0 + 4q + s
    int g8;      // ((8q + L/4) TS + 4 (L%4) + c0) * 2: the same over rows r0 + 8q + s, in the
                 // wave's column c0 (its only use)
    int row;     // (L TS + 8q) * 2: 16-byte row pieces (row L, columns 8q..)
    int ch;      // ((c0 + L) TS + 4q) * 2: 8-byte row pieces (row c0 + L, columns 4q..), c0 =
                 // the wave's channel column 16 col: every use is in the wave's own rows
    int blk;     // (DAB_RS L + 4q) * 2: a 16x16 row-major dA block, direct
    int blktr;   // ((4q + L/4) DAB_RS + 4 (L%4)) * 2: the same, transposed
    int frag;    // 8 lane: 8 bytes per lane in MFMA-operand order
    int tab;     // 4 (c0 + L): a float per channel of the wave's 16-channel column
    int th;      // ((4 wv + q) TS + 4 L) * 2: thread (row, c4) = (tid >> 4, 4 (tid & 15))
    int q16;     // 16 q: four floats per lane row
};
__device__ __forceinline__ LaneOfs lane_ofs(int lane, int wv) {
    const int c0 = 16 * (wv & 3);
    const int L = lane & 15, q = lane >> 4;
    LaneOfs o;
    o.tr = ((4 * q + (L >> 2)) * TS + 4 * (L & 3)) * 2;
    o.g8 = ((8 * q + (L >> 2)) * TS + 4 * (L & 3) + c0) * 2;
    o.row = (L * TS + 8 * q) * 2;
    o.ch = ((c0 + L) * TS + 4 * q) * 2;
    o.blk = (DAB_RS * L + 4 * q) * 2;
    o.blktr = ((4 * q + (L >> 2)) * DAB_RS + 4 * (L & 3)) * 2;
    o.frag = 8 * lane;
    o.tab = 4 * (c0 + L);
    o.th = ((4 * wv + q) * TS + 4 * L) * 2;
    o.q16 = 16 * q;
    return o;
}
__device__ __forceinline__ void launder(LaneOfs& o) {
    asm volatile("" : "+v"(o.tr), "+v"(o.g8), "+v"(o.row), "+v"(o.ch), "+v"(o.blk), "+v"(o.blktr),
                 "+v"(o.frag), "+v"(o.tab), "+v"(o.th), "+v"(o.q16));
}

template <class T>
__device__ __forceinline__ T lds_ld(const void* base, int bytes) {
    return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + bytes);
}
template <class T>
__device__ __forceinline__ void lds_st(void* base, int bytes, T v) {
    *reinterpret_cast<T*>(reinterpret_cast<char*>(base) + bytes) = v;
}
__device__ __forceinline__ bf16x4 lds_tr(const void* base, int bytes) {
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(reinterpret_cast<const char*>(base) + bytes)));
}
__device__ __forceinline__ bf16x8 cat8(bf16x4 a, bf16x4 b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}
// The tile readers of the loop with precomputed offsets (X a bf16 tile of row stride TS):
//   tr8 (X, r0, c0): X[r0 + 4q + s][c0 + L], X[r0 + 16 + 4q + s][c0 + L]   (as ld_tr8)
//   g8  (X, r0, c0): X[r0 + 8q + s][c0 + L], s = 0..7                       (as ld_tr8_g8)
//   row8(X, r0, c0): X[r0 + L][c0 + 8q + s]                                 (as ld_row8)
//   dir8(X, r0, c0): X[r0 + L][c0 + 4q + s], X[r0 + L][c0 + 16 + 4q + s]    (as ld_dir8)
//   ch4 (X, r0, c0): X[r0 + L][c0 + 4q + s], s = 0..3                       (as ld_ch4)
__device__ __forceinline__ int tb(int r0, int c0) { return (r0 * TS + c0) * 2; }
__device__ __forceinline__ bf16x4 tr4o(const uint16_t* X, const LaneOfs& o, int r0, int c0) {
    return lds_tr(X, o.tr + tb(r0, c0));
}
__device__ __forceinline__ bf16x8 tr8o(const uint16_t* X, const LaneOfs& o, int r0, int c0) {
    return cat8(lds_tr(X, o.tr + tb(r0, c0)), lds_tr(X, o.tr + tb(r0 + 16, c0)));
}
__device__ __forceinline__ bf16x8 g8o(const uint16_t* X, const LaneOfs& o, int r0, int c0) {
    return cat8(lds_tr(X, o.g8 + tb(r0, c0)), lds_tr(X, o.g8 + tb(r0 + 4, c0)));
}
__device__ __forceinline__ bf16x8 row8o(const uint16_t* X, const LaneOfs& o, int r0, int c0) {
    return lds_ld<bf16x8>(X, o.row + tb(r0, c0));
}
__device__ __forceinline__ bf16x8 dir8o(const uint16_t* X, const LaneOfs& o, int r0, int c0) {
    const uint2 a = lds_ld<uint2>(X, o.ch + tb(r0, c0)), b = lds_ld<uint2>(X, o.ch + tb(r0, c0 + 16));
    return __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
}
__device__ __forceinline__ bf16x4 ch4o(const uint16_t* X, const LaneOfs& o, int r0, int c0) {
    return lds_ld<bf16x4>(X, o.ch + tb(r0, c0));
}
__device__ __forceinline__ void st_ch4o(uint16_t* X, const LaneOfs& o, int r0, int c0, const float* f) {
    lds_st<uint2>(X, o.ch + tb(r0, c0), make_uint2(pk2(f[0], f[1]), pk2(f[2], f[3])));
}

// dA block b of the chunk (waves 0..9, after the raw tiles are in): the lane holds
// dA[t = 16W + lr][tau = 16J + 4lq + rr] and stores it at row lr, columns 4lq .. +3.
__device__ __forceinline__ void loop_dA_block(LoopSmem& sm, int b, const LaneOfs& o, int lane) {
    int W, J;
    tri_pair(b, W, J);
    const int lr = lane & 15, lq = lane >> 4;
    f32x4 at = {};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
        at = mfma32(row8o(&sm.Vt[0][0], o, 16 * J, 32 * ks), row8o(&sm.Dt[0][0], o, 16 * W, 32 * ks), at);
    float x[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) x[rr] = (W > J || 4 * lq + rr < lr) ? at[rr] : 0.f;
    lds_st<uint2>(&sm.dAb[b][0][0], o.blk, make_uint2(pk2(x[0], x[1]), pk2(x[2], x[3])));
}

// A block b (waves 0..9, after the operand tiles are in): the lane holds
// s A[t = 16I + 4lq + rr][tau = 16W + lr], the A operand of dv's 16x16x16 products.
__device__ __forceinline__ void loop_A_block(LoopSmem& sm, int b, float scale, const LaneOfs& o,
                                             int lane) {
    int I, W;
    tri_pair(b, I, W);
    const int lr = lane & 15, lq = lane >> 4;
    f32x4 at = {};
    float x[4];
    if (I == W) {
        // Rm_W Km_W^T over the channels, strictly causal, the u-bonus on the diagonal
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)     // channel slots in tr8 order on both operands
            at = mfma32(tr8o(&sm.RT[0][0], o, 32 * ks, 16 * W), tr8o(&sm.KT[0][0], o, 32 * ks, 16 * W), at);
        const float bon = lds_ld<float>(&sm.bonus[16 * W], o.tab - 64 * (b & 3));   // o.tab holds c0
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int tl = 4 * lq + rr;
            x[rr] = (tl > lr ? at[rr] : (tl == lr ? bon : 0.f)) * scale;
        }
    } else {
        // (s Rm_I p_IW) Kq_W^T, the pair tile pre-scaled
        const int pi = (I * (I - 1)) / 2 + W;
        const uint16_t* Rp = &sm.RpT[pi >> 2][0][0] + 16 * (pi & 3);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            at = mfma32(tr8o(Rp, o, 32 * ks, 0), tr8o(&sm.KqT[0][0], o, 32 * ks, 16 * W), at);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) x[rr] = at[rr];
    }
    lds_st<uint2>(&sm.Ab[b][0][0], o.frag, make_uint2(pk2(x[0], x[1]), pk2(x[2], x[3])));
}

// dr and dk of the wave's token block W (compile-time) and channel column ch = 16 col + lr (the
// factors and operands as in grads_products, the 16x16 blocks read from dAb).
template <bool SEQ, int W>
__device__ __forceinline__ void loop_products_rk(LoopSmem& sm, int col, float scale,
                                                 const GradLane& g, GradOut& out,
                                                 const LaneOfs& o) {
    const int TW = 16 * W, c0 = 16 * col;
    const uint16_t* KTp = &sm.KT[0][0];
    const uint16_t* RTp = &sm.RT[0][0];
    float ddv[4];
    {
        const float4 d = lds_ld<float4>(&sm.dd[TW], o.q16);
        ddv[0] = d.x; ddv[1] = d.y; ddv[2] = d.z; ddv[3] = d.w;
    }
    // ---------------- dr ----------------
    f32x4 ar;
    {
        f32x4 tmp = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            tmp = mfma32(row8o(&sm.Dt[0][0], o, TW, 32 * ks), row8o(&sm.Sin[0][0], o, c0, 32 * ks), tmp);
        ar = tmp * lds_ld<float>(&sm.emu[W][0], o.tab);
    }
    constexpr int bW = (W * (W + 1)) / 2;
#pragma unroll
    for (int J = 0; J < W; ++J) {
        const f32x4 t2 = mfma16(lds_ld<bf16x4>(&sm.dAb[bW + J][0][0], o.blk), ch4o(KTp, o, 0, 16 * J), f32x4{});
        ar += (t2 * lds_ld<float>(&sm.kb[J][0], o.tab)) * lds_ld<float>(&sm.fp[(W * (W - 1)) / 2 + J][0], o.tab);
    }
    ar = mfma16(lds_ld<bf16x4>(&sm.dAb[bW + W][0][0], o.blk), ch4o(KTp, o, 0, TW), ar);
    float xr[4];
    {
        float d[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float sar = scale * ar[rr];
            d[rr] = g.Fm[0][rr] * sar + (g.ulane[0] * ddv[rr]) * (float)g.krw[0][rr];
            xr[rr] = (float)g.rmb[0][rr] * sar;
        }
        out.drb[0] = cvt4(d[0], d[1], d[2], d[3]);
    }
    // ---------------- dk ----------------
    f32x4 ak, ak2;
    {
        f32x4 tmp = {};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            tmp = mfma32(row8o(&sm.Vt[0][0], o, TW, 32 * ks), row8o(&sm.dS[0][0], o, c0, 32 * ks), tmp);
        ak = tmp * lds_ld<float>(&sm.eg[W][0], o.tab);
        float pk = 0.f;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) pk += (float)g.kmb[0][rr] * ak[rr];
        const RowSums rs = row_sums(pk);                  // the column's sum over the 4 rows
        if (o.q16 == 0) lds_st<float>(&sm.Pk[W][0], o.tab, rs.lo + rs.hi);
    }
    ak2 = mfma16(lds_tr(&sm.dAb[bW + W][0][0], o.blktr), ch4o(RTp, o, 0, TW), f32x4{});
#pragma unroll
    for (int I = W + 1; I < 4; ++I) {
        const f32x4 t2 = mfma16(lds_tr(&sm.dAb[(I * (I + 1)) / 2 + W][0][0], o.blktr), ch4o(RTp, o, 0, 16 * I), f32x4{});
        ak2 += (t2 * lds_ld<float>(&sm.fp[(I * (I - 1)) / 2 + W][0], o.tab)) * lds_ld<float>(&sm.kb[W][0], o.tab);
    }
    {
        float d[4], xv[4];
        out.dup[0] = 0.f;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float akr = ak[rr] + scale * ak2[rr];
            const float rv = (float)g.rrw[0][rr], kv = (float)g.krw[0][rr];
            d[rr] = g.Fk[0][rr] * akr + (g.ulane[0] * ddv[rr]) * rv;
            out.dup[0] += (rv * kv) * ddv[rr];
            const float y = -(float)g.kmb[0][rr] * akr;
            xv[rr] = xr[rr] + y;
            out.dwv[0][rr] = y;
            out.fl[rr] = !SEQ && g.Fm[0][rr] * g.Fk[0][rr] > FLOOR_FF;
        }
        out.dkb[0] = cvt4(d[0], d[1], d[2], d[3]);
        out.dwv[0][2] += xv[3];
        out.dwv[0][1] += xv[3] + xv[2];
        out.dwv[0][0] += (xv[3] + xv[2]) + xv[1];
        out.lt[0] = ((xv[3] + xv[2]) + xv[1]) + xv[0];
    }
}

// dv of the wave's token block W (compile-time) and value column 16 col + lr (the A blocks read
// from Ab).
template <int W>
__device__ __forceinline__ f32x4 loop_products_v(LoopSmem& sm, int col, const LaneOfs& o) {
    const int TW = 16 * W, c0 = 16 * col;
    f32x4 av = {}, ab = {};          // 16x16x32 and 16x16x16 products in separate accumulators
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
        av = mfma32(tr8o(&sm.KtT[0][0], o, 32 * ks, TW), tr8o(&sm.dS[0][0], o, 32 * ks, c0), av);
    ab = mfma16(lds_ld<bf16x4>(&sm.Ab[(W * (W + 1)) / 2 + W][0][0], o.frag), tr4o(&sm.Dt[0][0], o, TW, c0), ab);
#pragma unroll
    for (int I = W + 1; I < 4; ++I)
        ab = mfma16(lds_ld<bf16x4>(&sm.Ab[(I * (I + 1)) / 2 + W][0][0], o.frag), tr4o(&sm.Dt[0][0], o, 16 * I, c0), ab);
    return av + ab;
}

// The raw pieces of one chunk a thread moves into LDS: thread (row, c4) = (tid >> 4,
// 4 (tid & 15)) holds token `row` of r, k, v, w, dO at channels c4 .. c4+3 and row i = row of
// S_in.
struct LoopPrefetch {
    uint2 r, k, v, w, d, s;
};

// Byte offsets of a thread's global pieces within a chunk, formed once per launch and passed
// through an empty asm every chunk like LaneOfs: an address is then the chunk's wave-uniform
// base (scalar registers) plus one of these, the base + 32-bit offset form of the vector
// memory instructions, with no 64-bit address arithmetic per chunk.
//   tok: token row `row` = tid >> 4 of r, k, v, w at channels c4 = 4 (tid & 15)
//   hd:  the same row of a head-first tensor (dO) and of the S_in tile
//   st:  token 16 (wv & 3) + lr, channels 8 lq of a gradient (the stores of loop_store)
// With B*H <= 65535 (check_shape) a token row is at most 8 MB, so every offset fits an int.
struct GlobOfs {
    int tok, hd, st;
};
template <bool SEQ>
__device__ __forceinline__ GlobOfs glob_ofs(int tid, int B, int H) {
    const int row = tid >> 4, c4 = (tid & 15) * 4, rs = (int)tok_rs<SEQ>(B, H);
    const int wv = tid >> 6, lane = tid & 63;
    GlobOfs g;
    g.tok = (row * rs + c4) * 2;
    g.hd = (row * KD + c4) * 2;
    g.st = ((16 * (wv & 3) + (lane & 15)) * rs + 8 * (lane >> 4)) * 2;
    return g;
}
__device__ __forceinline__ void launder(GlobOfs& g) {
    asm volatile("" : "+v"(g.tok), "+v"(g.hd), "+v"(g.st));
}
template <class T>
__device__ __forceinline__ T gld(const void* base, int bytes) {
    return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + (unsigned)bytes);
}

// Part PART (0: r, k; 1: v, w; 2: dO, S_in) of the loads of chunk c.  The three parts go out
// in three phases of the step before, so the vector-memory issue of the 16 waves does not
// pile up in one phase.
template <bool SEQ, int PART>
__device__ __forceinline__ void loop_issue(LoopPrefetch& f, const uint16_t* __restrict__ r,
                                           const uint16_t* __restrict__ k,
                                           const uint16_t* __restrict__ v,
                                           const uint16_t* __restrict__ w,
                                           const uint16_t* __restrict__ dO,
                                           const uint16_t* __restrict__ Hs, int bh, int c, int B,
                                           int H, int T, int NT, int tid, const GlobOfs& g) {
    const int t0 = c * CL, nvalid = min(CL, T - t0);
    // unconditional loads (rows past a ragged end read the last token and are zeroed when
    // stored): a load under a branch makes the next wait a full one
    int otok = g.tok, ohd = g.hd;
    if (nvalid < CL) {
        const int lrow = min(tid >> 4, nvalid - 1), c4 = (tid & 15) * 4;
        otok = (lrow * (int)tok_rs<SEQ>(B, H) + c4) * 2;
        ohd = (lrow * KD + c4) * 2;
    }
    const size_t base = tok_base<SEQ>(bh, t0, B, H, T);
    if (PART == 0) {
        f.r = gld<uint2>(r + base, otok);
        f.k = gld<uint2>(k + base, otok);
    } else if (PART == 1) {
        f.v = gld<uint2>(v + base, otok);
        f.w = gld<uint2>(w + base, otok);
    } else {
        f.d = gld<uint2>(dO + ((size_t)bh * T + t0) * KD, ohd);
        f.s = gld<uint2>(Hs + ((size_t)bh * (NT + 1) + c) * KD * KD, g.hd);
    }
}

// The staged gradients of chunk c to HBM: the waves of token block N (N = W of wave 4W + col)
// write tensor N (dr, dk, dv, dw), wave col the tokens 16 col .. 16 col + 15.
//   head-first (Out channel-major): lane (lq, lr) writes token 16 col + lr, channels 8 lq .. +7
//     and 32 + 8 lq .. +7 (the token rows are contiguous: each store covers 1 KB);
//   sequence-first (Out token-major): lane (rw, cg) = (lane >> 3, lane & 7) writes tokens
//     16 col + rw and + 8, channels 8 cg .. +7, so a store covers 128 contiguous bytes of 8
//     token rows B*H*128 bytes apart (16 rows of 64 bytes there stream ~1.3x slower); rows
//     past the end store the last token's values again (no branch around the stores).
template <bool SEQ, int N>
__device__ __forceinline__ void loop_store(const LoopSmem& sm, uint16_t* __restrict__ dr,
                                           uint16_t* __restrict__ dk, uint16_t* __restrict__ dv,
                                           uint16_t* __restrict__ dw, int bh, int c, int B, int H,
                                           int T, int col, int lane, const LaneOfs& o,
                                           const GlobOfs& g) {
    const int t0 = c * CL, nvalid = min(CL, T - t0);
    uint16_t* dst = (N == 0 ? dr : N == 1 ? dk : N == 2 ? dv : dw) + tok_base<SEQ>(bh, t0, B, H, T);
    if constexpr (SEQ) {
        const int rw = lane >> 3, c8 = 8 * (lane & 7);
        const size_t rs = tok_rs<SEQ>(B, H);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int tk = min(16 * col + rw + 8 * kk, nvalid - 1);
            const uint4 x = *reinterpret_cast<const uint4*>(&sm.Out[N][tk][c8]);
            *reinterpret_cast<uint4*>(dst + (size_t)tk * rs + c8) = x;
        }
    } else {
        const int tk = 16 * col + (lane & 15);
        const uint4 x0 = __builtin_bit_cast(uint4, g8o(&sm.Out[N][0][0], o, 0, 0));   // o.g8 holds c0
        const uint4 x1 = __builtin_bit_cast(uint4, g8o(&sm.Out[N][0][0], o, 32, 0));
        if (tk < nvalid) {
            char* p = reinterpret_cast<char*>(dst) + (unsigned)g.st;
            *reinterpret_cast<uint4*>(p) = x0;
            *reinterpret_cast<uint4*>(p + 64) = x1;
        }
    }
}

// Sum over aligned groups of 16 lanes (a DPP row); all 16 lanes get the same bits.
__device__ __forceinline__ float sum16lanes(float v) {
    v = sum8lanes(v);
    return v + dpp_mov<0x140>(v);                 // row_mirror: lane i <-> lane 15 - i
}

// The chunk walk of one wave of wkv6_bwd_loop, for its token block W (a compile-time constant:
// the cross-block loops, the block-dependent tables and every offset that depends on W are
// resolved at compile time; the wave runs this one instantiation for the whole launch, and all
// four have the same barriers).  col = the wave's channel column.
template <bool SEQ, int W>
__device__ __forceinline__ void bwd_loop_walk(
        LoopSmem& sm, const uint16_t* __restrict__ r, const uint16_t* __restrict__ k,
        const uint16_t* __restrict__ v, const uint16_t* __restrict__ w,
        const uint16_t* __restrict__ dO, const uint16_t* __restrict__ Hs,
        uint16_t* __restrict__ dr, uint16_t* __restrict__ dk, uint16_t* __restrict__ dv,
        uint16_t* __restrict__ dw, float scale, int B, int H, int T, int NT, int bh, int c_lo,
        int c_hi, LaneOfs o, GlobOfs go_, LoopPrefetch& pf, GradLane& gl, f32x4& Dst,
        float& du_acc) {
    constexpr int TW = 16 * W;
    for (int c = c_hi - 1; c >= c_lo; --c) {
        // The offsets and the lane indices come from opaque copies made in every iteration
        // (see LaneOfs): nothing derived from them is hoisted out of the walk.
        launder(o);
        launder(go_);
        int tid;
        asm volatile("" : "=v"(tid) : "0"((int)threadIdx.x));
        const int lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int col = wv & 3, lr = lane & 15, lq = lane >> 4;
        const int c0 = 16 * col, t4 = TW + 4 * lq;
        const int row = tid >> 4;                           // the thread's raw pieces: row
                                                            // (at byte o.th of a tile)
        const int t0 = c * CL, nvalid = min(CL, T - t0);
        // ---- S1: the raw pieces into LDS, the bonus, dd, dS_out(c) as a bf16 tile ----
        {
            LoopPrefetch x = pf;
            if (nvalid < CL) {             // the ragged last chunk only: a wave-uniform branch
                asm volatile("");          // (no per-chunk selects)
                if (row >= nvalid) {
                    const uint2 z = make_uint2(0u, 0u);
                    x.r = x.k = x.v = x.w = x.d = z;
                }
            }
            lds_st<uint2>(&sm.Vt[0][0], o.th, x.v);
            lds_st<uint2>(&sm.Dt[0][0], o.th, x.d);
            lds_st<uint2>(&sm.RT[0][0], o.th, x.r);
            lds_st<uint2>(&sm.KT[0][0], o.th, x.k);
            lds_st<uint2>(&sm.KtT[0][0], o.th, x.w);          // w scratch
            lds_st<uint2>(&sm.Sin[0][0], o.th, x.s);
            float rf[4], kf[4], ub[4];
            unpack4(x.r, rf);
            unpack4(x.k, kf);
            {
                const float4 uu = lds_ld<float4>(&sm.uh[0], 4 * (o.tab - 4 * c0));   // u[4 L .. 4 L + 3]
                ub[0] = uu.x; ub[1] = uu.y; ub[2] = uu.z; ub[3] = uu.w;
            }
            float b = (rf[0] * ub[0]) * kf[0];
#pragma unroll
            for (int s = 1; s < 4; ++s) b += (rf[s] * ub[s]) * kf[s];
            b = sum16lanes(b);
            const float e = sum16lanes(dot4_bf16(x.d, x.v));
            if (lr == 0) {
                sm.bonus[row] = b;
                sm.dd[row] = e;
            }
            const float d4[4] = {Dst[0], Dst[1], Dst[2], Dst[3]};
            st_ch4o(&sm.dS[0][0], o, 0, t4 - 4 * lq, d4);
        }
        // the next chunk's loads (past chunk 0 they reload chunk 0) go out in S2, S3 and S4,
        // the stores of the chunk before in S4
        const int cn = max(c - 1, c_lo);
        __syncthreads();

        // ---- S2: dA blocks; raw r, k, w at the lane's positions; the decay scan; Fm, Fk; Rm,
        // Km; Dv ----
        loop_issue<SEQ, 0>(pf, r, k, v, w, dO, Hs, bh, cn, B, H, T, NT, tid, go_);
        if (W < 2 || (W == 2 && col < 2)) loop_dA_block(sm, wv, o, lane);
        bf16x4 wrw;
        float kmf[4], rmf[4], qloc, m7;
        {
            gl.rrw[0] = tr4o(&sm.RT[0][0], o, TW, c0);         // x[16W + 4lq + s][ch]
            gl.krw[0] = tr4o(&sm.KT[0][0], o, TW, c0);
            wrw = tr4o(&sm.KtT[0][0], o, TW, c0);
            float cs[4], run = 0.f;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                float x = (float)wrw[rr];
                if (SEQ) x = t4 + rr < nvalid ? -ex2(x * RW_L2E) : 0.f;   // w = -exp(decay), :336
                run += fmaxf(x, W_MIN) * RW_L2E;
                cs[rr] = run;
            }
            // prefix over the four lane rows: row 0 run_0, row 1 run_0 + run_1, row 2 (run_0 +
            // run_1) + run_2, row 3 (run_0 + run_1) + (run_2 + run_3)
            const RowSums rs = row_sums(run);
            const float xi = ((lq & 1) ? rs.pair : run) + (lq >= 2 ? rs.lo : 0.f);
            const float excl = xi - run;
            const float tot = rs.lo + rs.hi;                    // the block's total
            m7 = rs.lo;                                         // G at token 16W+7
            qloc = tot - m7;                                    // b_W - mu_W
            if (lq == 0) {
                lds_st<float>(&sm.red[W][0], o.tab, tot);
                lds_st<float>(&sm.red[4 + W][0], o.tab, m7);
            }
            float rm[4], km[4];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                gl.Fm[0][rr] = ex2(excl + (rr ? cs[rr - 1] : 0.f) - m7);
                gl.Fk[0][rr] = ex2(m7 - (excl + cs[rr]));
                rm[rr] = (float)gl.rrw[0][rr] * gl.Fm[0][rr];
                km[rr] = (float)gl.krw[0][rr] * gl.Fk[0][rr];
                kmf[rr] = km[rr];
                rmf[rr] = rm[rr];
            }
            gl.rmb[0] = cvt4(rm[0], rm[1], rm[2], rm[3]);
            gl.kmb[0] = cvt4(km[0], km[1], km[2], km[3]);
        }
        {   // Dv[i] = sum_j S_in[i][j] dS[i][j], i = row
            const float x = sum16lanes(dot4_bf16(lds_ld<uint2>(&sm.Sin[0][0], o.th),
                                                 lds_ld<uint2>(&sm.dS[0][0], o.th)));
            if (lr == 0) sm.Dv[row] = x;
        }
        __syncthreads();                   // raw r, k, w read; block totals and mu in `red`

        // ---- S3: operand tiles (channel-major), the state-gradient operand, the tables ----
        loop_issue<SEQ, 1>(pf, r, k, v, w, dO, Hs, bh, cn, B, H, T, NT, tid, go_);
        {
            lds_st<bf16x4>(&sm.RT[0][0], o.ch + tb(0, TW), gl.rmb[0]);
            lds_st<bf16x4>(&sm.KT[0][0], o.ch + tb(0, TW), gl.kmb[0]);
            float after = 0.f, before = 0.f, tJs[4];            // G_63 - b_W, b_{W-1}
#pragma unroll
            for (int J = 0; J < 4; ++J) {
                tJs[J] = lds_ld<float>(&sm.red[J][0], o.tab);
                if (J > W) after += tJs[J];
                if (J < W) before += tJs[J];
            }
            const float eg = ex2(after + qloc), kq = ex2(qloc);
            float x[4];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) x[rr] = kmf[rr] * eg;
            st_ch4o(&sm.KtT[0][0], o, 0, TW, x);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) x[rr] = kmf[rr] * kq;
            st_ch4o(&sm.KqT[0][0], o, 0, TW, x);
            // s r e^{G_{t-1}} = s r Fm e^{mu_W}, mu_W = b_{W-1} + (G at 16W+7 within the block)
            const float emw = scale * ex2(before + m7);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) x[rr] = (float)gl.rrw[0][rr] * (gl.Fm[0][rr] * emw);
            st_ch4o(&sm.RiT[0][0], o, 0, TW, x);
            // the pair tiles of the block as the later one: s Rm_W p_WJ, p_WJ = e^{mu_W - b_J}
            float bJ = 0.f;
#pragma unroll
            for (int J = 0; J < W; ++J) {
                bJ += tJs[J];
                const float pfac = scale * ex2(before + m7 - bJ);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) x[rr] = rmf[rr] * pfac;
                constexpr int pbase = (W * (W - 1)) / 2;
                const int pi = pbase + J;
                st_ch4o(&sm.RpT[pi >> 2][0][0], o, 0, 16 * (pi & 3), x);
            }
        }
        {
            // tables per channel i = lane from the block totals and mu: b_J = G[16J+15],
            // mu_J = b_{J-1} + m7_J; each wave fills one or two rows
            const int i = lane;
            float bnd[4], mu[4], a = 0.f;
#pragma unroll
            for (int J = 0; J < 4; ++J) {
                mu[J] = a + sm.red[4 + J][i];
                a += sm.red[J][i];
                bnd[J] = a;
            }
            if (W == 0) {
                sm.emu[col][i] = ex2(col == 0 ? mu[0] : col == 1 ? mu[1] : col == 2 ? mu[2] : mu[3]);
            } else if (W == 1) {
                sm.eg[col][i] = ex2(bnd[3] - (col == 0 ? mu[0] : col == 1 ? mu[1] : col == 2 ? mu[2] : mu[3]));
            } else if (W == 2) {
                if (col < 3) {
                    sm.kb[col][i] = ex2(col == 0 ? bnd[0] - mu[0] : col == 1 ? bnd[1] - mu[1] : bnd[2] - mu[2]);
                } else {
                    sm.fp[0][i] = ex2(mu[1] - bnd[0]);          // (1, 0)
                    sm.fp[1][i] = ex2(mu[2] - bnd[0]);          // (2, 0)
                }
            } else {
                if (col == 0) {
                    sm.fp[2][i] = ex2(mu[2] - bnd[1]);          // (2, 1)
                    sm.fp[3][i] = ex2(mu[3] - bnd[0]);          // (3, 0)
                } else if (col == 1) {
                    sm.fp[4][i] = ex2(mu[3] - bnd[1]);          // (3, 1)
                    sm.fp[5][i] = ex2(mu[3] - bnd[2]);          // (3, 2)
                } else if (col == 2) {
                    const float e = ex2(bnd[3]);
                    sm.eG63[i] = e;
                    sm.Dv[i] *= e;
                }
            }
        }
        __syncthreads();

        // ---- S4: the products (dr, dk finished on the way), the state-gradient step ----
        if (c + 1 < c_hi) loop_store<SEQ, W>(sm, dr, dk, dv, dw, bh, c + 1, B, H, T, col, lane, o, go_);
        loop_issue<SEQ, 2>(pf, r, k, v, w, dO, Hs, bh, cn, B, H, T, NT, tid, go_);
        if (W < 2 || (W == 2 && col < 2)) loop_A_block(sm, wv, scale, o, lane);
        GradOut go;
        loop_products_rk<SEQ, W>(sm, col, scale, gl, go, o);
        {
            const float e = lds_ld<float>(&sm.eG63[0], o.tab);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) Dst[rr] *= e;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                Dst = mfma32(tr8o(&sm.Dt[0][0], o, 32 * ks, TW), dir8o(&sm.RiT[0][0], o, 0, 32 * ks), Dst);
        }
        du_acc += go.dup[0];
        __syncthreads();                   // A blocks in
        go.av[0] = loop_products_v<W>(sm, col, o);
        // dw: the suffix sums across the four lane rows (shuffles on all lanes)
        float later;
        {
            const float lt = go.lt[0];
            const RowSums rs = row_sums(lt);                    // sum over lq' >= lq:
            const float vsum = ((lq & 1) ? lt : rs.pair) + (lq < 2 ? rs.hi : 0.f);
            later = vsum - lt;
            if (lq == 0) lds_st<float>(&sm.red[W][0], o.tab, vsum);   // the wave's total
        }
        __syncthreads();                   // all products done; red, Pk in

        // ---- S5: dw; dr, dk, dv, dw staged (stored during the next step) ----
        {
            later += lds_ld<float>(&sm.Dv[0], o.tab) +
                     ((lds_ld<float>(&sm.Pk[0][0], o.tab) + lds_ld<float>(&sm.Pk[1][0], o.tab)) +
                      (lds_ld<float>(&sm.Pk[2][0], o.tab) + lds_ld<float>(&sm.Pk[3][0], o.tab)));
#pragma unroll
            for (int W2 = W + 1; W2 < 4; ++W2) later += lds_ld<float>(&sm.red[W2][0], o.tab);
            float g[4];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                g[rr] = go.dwv[0][rr] + later;
                // a floored token's gradient is 0 (the derivative of the floored forward)
                if (SEQ && t4 + rr < nvalid) {
                    const float wn = -ex2((float)wrw[rr] * RW_L2E);
                    g[rr] = wn < W_MIN ? 0.f : g[rr] * wn;
                }
                if (!SEQ && go.fl[rr]) g[rr] = 0.f;
            }
            if constexpr (SEQ) {
                // token-major (the store's row layout): X[TW + 4 lq + rr][c0 + lr], 2 bytes each
                const int tm = o.q16 * TS / 2 + (o.tab >> 1) + tb(TW, 0);   // X[TW + 4 lq][c0 + lr]
                auto st_tok = [&](uint16_t* X, bf16x4 x) {
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        lds_st<__bf16>(X, tm + tb(rr, 0), x[rr]);
                };
                st_tok(&sm.Out[0][0][0], go.drb[0]);
                st_tok(&sm.Out[1][0][0], go.dkb[0]);
                st_tok(&sm.Out[2][0][0], cvt4(go.av[0][0], go.av[0][1], go.av[0][2], go.av[0][3]));
                st_tok(&sm.Out[3][0][0], cvt4(g[0], g[1], g[2], g[3]));
            } else {
                lds_st<bf16x4>(&sm.Out[0][0][0], o.ch + tb(0, TW), go.drb[0]);
                lds_st<bf16x4>(&sm.Out[1][0][0], o.ch + tb(0, TW), go.dkb[0]);
                const float avf[4] = {go.av[0][0], go.av[0][1], go.av[0][2], go.av[0][3]};
                st_ch4o(&sm.Out[2][0][0], o, 0, TW, avf);
                st_ch4o(&sm.Out[3][0][0], o, 0, TW, g);
            }
        }
        // no barrier here: the next step's S1 touches nothing S5 reads or writes, and its B1
        // orders S5 before the next writes of Dv, red (S2) and Pk, Out (S4)
    }
    __syncthreads();
    {
        const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        loop_store<SEQ, W>(sm, dr, dk, dv, dw, bh, c_lo, B, H, T, wv & 3, threadIdx.x & 63, o, go_);
    }
}

// SEQ as for wkv6_bwd_chunk_grads.  One workgroup per (b,h, segment) (P segments of ceil(NT/P)
// chunks; P = 1 when B*H fills the device): segment p starts from dhT (p = P-1) or dSend[b,h][p]
// (wkv6_bwd_fold) and writes dh0 if p = 0.  du_part gets one 64-vector per (b,h, segment)
// ([h][b][p][i]).  The 16 waves: wave 4W + col owns token block W and channel column col.
template <bool SEQ>
__global__ void __launch_bounds__(NTHR_L)
wkv6_bwd_loop(const uint16_t* __restrict__ r, const uint16_t* __restrict__ k,
              const uint16_t* __restrict__ v, const uint16_t* __restrict__ w,
              const void* __restrict__ u, int u_dtype, const uint16_t* __restrict__ dO,
              const float* __restrict__ dhT, const uint16_t* __restrict__ Hs,
              uint16_t* __restrict__ dr, uint16_t* __restrict__ dk, uint16_t* __restrict__ dv,
              uint16_t* __restrict__ dw, float* __restrict__ du_part, float* __restrict__ dh0,
              const float* __restrict__ dSend, float scale, int B, int H, int T, int NT, int P) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
    LoopSmem& sm = *reinterpret_cast<LoopSmem*>(smem_raw);
    // workgroup = (b,h, segment): chunks [c_lo, c_hi) of the sequence, walked from the last
    const int bh = blockIdx.x / P, seg = blockIdx.x - bh * P, h = bh % H;
    const int NC = (NT + P - 1) / P, c_lo = seg * NC, c_hi = min(NT, c_lo + NC);
    const size_t sbase = (size_t)bh * KD * KD;
    // the lane's channel ch0 = 16 col + lr and first token t40 = 16 W + 4 lq
    const int ch0 = 16 * ((threadIdx.x >> 6) & 3) + (threadIdx.x & 15);
    const int t40 = 16 * (threadIdx.x >> 8) + 4 * ((threadIdx.x >> 4) & 3);
    LaneOfs o = lane_ofs(threadIdx.x & 63, threadIdx.x >> 6);
    GlobOfs go_ = glob_ofs<SEQ>(threadIdx.x, B, H);

    LoopPrefetch pf;
    loop_issue<SEQ, 0>(pf, r, k, v, w, dO, Hs, bh, c_hi - 1, B, H, T, NT, threadIdx.x, go_);
    loop_issue<SEQ, 1>(pf, r, k, v, w, dO, Hs, bh, c_hi - 1, B, H, T, NT, threadIdx.x, go_);
    loop_issue<SEQ, 2>(pf, r, k, v, w, dO, Hs, bh, c_hi - 1, B, H, T, NT, threadIdx.x, go_);
    if (threadIdx.x < KD) sm.uh[threadIdx.x] = load_u(u, u_dtype, h * KD + threadIdx.x);
    __syncthreads();
    GradLane gl;
    gl.ulane[0] = scale * load_u(u, u_dtype, h * KD + ch0);
    f32x4 Dst = {};                                         // dS[ch][t4 + rr]
    {
        // dhT for the last segment, else what the later segments hand this one
        const float* d0 = seg + 1 < P ? dSend + ((size_t)bh * (P - 1) + seg) * KD * KD
                                      : (dhT ? dhT + sbase : nullptr);
        if (d0) {
            const float4 x = *reinterpret_cast<const float4*>(d0 + ch0 * KD + t40);
            Dst[0] = x.x; Dst[1] = x.y; Dst[2] = x.z; Dst[3] = x.w;
        }
    }
    float du_acc = 0.f;
    switch (__builtin_amdgcn_readfirstlane(threadIdx.x >> 8)) {
    case 0:
        bwd_loop_walk<SEQ, 0>(sm, r, k, v, w, dO, Hs, dr, dk, dv, dw, scale, B, H, T, NT, bh, c_lo,
                              c_hi, o, go_, pf, gl, Dst, du_acc);
        break;
    case 1:
        bwd_loop_walk<SEQ, 1>(sm, r, k, v, w, dO, Hs, dr, dk, dv, dw, scale, B, H, T, NT, bh, c_lo,
                              c_hi, o, go_, pf, gl, Dst, du_acc);
        break;
    case 2:
        bwd_loop_walk<SEQ, 2>(sm, r, k, v, w, dO, Hs, dr, dk, dv, dw, scale, B, H, T, NT, bh, c_lo,
                              c_hi, o, go_, pf, gl, Dst, du_acc);
        break;
    default:
        bwd_loop_walk<SEQ, 3>(sm, r, k, v, w, dO, Hs, dr, dk, dv, dw, scale, B, H, T, NT, bh, c_lo,
                              c_hi, o, go_, pf, gl, Dst, du_acc);
        break;
    }
    // du over the sequence: lanes of one channel (lq), then the four token blocks in order
    {
        const RowSums rs = row_sums(du_acc);
        if (((threadIdx.x >> 4) & 3) == 0) sm.red[4 + (threadIdx.x >> 8)][ch0] = rs.lo + rs.hi;
    }
    if (dh0 && seg == 0)
        *reinterpret_cast<float4*>(dh0 + sbase + ch0 * KD + t40) = make_float4(Dst[0], Dst[1], Dst[2], Dst[3]);
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < KD) {
        const float acc = (sm.red[4][tid] + sm.red[5][tid]) + (sm.red[6][tid] + sm.red[7][tid]);
        du_part[(((size_t)h * B + bh / H) * P + seg) * KD + tid] = scale * acc;
    }
}

// T = 0: dh0 = dhT (zero without one), du = 0 (a kernel rather than a memset node, so the
// call can be captured in a graph).
__global__ void __launch_bounds__(256)
wkv6_bwd_empty(const float* __restrict__ dhT, float* __restrict__ dh0, void* __restrict__ du,
               int u_dtype, int n_state, int n_u) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (dh0 && i < n_state) dh0[i] = dhT ? dhT[i] : 0.f;
    if (i < n_u) {
        if (u_dtype == RWKV6_BF16) reinterpret_cast<uint16_t*>(du)[i] = 0;
        else reinterpret_cast<float*>(du)[i] = 0.f;
    }
}

// du[h][i] = sum_b sum_c du_part[h,b,c,i].  One block per head over its contiguous B*NT*64
// partials: thread t adds the float4 pieces t, t + 1024, ... (channels 4 (t & 15) .. +3; all
// its loads in flight together); the four lanes of a wave with the same quad, then the 16
// waves, are added in a fixed order (deterministic).
#define DU_THR 1024
__global__ void __launch_bounds__(DU_THR)
wkv6_du_reduce(const float* __restrict__ du_part, void* __restrict__ du, int u_dtype, int B,
               int H, int NT) {
    __shared__ float4 part[DU_THR / 64][16];
    const int h = blockIdx.x, t = threadIdx.x;
    const float4* src = reinterpret_cast<const float4*>(du_part + (size_t)h * B * NT * KD);
    const int n4 = B * NT * (KD / 4);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int k = t;
    for (; k + 7 * DU_THR < n4; k += 8 * DU_THR) {
        float4 x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = src[k + j * DU_THR];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc.x += x[j].x; acc.y += x[j].y; acc.z += x[j].z; acc.w += x[j].w;
        }
    }
    for (; k < n4; k += DU_THR) {
        const float4 x = src[k];
        acc.x += x.x; acc.y += x.y; acc.z += x.z; acc.w += x.w;
    }
    // within the wave: lanes j, j + 16, j + 32, j + 48 hold quad j (fixed-order exchanges)
    acc.x += lane_xor_swz<16>(acc.x); acc.y += lane_xor_swz<16>(acc.y);
    acc.z += lane_xor_swz<16>(acc.z); acc.w += lane_xor_swz<16>(acc.w);
    acc.x += lane_xor32(acc.x); acc.y += lane_xor32(acc.y);
    acc.z += lane_xor32(acc.z); acc.w += lane_xor32(acc.w);
    if ((t & 63) < 16) part[t >> 6][t & 15] = acc;
    __syncthreads();
    if (t < 16) {
        float4 tot = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < DU_THR / 64; ++j) {
            const float4 x = part[j][t];
            tot.x += x.x; tot.y += x.y; tot.z += x.z; tot.w += x.w;
        }
        const float v[4] = {tot.x, tot.y, tot.z, tot.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (u_dtype == RWKV6_BF16) reinterpret_cast<uint16_t*>(du)[h * KD + 4 * t + e] = f2bf(v[e]);
            else reinterpret_cast<float*>(du)[h * KD + 4 * t + e] = v[e];
        }
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

// The forward's workspace: the pre-pass pieces' end states S_q (fp32 [64][64]) and total
// log2-decays A_q (fp32 [64]), at most max_pieces pieces, then the start states of segments
// 1..P-1 (fp32 [64][64] each).
// The reverse walk's workspace: du partials per (b,h, segment), then (P > 1) the backward
// pieces' dS_q and A_q and the segments' starting state gradients dS_end.
inline size_t bwd_walk_workspace_bytes(int64_t BH, int64_t NT) {
    const int P = bwd_walk_segments(BH, NT);
    size_t n = round_up((size_t)(BH * P) * KD * 4);
    if (P > 1) {
        const size_t np = (size_t)(BH * (P - 1) * prepass_pieces(BH, NT, P, PIECE_TARGET).sub);
        n += round_up(np * KD * KD * 4) + round_up(np * KD * 4) + round_up((size_t)(BH * (P - 1)) * KD * KD * 4);
    }
    return n;
}
inline size_t fwd_workspace_bytes(int64_t BH, int64_t NT, int64_t max_pieces) {
    const int P = walk_segments(BH, NT);
    const size_t n = (size_t)(BH * (P - 1) * prepass_pieces(BH, NT, P, max_pieces).sub);
    const size_t starts = (size_t)(BH * (P - 1)) * KD * KD * 4;
    return std::max<size_t>(256, round_up(n * KD * KD * 4) + round_up(n * KD * 4) + round_up(starts));
}

}  // namespace

extern "C" {

size_t rwkv6_wkv_saved_bytes(int64_t B, int64_t H, int64_t T, int64_t K, int64_t V) {
    if (check_shape(B, H, T, K, V) != RWKV6_OK) return 0;
    const int64_t NT = nchunks(T);
    return round_up((size_t)(B * H) * (NT + 1) * KD * KD * 2);        // bf16 S_in per chunk + final
}

size_t rwkv6_wkv_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                                 int for_bwd) {
    if (check_shape(B, H, T, K, V) != RWKV6_OK) return 0;
    const size_t BH = (size_t)(B * H), NT = (size_t)(nchunks(T) > 0 ? nchunks(T) : 1);
    if (!for_bwd) return fwd_workspace_bytes((int64_t)BH, nchunks(T), PIECE_TARGET);
    if (bwd_walk_segments((int64_t)BH, nchunks(T))) return bwd_walk_workspace_bytes((int64_t)BH, nchunks(T));
    // dHs, du_part per chunk, dS_loc, dec
    return 2 * round_up(BH * NT * KD * KD * 2) + 2 * round_up(BH * NT * KD * 4);
}

}  // extern "C"

namespace {

constexpr int kMaxDevices = 64;

// The device a call's kernels run on: the stream's, or the current one for the NULL stream.
int stream_device(hipStream_t stream, int* dev, int* cur) {
    if (hipGetDevice(cur) != hipSuccess) return RWKV6_ERR_LAUNCH;
    *dev = *cur;
    if (stream) {
        hipDevice_t d = 0;
        if (hipStreamGetDevice(stream, &d) != hipSuccess) return RWKV6_ERR_INVALID_ARG;
        *dev = d;
    }
    return (*dev < 0 || *dev >= kMaxDevices) ? RWKV6_ERR_UNSUPPORTED : RWKV6_OK;
}

// Per-device set-up that is done once it has succeeded, with that device current: a failed
// attempt is not cached, the next call tries again.  After the first success a call costs one
// atomic load.  Set-up runs host API calls (attribute and symbol queries, no allocation); a
// caller that captures the library's launches into a HIP graph makes one eager call on the
// device first, so that none of it runs under capture.
struct DeviceOnce {
    std::mutex m;
    std::atomic<bool> done{false};
};
template <class F>
int device_once(DeviceOnce& slot, int dev, int cur, F&& body) {
    if (slot.done.load(std::memory_order_acquire)) return RWKV6_OK;
    std::lock_guard<std::mutex> lock(slot.m);
    if (slot.done.load(std::memory_order_relaxed)) return RWKV6_OK;
    hipError_t e = dev == cur ? hipSuccess : hipSetDevice(dev);
    if (e == hipSuccess) e = body();
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess) return RWKV6_ERR_LAUNCH;
    slot.done.store(true, std::memory_order_release);
    return RWKV6_OK;
}

// The dynamic-LDS limit of every kernel here that takes more than 64 KB, raised once per
// device instead of on every call.
DeviceOnce g_lds_attr[kMaxDevices];

int lds_attributes(hipStream_t stream) {
    int dev = 0, cur = 0;
    int st = stream_device(stream, &dev, &cur);
    if (st != RWKV6_OK) return st;
    return device_once(g_lds_attr[dev], dev, cur, [] {
        struct Lds {
            const void* fn;
            size_t bytes;
        };
        const Lds list[] = {
            {reinterpret_cast<const void*>(wkv6_fwd_walk<false>), sizeof(WalkSmem)},
            {reinterpret_cast<const void*>(wkv6_fwd_walk<true>), sizeof(WalkSmem)},
            {reinterpret_cast<const void*>(wkv6_bwd_loop<false>), sizeof(LoopSmem)},
            {reinterpret_cast<const void*>(wkv6_bwd_loop<true>), sizeof(LoopSmem)},
            {reinterpret_cast<const void*>(wkv6_bwd_chunk_grads<false>), sizeof(GradSmem)},
            {reinterpret_cast<const void*>(wkv6_bwd_chunk_grads<true>), sizeof(GradSmem)},
        };
        hipError_t e = hipSuccess;
        for (const Lds& x : list)
            if (e == hipSuccess)
                e = hipFuncSetAttribute(x.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)x.bytes);
        return e;
    });
}

// max_pieces bounds the pre-pass pieces (the workspace's capacity): PIECE_TARGET for a
// workspace sized by rwkv6_wkv_workspace_bytes, the scratch array's capacity without one.
template <bool SEQ>
int wkv_fwd_impl(const void* r, const void* k, const void* v, const void* w, const void* u,
                 int u_dtype, const float* h0, void* o, float* hT, void* saved, void* workspace,
                 int64_t B, int64_t H, int64_t T, int64_t K, int64_t V, float scale,
                 void* stream, void* const* phase_events, int64_t max_pieces = PIECE_TARGET) {
    int st = check_shape(B, H, T, K, V);
    if (st != RWKV6_OK) return st;
    if (u_dtype != RWKV6_F32 && u_dtype != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    if (!u || !saved || (T > 0 && (!r || !k || !v || !w || !o || !workspace)))
        return RWKV6_ERR_INVALID_ARG;
    if (!al16(r) || !al16(k) || !al16(v) || !al16(w) || !al16(u) || !al16(o) || !al16(saved) ||
        !al16(workspace) || (h0 && !al16(h0)) || (hT && !al16(hT)))
        return RWKV6_ERR_ALIGNMENT;
    {
        const size_t act = (size_t)(B * H * T) * KD * 2, st = (size_t)(B * H) * KD * KD * 4;
        const size_t ub = (size_t)H * KD * (u_dtype == RWKV6_BF16 ? 2 : 4);
        if (any_alias({{o, act}, {hT, st}, {saved, rwkv6_wkv_saved_bytes(B, H, T, K, V)},
                       {workspace, fwd_workspace_bytes(B * H, nchunks(T), max_pieces)}},
                      {{r, act}, {k, act}, {v, act}, {w, act}, {u, ub}, {h0, st}}))
            return RWKV6_ERR_INVALID_ARG;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t NT = nchunks(T);
    const int BH = (int)(B * H);
    const int P = walk_segments(BH, NT);
    const Pieces pc = prepass_pieces(BH, NT, P, max_pieces);
    const int npieces = (P - 1) * pc.sub;                  // per sequence
    uint16_t* Hs = reinterpret_cast<uint16_t*>(saved);
    float* Sseg = reinterpret_cast<float*>(workspace);
    float* Aseg = reinterpret_cast<float*>(reinterpret_cast<char*>(Sseg) +
                                           round_up((size_t)BH * npieces * KD * KD * 4));
    float* Sstart = reinterpret_cast<float*>(reinterpret_cast<char*>(Aseg) +
                                             round_up((size_t)BH * npieces * KD * 4));
    if ((st = lds_attributes(s)) != RWKV6_OK) return st;
    mark(phase_events, 0, s);
    if (P > 1) {
        hipLaunchKernelGGL((wkv6_fwd_pieces<SEQ>), dim3((unsigned)(BH * npieces)), dim3(NTHR_W), 0, s,
                           (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)w, Sseg, Aseg,
                           (int)B, (int)H, (int)T, (int)NT, (int)((NT + P - 1) / P), pc.sub, pc.ncs,
                           npieces);
        hipLaunchKernelGGL(wkv6_fwd_fold, dim3((unsigned)(BH * (KD * KD / FOLD_THR))), dim3(FOLD_THR), 0,
                           s, Sseg, Aseg, h0, Sstart, npieces, pc.sub, P);
    }
    mark(phase_events, 1, s);
    mark(phase_events, 2, s);
    mark(phase_events, 3, s);
    mark(phase_events, 4, s);
    hipLaunchKernelGGL((wkv6_fwd_walk<SEQ>), dim3((unsigned)(BH * P)), dim3(NTHR_W),
                       sizeof(WalkSmem), s, (const uint16_t*)r, (const uint16_t*)k,
                       (const uint16_t*)v, (const uint16_t*)w, u, u_dtype, h0, (uint16_t*)o, Hs,
                       hT, Sstart, scale, (int)B, (int)H, (int)T, (int)NT, P);
    mark(phase_events, 5, s);
    return launch_status();
}

template <bool SEQ>
int wkv_bwd_impl(const void* r, const void* k, const void* v, const void* w, const void* u,
                 int u_dtype, const void* dO, const float* dhT, const void* saved, void* dr,
                 void* dk, void* dv, void* dw, void* du, float* dh0, void* workspace, int64_t B,
                 int64_t H, int64_t T, int64_t K, int64_t V, float scale, void* stream,
                 void* const* phase_events) {
    int st = check_shape(B, H, T, K, V);
    if (st != RWKV6_OK) return st;
    if (u_dtype != RWKV6_F32 && u_dtype != RWKV6_BF16) return RWKV6_ERR_INVALID_ARG;
    if (!u || !du || !saved || !workspace ||
        (T > 0 && (!r || !k || !v || !w || !dO || !dr || !dk || !dv || !dw)))
        return RWKV6_ERR_INVALID_ARG;
    if (!al16(r) || !al16(k) || !al16(v) || !al16(w) || !al16(u) || !al16(dO) || !al16(saved) ||
        !al16(dr) || !al16(dk) || !al16(dv) || !al16(dw) || !al16(workspace) ||
        (dhT && !al16(dhT)) || (dh0 && !al16(dh0)))
        return RWKV6_ERR_ALIGNMENT;
    {
        const size_t act = (size_t)(B * H * T) * KD * 2, st = (size_t)(B * H) * KD * KD * 4;
        const size_t ub = (size_t)H * KD * (u_dtype == RWKV6_BF16 ? 2 : 4);
        if (any_alias({{dr, act}, {dk, act}, {dv, act}, {dw, act}, {du, ub}, {dh0, st},
                       {workspace, rwkv6_wkv_workspace_bytes(B, H, T, K, V, 1)}},
                      {{r, act}, {k, act}, {v, act}, {w, act}, {u, ub}, {dO, act}, {dhT, st},
                       {saved, rwkv6_wkv_saved_bytes(B, H, T, K, V)}}))
            return RWKV6_ERR_INVALID_ARG;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if ((st = lds_attributes(s)) != RWKV6_OK) return st;
    const int64_t NT = nchunks(T);
    const int BH = (int)(B * H);
    const uint16_t* Hs = reinterpret_cast<const uint16_t*>(saved);
    const size_t NTa = (size_t)(NT > 0 ? NT : 1);
    uint16_t* dHs = reinterpret_cast<uint16_t*>(workspace);
    float* du_part = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) +
                                              round_up((size_t)BH * NTa * KD * KD * 2));
    mark(phase_events, 0, s);
    if (NT == 0) {                          // T = 0: dh0 = dhT, du = 0
        const int n = std::max<int>(BH * KD * KD, (int)H * KD);
        hipLaunchKernelGGL(wkv6_bwd_empty, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dhT,
                           dh0, du, u_dtype, BH * KD * KD, (int)H * KD);
        for (int i = 1; i <= 7; ++i) mark(phase_events, i, s);
        return launch_status();
    }
    if (const int P = bwd_walk_segments(BH, NT)) {
        // one reverse walk per (b,h, segment): gradients and state gradients in one pass; with
        // P > 1 segments the pieces of segments 1..P-1 and their fold first give each segment
        // its starting state gradient
        du_part = reinterpret_cast<float*>(workspace);
        const float* dSend = nullptr;
        if (P > 1) {
            const Pieces pc = prepass_pieces(BH, NT, P, PIECE_TARGET);
            const int npieces = (P - 1) * pc.sub;
            float* dSp = reinterpret_cast<float*>(reinterpret_cast<char*>(du_part) +
                                                  round_up((size_t)BH * P * KD * 4));
            float* Ap = reinterpret_cast<float*>(reinterpret_cast<char*>(dSp) +
                                                 round_up((size_t)BH * npieces * KD * KD * 4));
            float* dSe = reinterpret_cast<float*>(reinterpret_cast<char*>(Ap) +
                                                  round_up((size_t)BH * npieces * KD * 4));
            hipLaunchKernelGGL((wkv6_bwd_pieces<SEQ>), dim3((unsigned)(BH * npieces)), dim3(NTHR_W), 0,
                               s, (const uint16_t*)r, (const uint16_t*)w, (const uint16_t*)dO, dSp, Ap,
                               scale, (int)B, (int)H, (int)T, (int)NT, (int)((NT + P - 1) / P),
                               pc.sub, pc.ncs, npieces);
            mark(phase_events, 1, s);
            mark(phase_events, 2, s);
            hipLaunchKernelGGL(wkv6_bwd_fold, dim3((unsigned)(BH * (KD * KD / FOLD_THR))), dim3(FOLD_THR),
                               0, s, dSp, Ap, dhT, dSe, npieces, pc.sub, P);
            dSend = dSe;
        } else {
            mark(phase_events, 1, s);
            mark(phase_events, 2, s);
        }
        mark(phase_events, 3, s);
        mark(phase_events, 4, s);
        hipLaunchKernelGGL(wkv6_bwd_loop<SEQ>, dim3((unsigned)(BH * P)), dim3(NTHR_L), sizeof(LoopSmem), s,
                           (const uint16_t*)r, (const uint16_t*)k, (const uint16_t*)v,
                           (const uint16_t*)w, u, u_dtype, (const uint16_t*)dO, dhT, Hs,
                           (uint16_t*)dr, (uint16_t*)dk, (uint16_t*)dv, (uint16_t*)dw, du_part, dh0,
                           dSend, scale, (int)B, (int)H, (int)T, (int)NT, P);
        mark(phase_events, 5, s);
        mark(phase_events, 6, s);
        hipLaunchKernelGGL(wkv6_du_reduce, dim3((unsigned)H), dim3(DU_THR), 0, s, du_part, du, u_dtype,
                           (int)B, (int)H, P);
        mark(phase_events, 7, s);
        return launch_status();
    }
    // chunk-parallel state gradients, then the gradient kernel over all (chunk, b,h)
    uint16_t* dSloc = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(du_part) +
                                                  round_up((size_t)BH * NTa * KD * 4));
    float* dec = reinterpret_cast<float*>(reinterpret_cast<char*>(dSloc) +
                                          round_up((size_t)BH * NTa * KD * KD * 2));
    hipLaunchKernelGGL(wkv6_bwd_chunk_dstate<SEQ>, dim3((unsigned)NT, (unsigned)BH), dim3(NTHR), 0,
                       s, (const uint16_t*)r, (const uint16_t*)dO, (const uint16_t*)w, dSloc, dec,
                       scale, (int)B, (int)H, (int)T, (int)NT);
    mark(phase_events, 1, s);
    mark(phase_events, 2, s);
    hipLaunchKernelGGL(wkv6_state_scan_bwd, dim3((unsigned)BH * SCAN_BLK), dim3(NTHR), 0, s, dSloc,
                       dec, dhT, dHs, dh0, (int)NT);
    mark(phase_events, 3, s);
    mark(phase_events, 4, s);
    hipLaunchKernelGGL(wkv6_bwd_chunk_grads<SEQ>, dim3((unsigned)NT, (unsigned)BH), dim3(NTHR_G),
                       sizeof(GradSmem), s, (const uint16_t*)r, (const uint16_t*)k,
                       (const uint16_t*)v, (const uint16_t*)w, u, u_dtype, (const uint16_t*)dO, Hs,
                       (const uint16_t*)dHs, (uint16_t*)dr, (uint16_t*)dk, (uint16_t*)dv,
                       (uint16_t*)dw, du_part, scale, (int)B, (int)H, (int)T, (int)NT);
    mark(phase_events, 5, s);
    mark(phase_events, 6, s);
    hipLaunchKernelGGL(wkv6_du_reduce, dim3((unsigned)H), dim3(DU_THR), 0, s, du_part, du, u_dtype,
                       (int)B, (int)H, (int)NT);
    mark(phase_events, 7, s);
    return launch_status();
}

}  // namespace

// ---------------------------------------------------------------------------
// forward without a workspace argument
// ---------------------------------------------------------------------------
// For callers that cannot allocate (code under HIP graph capture, tight serving loops): the
// forward's only scratch, the end states of its pre-pass pieces (S_q fp32 [64][64] and A_q
// fp32 [64] per piece) and the segments' start states (fp32 [64][64] per segment after the
// first), lives in this file-scope device array instead of the caller's workspace.
// walk_segments() gives B*H*P <= 256 when P > 1, so B*H*(P-1) < 256, and
// this entry caps the pieces at WKV_SCRATCH_SEGS (fewer, longer pieces than with a workspace
// when the cap binds): WKV_SCRATCH_BYTES covers every shape.
// Each GPU holds its own copy for the life of the process; calls on one GPU share it (the
// last call's contents stay), so such calls must not overlap in time on one GPU.  Nothing in
// it has to start at zero: the pre-pass writes every piece state the output walk reads.
#define WKV_SCRATCH_SEGS 256
#define WKV_SCRATCH_BYTES ((size_t)WKV_SCRATCH_SEGS * (2 * KD * KD * 4 + KD * 4))
static __device__ __align__(256) unsigned char scratch[WKV_SCRATCH_BYTES];

namespace {

DeviceOnce g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the GPU that runs `stream` (the current device for the
// NULL stream).  Looked up once per device, with that device current (device_once); in host
// code the array's name is only a stand-in, never a device address.
int scratch_address(hipStream_t stream, void** out) {
    int dev = 0, cur = 0;
    int st = stream_device(stream, &dev, &cur);
    if (st != RWKV6_OK) return st;
    st = device_once(g_scratch_once[dev], dev, cur, [dev] {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess && !p) e = hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
        return e;
    });
    *out = st == RWKV6_OK ? g_scratch_ptr[dev] : nullptr;
    return st;
}

}  // namespace

extern "C" {

int rwkv6_wkv_fwd_noalloc(const void* r, const void* k, const void* v, const void* w,
                          const void* u, int u_dtype, const float* h0, void* o, float* hT,
                          void* saved, int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                          float scale, void* stream) {
    int st = check_shape(B, H, T, K, V);
    if (st != RWKV6_OK) return st;
    if (fwd_workspace_bytes(B * H, nchunks(T), WKV_SCRATCH_SEGS) > WKV_SCRATCH_BYTES)
        return RWKV6_ERR_UNSUPPORTED;
    void* ws = nullptr;
    if ((st = scratch_address(reinterpret_cast<hipStream_t>(stream), &ws)) != RWKV6_OK) return st;
    return wkv_fwd_impl<false>(r, k, v, w, u, u_dtype, h0, o, hT, saved, ws, B, H, T, K, V, scale,
                               stream, nullptr, WKV_SCRATCH_SEGS);
}

int rwkv6_wkv_fwd_ex(const void* r, const void* k, const void* v, const void* w, const void* u,
                     int u_dtype, const float* h0, void* o, float* hT, void* saved,
                     void* workspace, int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                     float scale, void* stream, void* const* phase_events) {
    return wkv_fwd_impl<false>(r, k, v, w, u, u_dtype, h0, o, hT, saved, workspace, B, H, T, K, V,
                               scale, stream, phase_events);
}

int rwkv6_wkv_bwd_ex(const void* r, const void* k, const void* v, const void* w, const void* u,
                     int u_dtype, const void* dO, const float* dhT, const void* saved, void* dr,
                     void* dk, void* dv, void* dw, void* du, float* dh0, void* workspace,
                     int64_t B, int64_t H, int64_t T, int64_t K, int64_t V, float scale,
                     void* stream, void* const* phase_events) {
    return wkv_bwd_impl<false>(r, k, v, w, u, u_dtype, dO, dhT, saved, dr, dk, dv, dw, du, dh0,
                               workspace, B, H, T, K, V, scale, stream, phase_events);
}

int rwkv6_wkv_fwd(const void* r, const void* k, const void* v, const void* w, const void* u,
                  int u_dtype, const float* h0, void* o, float* hT, void* saved,
                  void* workspace, int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                  float scale, void* stream) {
    return wkv_fwd_impl<false>(r, k, v, w, u, u_dtype, h0, o, hT, saved, workspace, B, H, T, K, V,
                               scale, stream, nullptr);
}

int rwkv6_wkv_bwd(const void* r, const void* k, const void* v, const void* w, const void* u,
                  int u_dtype, const void* dO, const float* dhT, const void* saved, void* dr,
                  void* dk, void* dv, void* dw, void* du, float* dh0, void* workspace,
                  int64_t B, int64_t H, int64_t T, int64_t K, int64_t V, float scale,
                  void* stream) {
    return wkv_bwd_impl<false>(r, k, v, w, u, u_dtype, dO, dhT, saved, dr, dk, dv, dw, du, dh0,
                               workspace, B, H, T, K, V, scale, stream, nullptr);
}

int rwkv6_wkv_fwd_seqfirst(const void* r, const void* k, const void* v, const void* decay,
                           const void* u, int u_dtype, const float* h0, void* o, float* hT,
                           void* saved, void* workspace, int64_t B, int64_t H, int64_t T,
                           int64_t K, int64_t V, float scale, void* stream) {
    return wkv_fwd_impl<true>(r, k, v, decay, u, u_dtype, h0, o, hT, saved, workspace, B, H, T, K,
                              V, scale, stream, nullptr);
}

int rwkv6_wkv_bwd_seqfirst(const void* r, const void* k, const void* v, const void* decay,
                           const void* u, int u_dtype, const void* dO, const float* dhT,
                           const void* saved, void* dr, void* dk, void* dv, void* d_decay,
                           void* du, float* dh0, void* workspace, int64_t B, int64_t H,
                           int64_t T, int64_t K, int64_t V, float scale, void* stream) {
    return wkv_bwd_impl<true>(r, k, v, decay, u, u_dtype, dO, dhT, saved, dr, dk, dv, d_decay, du,
                              dh0, workspace, B, H, T, K, V, scale, stream, nullptr);
}

}  // extern "C"
