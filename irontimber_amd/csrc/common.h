// Shared device helpers for the gfx950 kernels of this library.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rec_index.h"

namespace it {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// D = A(16x32) * B(32x16) + C on the matrix cores, f16 inputs, f32 accumulate (gfx950).
// Lane l holds A row (l & 15) and B column (l & 15), each with 8 consecutive k values of the
// lane's k-group (l >> 4); D element i of lane l is row 4*(l >> 4) + i, column l & 15.
__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// D = A(32x16) * B(16x32) + C; lane l holds A row / B column (l & 31) with 8 k values of k-group
// (l >> 5); D element i of lane l is row 8*(i/4) + 4*(l >> 5) + (i & 3), column l & 31.
__device__ __forceinline__ f16v mfma32x32x16(h8 a, h8 b, f16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16). Within each 16-lane group, source lane s points
// at 4 consecutive 16-bit values; result lane i, slot e is element (i & 3) of source lane 4e + i/4.
// With a row-major [row][col] tile and source lane s addressing &T[r0 + s/4][c0 + 4*(s & 3)], lane i
// receives T[r0 + e][c0 + i] for e = 0..3: four consecutive rows of one column.
// The lanes exchange data: issue it with the whole wave active (no divergent branch around it),
// and keep each 4-lane 32-byte segment 32-byte aligned (row pitch a multiple of 32 bytes).
typedef short s4v __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ h4 lds_tr4(const _Float16* p) {
    typedef __attribute__((address_space(3))) s4v lds_s4v;
    const s4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v*)(__attribute__((address_space(3))) char*)(p));
    return __builtin_bit_cast(h4, v);
}
__device__ __forceinline__ h8 cat_h4(h4 a, h4 b) { return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }

__device__ __forceinline__ h8 ld_h8(const void* p) { return __builtin_bit_cast(h8, *(const u4*)p); }
__device__ __forceinline__ f4 ld_f4(const float* p) { return *(const f4*)p; }
// 8 consecutive activations as two f4, from f32 or (16-byte aligned) f16 storage
__device__ __forceinline__ void ld8(const float* p, f4& a, f4& b) { a = ld_f4(p); b = ld_f4(p + 4); }
__device__ __forceinline__ void ld8(const _Float16* p, f4& a, f4& b) {
    const h8 h = ld_h8(p);
    a = f4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
    b = f4{(float)h[4], (float)h[5], (float)h[6], (float)h[7]};
}
// store 4 activations as f32 or f16 (round to nearest even)
__device__ __forceinline__ void st4(float* p, f4 y) { *(f4*)p = y; }
__device__ __forceinline__ void st4(_Float16* p, f4 y) {
    *(h4*)p = h4{(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
}

// Split 8 f32 values into f16 hi + f16 lo with hi + lo == x to ~2^-22 relative: two MFMAs with
// the halves reproduce an f32-accurate dot product against exact f16 operands.
__device__ __forceinline__ void split_hi_lo(f4 x0, f4 x1, h8& hi, h8& lo) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        _Float16 a = (_Float16)x0[j], b = (_Float16)x1[j];
        hi[j] = a; hi[j + 4] = b;
        lo[j] = (_Float16)(x0[j] - (float)a); lo[j + 4] = (_Float16)(x1[j] - (float)b);
    }
}
__device__ __forceinline__ h8 to_h8(f4 x0, f4 x1) {
    h8 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) { r[j] = (_Float16)x0[j]; r[j + 4] = (_Float16)x1[j]; }
    return r;
}

// Wave-wide max / sum of a float: DPP within 16-lane rows (xor 1, xor 2 by quad_perm, then the
// half-row and row mirrors), then the four row results through readlane. Every lane returns the
// full result; no LDS round trip.
template <int CTRL> __device__ __forceinline__ float dppc(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dppc<0xB1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dppc<0x4E>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dppc<0x141>(v));   // row_half_mirror
    v = fmaxf(v, dppc<0x140>(v));   // row_mirror
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dppc<0xB1>(v);
    v += dppc<0x4E>(v);
    v += dppc<0x141>(v);
    v += dppc<0x140>(v);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (a + b) + (c + d);
}

// An offset that is the same in every lane, moved into scalar registers: arithmetic on it stays on
// the scalar unit, and a kernel-argument pointer plus it plus a lane offset needs no 64-bit vector
// arithmetic (each wave64 vector instruction costs 4 cycles, a 64-bit multiply several). The
// pointer itself is not passed through an integer, which would lose its global address space.
__device__ __forceinline__ size_t uniform_off(size_t v) {
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return ((size_t)hi << 32) | lo;
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// s_waitcnt immediate that waits until at most N vector-memory operations of this wave are still
// outstanding, leaving the other counters alone. gfx9-family simm16 layout (gfx950 included):
// bits [3:0] vmcnt[3:0], [6:4] expcnt (7 = no wait), [11:8] lgkmcnt (15 = no wait),
// [15:14] vmcnt[5:4]. Used where a wait for the global->LDS copies must not also wait for LDS
// reads (the builtin __syncthreads() fence would wait for every counter).
#define IT_WAIT_VMCNT(N) __builtin_amdgcn_s_waitcnt((((N) & 15) | (((N) >> 4) << 14)) | 0x0F70)

// Lane exchanges written as inline asm: v_permlane16_swap_b32 / v_permlane32_swap_b32 swap the odd
// 16-lane rows (resp. the upper 32 lanes) of the first operand with the even rows (lower lanes) of
// the second, so with both holding v each lane sees its partner l ^ 16 (l ^ 32). Written out
// because the compiler folds the builtin's two results when both inputs are the same value, and
// kept off LDS (a ds_bpermute would make the next wait on LDS results also wait for every LDS
// operand read in flight).
// Hazard: the ISA requires two wait states between a VALU write of a VGPR and a permlane swap
// reading it, and the compiler's hazard recognizer does not look inside inline asm, so each swap
// carries its own "s_nop 1" (two wait states). A missing wait reads a stale register and breaks
// every reduction built on these helpers: the split-K records, the decode merge and the GDN
// L2 norms, all of which the GPU parity tests check against the oracle.
__device__ __forceinline__ void swap16(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// Two values reduced by one swap: fold16(a, b) returns, in the even 16-lane rows, a summed over
// the row pair (rows 0+1, 2+3) and, in the odd rows, b summed likewise; fold32(a, b) returns a
// summed over lanes l and l ^ 32 in the lower half and b in the upper half. Halves the swaps of a
// reduction of several values whose results may end up in different lanes.
__device__ __forceinline__ float fold16(float a, float b) { swap16(a, b); return a + b; }
__device__ __forceinline__ float fold32(float a, float b) { swap32(a, b); return a + b; }
// max / sum over lanes l and l ^ 32, and over l and l ^ 16
__device__ __forceinline__ float max_xor32(float v) { float a = v, b = v; swap32(a, b); return fmaxf(a, b); }
__device__ __forceinline__ float sum_xor32(float v) { float a = v, b = v; swap32(a, b); return a + b; }
__device__ __forceinline__ float max_xor16(float v) { float a = v, b = v; swap16(a, b); return fmaxf(a, b); }
__device__ __forceinline__ float sum_xor16(float v) { float a = v, b = v; swap16(a, b); return a + b; }

// Piece layout of the f32 split-K records (two-launch decode and verify whose merge is the wave
// merge, for the f16 and the f32 KV cache): the same values as the 260-word record, arranged for
// the merge, whose lane l reads split l of one (row, 16-dim block). O goes into 64-byte pieces
// [rows][16 blocks][smax][16 floats], so consecutive lanes read consecutive pieces, and {m, l} into
// [rows][smax] after them (rec_index.h: piece_o, piece_h).
__device__ __forceinline__ float* prec_o(float* part, int th, int db, int s, int smax) {
    return part + idx::piece_o(th, db, s, smax);
}
__device__ __forceinline__ float* prec_h(float* part, int rows, int th, int s, int smax) {
    return part + idx::piece_h(rows, th, s, smax);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
// The same on the hardware exp2 and reciprocal (a few ulp, ~1e-7 relative): for epilogues that apply
// the gate to many values per lane, where the accurate forms (~20 VALU ops each) dominate.
__device__ __forceinline__ float sigmoid_hw(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}
__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float softplusf_(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }
// SiLU, softplus and e^x on the hardware exp2 / log2 / reciprocal (a few ulp): for short serial
// chains with one wave per SIMD, where every instruction is on the critical path.
__device__ __forceinline__ float silu_hw(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}
__device__ __forceinline__ float softplus_hw(float x) {
    return x > 20.0f ? x : __builtin_amdgcn_logf(1.0f + __builtin_amdgcn_exp2f(x * 1.4426950408889634f)) *
                               0.6931471805599453f;
}
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

}  // namespace it
