/*
 * qmm_kernels.hip -- gfx950 (CDNA4) kernels for the small-M affine-quantised matmul
 *
 *     y[M,N] = x[M,K] . dequant(W)[N,K]^T      (+ optional linear bias)
 *
 * over MLX's affine format: W packed little-endian in uint32 words (4-bit: 8 codes per word,
 * 8-bit: 4), one scale and one bias per `gs` consecutive k (gs = 32, 64 or 128).  This is
 * the operation of DFlashKit's SmallMQuantizedMatmul (Sources/DFlashKit/
 * SmallMQuantizedMatmul.swift:54-165) designed for CDNA4 rather than translated from the
 * Metal kernel.  Built with --genco into a code object that the runtime loads with
 * hipModuleLoadData.
 *
 * Fast path (qmm_mt8 family, M <= 8)
 * ----------------------------------
 * Every weight byte is read from HBM once and reused by all M rows.  The dot product is
 * factored per quantisation group g:
 *
 *     y[m,n] = sum_g  s[n,g] * (sum_{k in g} x[m,k] q[n,k])  +  b[n,g] * (sum_{k in g} x[m,k])
 *
 * so the codes enter the matrix cores as exact small integers:
 *
 *  - 4-bit: a nibble q is turned into the 16-bit float (MAGIC + q) with one AND-OR
 *    ((p >> 4i) & 0x000F000F | 0x43004300 gives the bf16 pair 128+q_i, 128+q_{i+4}; fp16 uses
 *    0x6400, i.e. 1024+q).  Seven VALU ops make the 8-element MFMA operand of a word.
 *    The MFMA then returns sum x*(MAGIC+q); the epilogue removes MAGIC*sum(x) through
 *    the bias term:  acc += s*P + (b - MAGIC*s)*X.
 *  - 8-bit: v_cvt_f32_ubyte{0..3} + a pack to bf16/fp16 (exact for 0..255), no offset.
 *
 * The 16x16x32 MFMA has 16 columns (= 16 output features of W) and 16 rows, of which a
 * verify pass only needs 8.  The other 8 rows carry a second quantisation group: the A
 * operand (x) is block-diagonal -- rows 0-7 hold x for the k slots of lane groups 0-1, rows
 * 8-15 hold x for lane groups 2-3 -- and the B operand is arranged (with v_permlane16/32_swap
 * where the group size needs it) so that lanes 0-31 carry group a and lanes 32-63 group b.
 * One MFMA therefore produces two independent per-group partial sums and no MFMA work is
 * spent on padding rows.
 *
 * x (M rows of the k-block) is staged once per workgroup in LDS, pre-permuted into the MFMA
 * k order, with the per-group sums sum_{k in g} x[m,k] next to it.  Weights, scales and
 * biases stream straight from HBM into VGPRs through global loads (a scalar base plus a
 * 32-bit lane offset), one work unit in flight per wave at 4-bit g64.
 *
 * Work decomposition: see qmm_params.h.  One workgroup per CU (the LDS request keeps two
 * from sharing a CU) of 12 streaming waves, which take units of (16-column tile, chunk) from
 * an LDS counter, and one publisher wave, which writes finished tiles.
 *
 * Generic path (qmm_generic): the stock-op stand-in -- one wave per output element, plain
 * per-element dequantisation, W re-read for every row.  It exists so that the drop-in layer
 * has a fall-through for shapes outside the fast kernel's window, and so that tests can
 * prove the fast kernel really ran (its result is not bit-identical to this one).
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "qmm_params.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#ifndef DFQ_WAVES
#define DFQ_WAVES 12       /* streaming waves per workgroup; the host is built with the same value */
#endif
#ifndef DFQ_PF_LOADS
#define DFQ_PF_LOADS 4     /* 16-byte weight loads in flight per lane (4 KB per wave) */
#endif
constexpr int kWaves = DFQ_WAVES;
constexpr uint32_t kTileDone = 0x80000000u;  // tile counter value once its units are summed
constexpr uint32_t kTileOut = 0x80000001u;   // ... and once its publisher wave wrote it
constexpr int kThreads = kWaves * 64;        // streaming threads
#ifndef DFQ_PUBLISHERS
/* publisher waves per workgroup (one per SIMD); the host is built with the same value.  They
 * take the workgroup's tiles round-robin, so that several tiles' fix-ups (round trips through
 * the L2) overlap.  Measured on MI355X, M = 8, K = 5120: N = 17408 16.6 -> 15.7 us and
 * N = 5120 10.6 -> 9.6 us from one publisher to two.  From two to four, 8 rows stay within
 * 0.15 us at every shape, but 13..16 rows over two k-blocks, where every tile is exchanged,
 * gain (us, 4-bit g64, K = 5120): 16 rows N = 17408 18.16 -> 16.72, 13 rows 18.05 -> 16.59,
 * N = 34816 31.97 -> 27.82 (g128 33.49 -> 29.01), the gate|up epilogue 32.70 -> 28.34, the LM
 * head 115.4 -> 114.9; the 16-row verify forward 4,918 -> 4,613 us (8 rows 3,949 -> 3,953). */
#define DFQ_PUBLISHERS 4
#endif
constexpr int kPublishers = DFQ_PUBLISHERS;
constexpr int kBlock = kThreads + 64 * kPublishers;  // + the publisher waves
static_assert(kBlock <= 1024, "a workgroup holds at most 1024 threads");
/* x is staged by the first 8 waves only (two per SIMD).  A workgroup's waves start over
 * about 1 us, and staging is VALU-bound: spread over all 12 streaming waves, the last waves
 * to start finish it last and hold up the staging barrier.  With the late waves free of it
 * they only issue their first weights.  Measured on MI355X at M = 8 (us, against staging
 * on all 12 waves): N = 17408, K = 5120 15.16 against 15.44; gate|up N = 34816 23.25 against
 * 23.6; N = 5120, K = 17408 15.98 against 16.2; N = K = 5120 9.67 against 9.85; 16 rows at
 * N = 17408 18.62 against 18.84; one row and N = 7168 within noise; one row at N = K = 4096
 * (eight units a workgroup: the four waves with none fetch an unused unit, now ahead of the
 * staging waves' weights) 7.35 against 7.05. */
constexpr int kStageThreads = DFQ_STAGE_THREADS;
static_assert(kStageThreads == 8 * 64, "x is staged by the first eight waves");
static_assert(kThreads >= kStageThreads, "the staging waves are streaming waves");

/* The dynamic LDS block of a qmm_mt8 workgroup (its layout is fixed by the host plan). */
__device__ __forceinline__ uint8_t* lds_base() {
    extern __shared__ __attribute__((aligned(16))) uint8_t dfq_lds[];
    return dfq_lds;
}


/* ---------------------------------------------------------------------------------- */
/* Per-format constants                                                                */
/* ---------------------------------------------------------------------------------- */

template <int BITS, int GS>
struct Cfg {
    static_assert(BITS == 4 || BITS == 8, "bits");
    static_assert(GS == 32 || GS == 64 || GS == 128, "group size");
    static constexpr int KSTEP = 512 / BITS;  // k per row in one 64-byte step
    static constexpr int NS = (BITS == 4) ? (GS == 128 ? 2 : 1) : (GS / 32);  // steps/super-step
    static constexpr int KSS = KSTEP * NS;    // k per super-step
    static constexpr int GPS = KSS / GS;      // groups per super-step (4 or 2)
    static constexpr int NP = GPS / 2;        // partial accumulators per super-step
    static constexpr int NOPS = (BITS == 4) ? 4 * NS : 2 * NS;  // MFMA B operands
    static constexpr int NOW = (BITS == 4) ? NOPS : 2 * NOPS;   // operand words
    static constexpr int CPS = KSS / 8;       // 8-element chunks per super-step
    /* groups of a unit of the packed layout, and of the chunks the 1..8-row kernels take
     * where K allows: 8, one 16-byte scale load per lane; 16 for 4-bit group 32 (two loads,
     * the c16 kernels), so that a unit holds 4 KB of codes as at group 64 rather than 2 KB */
    static constexpr int CG = (BITS == 4 && GS == 32) ? 16 : 8;

    /* chunk index (within the super-step) read by lane group q for operand o is
     * base_chunk(q) + delta_chunk(o); the group (within the super-step) that lane group q
     * accumulates in partial p is group_of(p, q). */
    __device__ static constexpr int base_chunk(int q) {
        if (BITS == 4) {
            if (GS == 32) return 8 * (q >> 1) + (q & 1);
            if (GS == 64) return 4 * q;
            return 4 * q + 8 * (q >> 1);
        }
        if (GS == 32) return 2 * q;
        if (GS == 64) return 2 * q + 4 * (q >> 1);
        return 2 * q + 12 * (q >> 1);
    }
    __host__ __device__ static constexpr int delta_chunk(int o) {
        if (BITS == 4) {
            if (GS == 32) return (o == 0) ? 0 : (o == 1) ? 4 : (o == 2) ? 2 : 6;
            if (GS == 64) return o;
            return (o >> 2) * 8 + (o & 3);
        }
        if (GS == 32) return o;
        return (o >> 1) * 4 + (o & 1);
    }
    __host__ __device__ static constexpr int partial_of(int o) {
        return (BITS == 4 && GS == 32) ? (o & 1) : 0;
    }
    __device__ static constexpr int group_of(int p, int q) {
        return (BITS == 4 && GS == 32) ? 2 * (q >> 1) + p : (q >> 1);
    }
};

/* v_permlane16_swap / v_permlane32_swap with explicit wait states on both sides.  The
 * compiler (ROCm 7.2) pads the VALU-write -> swap-read side but not the swap-write ->
 * VALU-read side; a VALU op issued right after the swap has been seen to read the swapped
 * register's old contents on gfx950.  Semantics as the builtins: a is VDST, b is VSRC;
 * the 16-lane (32-lane) rows are exchanged between the two registers. */
__device__ __forceinline__ void permlane16_swap(uint32_t& a, uint32_t& b) {
    __asm__ volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 4" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(uint32_t& a, uint32_t& b) {
    __asm__ volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 4" : "+v"(a), "+v"(b));
}

/* Scales and biases arrive in one load: lane rows 0 and 2 (lane groups q = 0, 2) hold the
 * scale words, rows 1 and 3 the bias words of the same lane positions.  v_permlane16_swap of
 * the loaded value with a copy of itself exchanges the odd rows of the first with the even
 * rows of the second, leaving scales in every row of one and biases in every row of the
 * other.  All swaps share one wait-state pad on each side. */
__device__ __forceinline__ void split_scale_bias(uint32_t w, uint32_t& sw, uint32_t& bw) {
    sw = w;
    bw = w;
    __asm__ volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 4" : "+v"(sw), "+v"(bw));
}
__device__ __forceinline__ void split_scale_bias(u32x4_t w, u32x4_t& sv, u32x4_t& bv) {
    uint32_t s0 = w[0], s1 = w[1], s2 = w[2], s3 = w[3];
    uint32_t b0 = w[0], b1 = w[1], b2 = w[2], b3 = w[3];
    __asm__ volatile(
        "s_nop 1\n\t"
        "v_permlane16_swap_b32 %0, %4\n\t"
        "v_permlane16_swap_b32 %1, %5\n\t"
        "v_permlane16_swap_b32 %2, %6\n\t"
        "v_permlane16_swap_b32 %3, %7\n\t"
        "s_nop 4"
        : "+v"(s0), "+v"(s1), "+v"(s2), "+v"(s3), "+v"(b0), "+v"(b1), "+v"(b2), "+v"(b3));
    sv = u32x4_t{s0, s1, s2, s3};
    bv = u32x4_t{b0, b1, b2, b3};
}

/* Rearrange the raw words of one super-step (R[step][word], word j of lane group q covering
 * k chunk 4q+j (4-bit) / 2q+j/2 (8-bit)) so that lanes 0-31 of every operand hold one
 * quantisation group and lanes 32-63 another. */
template <int BITS, int GS>
__device__ __forceinline__ void build_operand_words(const u32x4_t (&R)[Cfg<BITS, GS>::NS],
                                                    uint32_t (&OW)[Cfg<BITS, GS>::NOW]) {
    if constexpr (BITS == 4 && GS == 32) {
        OW[0] = R[0][0]; OW[1] = R[0][1]; OW[2] = R[0][2]; OW[3] = R[0][3];
        permlane16_swap(OW[0], OW[1]);
        permlane16_swap(OW[2], OW[3]);
    } else if constexpr (BITS == 4 && GS == 64) {
#pragma unroll
        for (int j = 0; j < 4; ++j) OW[j] = R[0][j];
    } else if constexpr (BITS == 4 && GS == 128) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            OW[j] = R[0][j]; OW[4 + j] = R[1][j];
            permlane32_swap(OW[j], OW[4 + j]);
        }
    } else if constexpr (BITS == 8 && GS == 32) {
#pragma unroll
        for (int j = 0; j < 4; ++j) OW[j] = R[0][j];
    } else if constexpr (BITS == 8 && GS == 64) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            OW[j] = R[0][j]; OW[4 + j] = R[1][j];
            permlane32_swap(OW[j], OW[4 + j]);
        }
    } else {  // 8-bit, group 128
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            OW[j] = R[0][j]; OW[4 + j] = R[2][j]; OW[8 + j] = R[1][j]; OW[12 + j] = R[3][j];
            permlane32_swap(OW[j], OW[4 + j]);
            permlane32_swap(OW[8 + j], OW[12 + j]);
        }
    }
}

/* Operand words for the 16-row form: every MFMA operand holds one quantisation group in all
 * four lane groups, so that a full 16-row A operand (x rows 0-15) can be used.  The per-lane
 * form above holds one group per lane half (lane groups 0-1 / 2-3); exchanging the upper half
 * of the low lanes' words with the lower half of the high lanes' words (v_permlane32_swap:
 * VDST's lanes 32-63 <-> VSRC's lanes 0-31) gives the 16-row form.  Where the per-lane form
 * is itself that exchange of the loaded words (4-bit g128, 8-bit g64), the loaded words are
 * already in the 16-row form.  Operand o then reads, for lane group q, chunk
 * base_chunk((q & 1) + 2h) + (q >> 1) * delta_chunk(NOPS/2) + delta_chunk(o - h*NOPS/2) of the
 * super-step (h = o >= NOPS/2), and accumulates group group_of(partial_of(o), 2h). */
/* The 16-row form's chunk rule needs the second half of the operands to read the chunks of
 * the first half moved by one fixed delta, with the same partial index. */
template <class C>
__host__ __device__ constexpr bool wide_layout_holds() {
    for (int o = C::NOPS / 2; o < C::NOPS; ++o)
        if (C::delta_chunk(o) != C::delta_chunk(o - C::NOPS / 2) + C::delta_chunk(C::NOPS / 2) ||
            C::partial_of(o) != C::partial_of(o - C::NOPS / 2))
            return false;
    return true;
}

template <int BITS, int GS>
__device__ __forceinline__ void build_operand_words_wide(const u32x4_t (&R)[Cfg<BITS, GS>::NS],
                                                         uint32_t (&OW)[Cfg<BITS, GS>::NOW]) {
    using C = Cfg<BITS, GS>;
    if constexpr ((BITS == 4 && GS == 128) || (BITS == 8 && GS == 64)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            OW[j] = R[0][j];
            OW[4 + j] = R[1][j];
        }
    } else {
        build_operand_words<BITS, GS>(R, OW);
        constexpr int H = C::NOW / 2;
        if constexpr (H == 2) {
            __asm__ volatile(
                "s_nop 1\n\tv_permlane32_swap_b32 %0, %2\n\tv_permlane32_swap_b32 %1, %3\n\t"
                "s_nop 4"
                : "+v"(OW[0]), "+v"(OW[1]), "+v"(OW[2]), "+v"(OW[3]));
        } else {
#pragma unroll
            for (int h = 0; h < H; ++h) permlane32_swap(OW[h], OW[H + h]);
        }
    }
}

/* 8 nibbles of a word -> bf16/fp16 (MAGIC + q) pairs (q_i, q_{i+4}) in VGPR i: seven VALU
 * ops per word (three shifts, four v_and_or_b32).  gfx9 VOP3 takes no literal constant, so
 * with constant mask and magic the compiler would split each and-or into a v_and_b32 and a
 * v_or_b32 with literals; the caller passes both as opaque register values (mask in an SGPR,
 * magic in a VGPR, loop-invariant) and the compiler forms v_and_or_b32 itself.  It has to
 * be the compiler's instruction, not inline asm: the MFMA that reads the result needs wait
 * states after a VALU write, and the compiler only pads hazards it can see. */
template <bool F16>
__device__ __forceinline__ u32x4_t nibble_operand(uint32_t p, uint32_t mask, uint32_t magic) {
    u32x4_t v;
    v[0] = (p & mask) | magic;
    v[1] = ((p >> 4) & mask) | magic;
    v[2] = ((p >> 8) & mask) | magic;
    v[3] = ((p >> 12) & mask) | magic;
    return v;
}

template <bool F16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (F16) {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
    } else {
        /* exact: integers <= 255 have zero low mantissa bits, so truncation is exact */
        return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
    }
}

/* Two words of 4 bytes -> 8 exact 16-bit float codes in k order. */
template <bool F16>
__device__ __forceinline__ u32x4_t byte_operand(uint32_t a, uint32_t b) {
    u32x4_t v;
    v[0] = pack2<F16>((float)(a & 0xffu), (float)((a >> 8) & 0xffu));
    v[1] = pack2<F16>((float)((a >> 16) & 0xffu), (float)(a >> 24));
    v[2] = pack2<F16>((float)(b & 0xffu), (float)((b >> 8) & 0xffu));
    v[3] = pack2<F16>((float)((b >> 16) & 0xffu), (float)(b >> 24));
    return v;
}

template <bool F16>
__device__ __forceinline__ f32x4_t mfma(u32x4_t a, u32x4_t b, f32x4_t c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

/* 16-bit float held in the low (sh = 16) or high (sh = 0) half of a word -> fp32. */
template <bool F16>
__device__ __forceinline__ float half_of(uint32_t w, uint32_t sh_lo16) {
    if constexpr (F16) {
        uint32_t h = (w << sh_lo16) >> 16;
        return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    } else {
        return __uint_as_float((w << sh_lo16) & 0xffff0000u);
    }
}

/* Byte selectors for v_perm_b32(0, w, sel) that move the low (kSelLo) or high (kSelHi)
 * 16-bit half of w into the high half of the result, zeroing the low half: a bf16 half
 * becomes its fp32 value in one op even when the half is chosen per lane. */
constexpr uint32_t kSelLo = 0x01000c0cu;
constexpr uint32_t kSelHi = 0x03020c0cu;

/* 16-bit float in the half of w that `sel` (kSelLo / kSelHi) picks -> fp32. */
template <bool F16>
__device__ __forceinline__ float half_sel(uint32_t w, uint32_t sel) {
    const uint32_t h = __builtin_amdgcn_perm(0u, w, sel);
    if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(h >> 16));
    else return __uint_as_float(h);
}

template <bool F16>
__device__ __forceinline__ float elem_to_f32(uint32_t bits16) {
    if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
    else return __uint_as_float(bits16 << 16);
}

template <bool F16>
__device__ __forceinline__ uint16_t f32_to_out(float f) {
    if constexpr (F16) {
        return __builtin_bit_cast(uint16_t, (_Float16)f);
    } else {
        uint32_t u = __float_as_uint(f);
        if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
        u += 0x7fffu + ((u >> 16) & 1u);
        return (uint16_t)(u >> 16);
    }
}

/* s + the 8 elements of a 16-byte chunk, added pairwise in k order with v_dot2c against
 * (1, 1): four VALU ops per chunk.  Each element goes through a plain 32-bit temporary: the
 * builtin applied directly to an element of a 128-bit vector has been compiled (ROCm 7.2)
 * to read the vector's first register for every element.  It stays the compiler's own
 * instruction (not inline asm) so that the wait states a following DPP or MFMA read needs
 * are inserted. */
template <bool F16>
__device__ __forceinline__ float chunk_dot(u32x4_t v, float s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t e = v[i];
        if constexpr (F16)
            s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, e),
                                       __builtin_bit_cast(f16x2_t, 0x3c003c00u), s, false);
        else
            s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, e),
                                                __builtin_bit_cast(bf16x2_t, 0x3f803f80u), s,
                                                false);
    }
    return s;
}

/* v from another lane of the same 16-lane row (DPP control CTRL; lanes whose source is
 * outside the row read 0). */
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

/* (x0..x7) -> (x0,x4, x1,x5, x2,x6, x3,x7): the k order of a nibble operand. */
__device__ __forceinline__ u32x4_t nibble_permute(u32x4_t v) {
    u32x4_t o;
    o[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
    o[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
    o[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
    o[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
    return o;
}

#ifndef DFQ_XCD_ORDER
#define DFQ_XCD_ORDER 1
#endif
/* The range a workgroup takes.  Workgroup b of a launch runs on XCD b % 8 (MI355X deals
 * workgroups to its eight XCDs round-robin), and each XCD has its own L2.  Neighbouring ranges
 * share a tile, and with it the cache lines of that tile's scales and biases (and, in the MLX
 * layout, of its rows' codes at the chunk boundary); so XCD x takes one contiguous block of
 * ranges -- blocks of G / 8, the first G % 8 XCDs one more -- and a line two neighbours share
 * is fetched from HBM once, into one L2. */
__device__ __forceinline__ int xcd_order(int b, int G) {
    if (!DFQ_XCD_ORDER) return b;
    const int per = G >> 3, rem = G & 7, x = b & 7;
    return x * per + min(x, rem) + (b >> 3);
}

/* With p.xcd_pair (Gkb a multiple of 8): the i-th workgroup of XCD x takes range
 * x * Gkb / 8 + i / nkb of k-block i % nkb, so that the nkb parts of a tile (the same range
 * index in every k-block) run on one XCD. */
__device__ __forceinline__ int launch_order(const QmmParams& p, int b, int G) {
    if (!p.xcd_pair) return xcd_order(b, G);
    const int x = b & 7, i = b >> 3;
    const int kb = i % p.nkb;
    return kb * p.Gkb + x * (p.Gkb >> 3) + i / p.nkb;
}

/* The split of the U units of a k-block over G workgroups: workgroup c owns
 * [c*base + min(c, rem), +base + (c < rem)), with base = U / G and rem = U % G computed on
 * the host. */
__device__ __forceinline__ int wg_start(int c, int base, int rem) {
    return c * base + (c < rem ? c : rem);
}

/* Index of the workgroup (within the k-block) whose range holds unit u. */
__device__ __forceinline__ int owner_wg(int u, int base, int rem) {
    const int big = rem * (base + 1);
    return u < big ? u / (base + 1) : rem + (u - big) / base;
}

/* k-block kb holds chunks [c0, c0 + SS) of K (the chunks spread over the k-blocks with
 * sizes differing by at most one); its T*SS units go to the Gkb workgroups as above, or, in
 * an aligned split, its T tiles do (base and rem then count tiles, and a range is whole
 * tiles). */
struct KBlock {
    int c0, SS, base, rem;
    bool aligned;
};
__device__ __forceinline__ KBlock kblock(const QmmParams& p, int kb) {
    const int c0 = kb * p.chunks / p.nkb, c1 = (kb + 1) * p.chunks / p.nkb;
    const int SS = c1 - c0, U = p.aligned ? p.T : p.T * SS;
    return KBlock{c0, SS, U / p.Gkb, U % p.Gkb, p.aligned != 0};
}

/* First unit of workgroup c's range in k-block k. */
__device__ __forceinline__ int range_start(const KBlock& k, int c) {
    const int s = wg_start(c, k.base, k.rem);
    return k.aligned ? s * k.SS : s;
}

/* The first workgroup (within the k-block) whose range holds units of tile t, and how many
 * workgroups of the k-block hold its units (one in an aligned split). */
__device__ __forceinline__ int tile_first_owner(const KBlock& k, int t) {
    return k.aligned ? owner_wg(t, k.base, k.rem) : owner_wg(t * k.SS, k.base, k.rem);
}
__device__ __forceinline__ int tile_owners(const KBlock& k, int t) {
    return k.aligned ? 1 : owner_wg(t * k.SS + k.SS - 1, k.base, k.rem) -
                               owner_wg(t * k.SS, k.base, k.rem) + 1;
}

/* A partial tile (8*mt rows x 16 columns, fp32) is held by lanes 0 .. 32*mt-1: lane (q, n)
 * holds x rows 4q..4q+3 of column n.  In LDS and workspace slots it is laid out [mt][n][8]
 * (128 floats per row tile); tile_off gives a lane's four floats. */
__device__ __forceinline__ int tile_off(int lane) {
    return (lane >> 5) * 128 + (lane & 15) * 8 + ((lane >> 4) & 1) * 4;
}

/* Partial-tile slot j of k-block kb for tile t in the workspace: [T][nkb][nslot_kb][mt*128]
 * fp32, at the lane's four floats. */
__device__ __forceinline__ float* tile_slot(const QmmParams& p, int t, int kb, int j, int lane) {
    return p.slots + ((size_t)(t * p.nkb + kb) * p.nslot_kb + j) * p.mt * 128 + tile_off(lane);
}

__device__ __forceinline__ void put16(uint16_t* ptr, uint16_t v) { *ptr = v; }
__device__ __forceinline__ void put_tile4(float* ptr, f32x4_t v) { *(f32x4_t*)ptr = v; }

/* Keys of the greedy accept: the logit's bits made order-preserving (sign flip, or full
 * flip for negatives) in the high word and ~index in the low word, so the largest key is
 * the largest logit and, among equal logits, the first index (MLX's argMax); 0 = none. */
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)~(uint32_t)idx;
}

__device__ __forceinline__ uint64_t max_key_wave(uint64_t k) {
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)k, s, 64);
        const uint32_t hi = __shfl_xor((uint32_t)(k >> 32), s, 64);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        k = o > k ? o : k;
    }
    return k;
}

/* Folds output element (its rounded bits o, column col) into a row's running key; NaN is
 * skipped. */
template <bool F16>
__device__ __forceinline__ void fold_key(uint64_t& best, uint16_t o, int col) {
    const float f = elem_to_f32<F16>(o);
    if (f != f) return;
    const uint64_t k = argmax_key(f, col);
    best = k > best ? k : best;
}

/* silu(g) * u as the MLP activation computes it from a stored gate|up output: g and u
 * rounded to the output dtype first, then silu in fp32 and one rounding (the same
 * arithmetic as silu_mul below, so the fused epilogue is bit-identical to it). */
template <bool F16>
__device__ __forceinline__ uint16_t silu_mul_round(float g, float u) {
    const float gr = elem_to_f32<F16>(f32_to_out<F16>(g));
    const float ur = elem_to_f32<F16>(f32_to_out<F16>(u));
    return f32_to_out<F16>(gr / (1.0f + __expf(-gr)) * ur);
}

/* The gate|up epilogue (p.epi): the weight's rows are interleaved by 8, so tile t holds gate
 * columns 8t..8t+7 in its columns 0-7 and the matching up columns in 8-15; lane n < 8 takes
 * its up partner from lane n + 8 (DPP row_ror:8, every lane active) and writes h[m][8t+n]. */
template <bool F16>
__device__ __forceinline__ void store_h(const QmmParams& p, int t, int lane, f32x4_t v) {
    const int q = lane >> 4, n = lane & 15;
    float lb = 0.0f;
    if (p.lbias) lb = elem_to_f32<F16>(((const uint16_t*)p.lbias)[t * 16 + n]);
    f32x4_t u;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        v[r] += lb;
        u[r] = dpp_f32<0x128>(v[r]);
    }
    if (lane >= 32 * p.mt || n >= 8) return;
    const int H = p.N / 2;
    uint16_t* h = (uint16_t*)p.y;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * q + r;
        if (m < p.M) put16(h + (size_t)m * H + t * 8 + n, silu_mul_round<F16>(v[r], u[r]));
    }
}

/* Tile t as held by the lanes, plus the linear bias, to y; in greedy-accept mode (AM, the
 * kernels built for dfq_qmm_argmax_accept) also folded into the lane's keys of rows
 * 4q..4q+3 (best), and y may be NULL. */
template <bool F16, bool AM = false>
__device__ __forceinline__ void store_y(const QmmParams& p, int t, int lane, f32x4_t v,
                                        uint64_t (&best)[4]) {
    if (p.epi) {
        store_h<F16>(p, t, lane, v);
        return;
    }
    const int q = lane >> 4, n = lane & 15;
    const int col = t * 16 + n;
    if (lane >= 32 * p.mt || col >= p.N) return;
    float lb = 0.0f;
    if (p.lbias) lb = elem_to_f32<F16>(((const uint16_t*)p.lbias)[col]);
    uint16_t* y = (uint16_t*)p.y;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * q + r;
        if (m >= p.M) continue;
        const uint16_t o = f32_to_out<F16>(v[r] + lb);
        if (!AM || y) put16(y + (size_t)m * p.N + col, o);
        if constexpr (AM) fold_key<F16>(best[r], o, col);
    }
}

/* Scopes of the exchange atomics: device (agent) scope is coherent across the XCDs' L2s, so
 * the atomics are performed past them, in memory; between workgroups on one XCD the L2 they
 * share performs them (workgroup scope: not written through to memory). */
constexpr int kDeviceScope = __HIP_MEMORY_SCOPE_AGENT;
/* Levels of the exchange tree of an aligned split: up to 8 k-blocks (the host plan's most) */
constexpr int kTreeLevels = 3;
constexpr int kL2Scope = __HIP_MEMORY_SCOPE_WORKGROUP;

/* Two fp32 values in one 64-bit exchange word, each as the bitwise complement of its bits, so
 * that a word is zero only when empty: both values would have to be 0xFFFFFFFF, a NaN
 * payload that bf16/fp16 arithmetic does not produce and that is mapped to another NaN. */
__device__ __forceinline__ uint64_t pair_word(float a, float b) {
    uint32_t x = __float_as_uint(a), y = __float_as_uint(b);
    if (x == 0xFFFFFFFFu) x = 0xFFC00000u;
    if (y == 0xFFFFFFFFu) y = 0xFFC00000u;
    return (uint64_t)~x | ((uint64_t)~y << 32);
}
__device__ __forceinline__ float pair_value(uint64_t w, int e) {
    return __uint_as_float(~(uint32_t)(w >> (32 * e)));
}

/* One two-party exchange of the plain path at the words sl[0..1] (two elements each), for
 * the words with go[h] set: the party that gets back a non-zero word adds the other's pair
 * into w, zeroes the word and keeps go[h]; the other clears go[h]. */
template <int SCOPE>
__device__ __forceinline__ void pair_exchange(uint64_t* sl, bool (&go)[2], f32x4_t& w) {
    uint64_t old[2] = {0, 0};
#pragma unroll
    for (int h = 0; h < 2; ++h)
        if (go[h])
            old[h] = __hip_atomic_exchange(sl + h, pair_word(w[2 * h], w[2 * h + 1]),
                                           __ATOMIC_RELAXED, SCOPE);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        go[h] = old[h] != 0;
        if (!go[h]) continue;
        w[2 * h] += pair_value(old[h], 0);
        w[2 * h + 1] += pair_value(old[h], 1);
        __hip_atomic_store(sl + h, 0ull, __ATOMIC_RELAXED, SCOPE);
    }
}

/* The gate|up epilogue of the 1..8-row kernels, which needs g and u of one element summed by
 * the same party, on the lanes that hold g (with u taken from the partner lane): each pair of
 * elements has a g word sg[h] and a u word su[h].  u goes in first; once that has completed,
 * g is exchanged, and the party that gets back a non-zero g word finishes: the other's u is
 * in its u word by then (deposited before the other's g), or came back from our own u
 * exchange (then our u sits in the word and is cleared).  The 16-row form (publish) measured
 * 0.3 us slower here (24.6 against 24.3 us at 8 rows, 2 x 17408 x 5120, where only the tiles
 * cut by a range are exchanged). */
template <int SCOPE>
__device__ __forceinline__ void pair_exchange_gu(uint64_t* sg, uint64_t* su, bool (&go)[2],
                                                 f32x4_t& g, f32x4_t& u) {
    uint64_t ou[2] = {0, 0}, og[2] = {0, 0};
#pragma unroll
    for (int h = 0; h < 2; ++h)
        if (go[h])
            ou[h] = __hip_atomic_exchange(su + h, pair_word(u[2 * h], u[2 * h + 1]),
                                          __ATOMIC_RELAXED, SCOPE);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int h = 0; h < 2; ++h)
        if (go[h])
            og[h] = __hip_atomic_exchange(sg + h, pair_word(g[2 * h], g[2 * h + 1]),
                                          __ATOMIC_RELAXED, SCOPE);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        go[h] = og[h] != 0;
        if (!go[h]) continue;
        uint64_t upw;
        if (ou[h]) {
            upw = ou[h];
            __hip_atomic_store(su + h, 0ull, __ATOMIC_RELAXED, SCOPE);
        } else {
            upw = __hip_atomic_exchange(su + h, 0ull, __ATOMIC_RELAXED, SCOPE);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            g[2 * h + e] += pair_value(og[h], e);
            u[2 * h + e] += pair_value(upw, e);
        }
        __hip_atomic_store(sg + h, 0ull, __ATOMIC_RELAXED, SCOPE);
    }
}

/* Contribute a partial tile to the workspace.
 *
 * Two contributors (the usual case: a tile split between two workgroups): every two
 * elements of the tile share a 64-bit word of the tile's slot, each held as the bitwise
 * complement of its fp32 bits, zero at rest.  Each contributor swaps its pair in with one
 * atomic exchange; whoever gets back a non-zero word arrived second, adds the two values
 * (fp32 addition of two terms does not depend on their order), writes those y elements and
 * zeroes the word.  One round trip, no counter.  Two values per word instead of a tag and
 * one value halve the device-scope atomics and resets: the headline call measured 15.87 ->
 * 15.58 us, N = 1024 (every tile exchanged) 7.86 -> 7.64 us.
 *
 * Three or more contributors in an aligned split (whole tiles per workgroup, one part per
 * k-block): the parts meet over a binary tree of the k-blocks, one exchange per internal node
 * (see publish), and the second arrival at the root writes y.  For three: k-blocks 0 and 1
 * exchange at the tile's first word set, and whoever completes a word carries the pair's sum
 * into the second set, where k-block 2's part waits or arrives; the sum is (A + B) + C
 * whatever the order of arrival, so the result does not depend on timing.  This replaces the
 * second pass of such splits: the down projection (M=8, N=5120, K=17408) measured
 * 18.3-18.5 -> 16.9-17.1 us.
 *
 * Other tiles with more contributors belong to reduce splits, which store their parts with no
 * round trip and leave the sum to the second pass (a per-tile arrival counter here costs
 * the publisher two memory round trips per tile under full HBM load, which made such
 * splits 1.7-2.2x slower than the second pass).
 *
 * The workspace is zero again when the kernel ends.  Workgroups on different XCDs exchange
 * these partials: every access to a slot is an agent-scope atomic (coherent across the
 * XCDs' L2s without a whole-cache write-back or invalidate). */
template <bool F16, int MT, bool AM>
__device__ __forceinline__ void publish(const QmmParams& p, const KBlock& kbk, int t, int kb,
                                        int lane, f32x4_t v, uint64_t (&best)[4]) {
    const int q = lane >> 4, n = lane & 15;
    const bool act = lane < 32 * p.mt;  // lanes holding the tile
    const int nwg = tile_owners(kbk, t);
    const uint32_t total = (uint32_t)(p.nkb * nwg);
    /* one part: stored by the caller; more than two outside an aligned split: reduce splits */
    const bool chain = total >= 3 && p.aligned;
    if (total != 2 && !chain) return;
    /* the tile's workspace area: nkb*nslot_kb slots of mt*128 floats.  A lane's pairs sit at
     * two words of each set of 64*mt words.  The parts of an aligned split (one per k-block)
     * are summed over a binary tree of the k-blocks: at level L, node i adds the sums of its
     * children 2i and 2i+1 (k-blocks [2i << (L-1), (2i+1) << (L-1)) and the next such run),
     * exchanged at set r - 1, r = (2i+1) << (L-1) being the right child's first k-block (a
     * node without a right child passes its sum up); whoever completes a node carries its
     * sum up, and the second arrival at the root writes y.  The sum's order is fixed by the
     * tree, whatever the order of arrival: (P0 + P1) + P2 for three k-blocks. */
    /* the tile's words as a uniform base plus a 32-bit lane offset (a 64-bit per-lane pointer
     * live across the exchanges costs registers the 16-row kernels do not have) */
    uint64_t* const tb =
        (uint64_t*)((uint32_t*)p.slots + (size_t)t * p.nkb * p.nslot_kb * p.mt * 128);
    const uint32_t lw = (uint32_t)tile_off(lane) >> 1;
    const int nparts = chain ? (int)total : 2, leaf = chain ? kb : 0;
    /* exchanged through one XCD's L2 when both parts come from it: a paired launch, or a
     * one-k-block split whose two owners (neighbouring ranges) lie in one XCD's block of
     * ranges (xcd_order) */
    bool l2 = p.xcd_pair != 0;
    if (!l2 && p.xcd8 && p.nkb == 1 && DFQ_XCD_ORDER) {
        const int r0 = tile_first_owner(kbk, t), per = p.Gkb >> 3, rem = p.Gkb & 7;
        l2 = owner_wg(r0, per, rem) == owner_wg(r0 + 1, per, rem);
    }
    bool go[2] = {true, true};
    if (MT == 1 && p.epi) {
        /* lanes n < 8 hold g and take u from lane n + 8 (g words, then u words) */
        f32x4_t u;
#pragma unroll
        for (int r = 0; r < 4; ++r) u[r] = dpp_f32<0x128>(v[r]);
        if (!act || n >= 8) return;
        f32x4_t g = v;
#pragma unroll
        for (int L = 1; L <= kTreeLevels; ++L) {
            const int r = ((leaf >> L) * 2 + 1) << (L - 1);
            if (r >= nparts || !(go[0] || go[1])) continue;
            uint64_t* sj = tb + (lw + (uint32_t)((r - 1) * 64 * p.mt));
            if (l2) pair_exchange_gu<kL2Scope>(sj, sj + 32, go, g, u);
            else pair_exchange_gu<kDeviceScope>(sj, sj + 32, go, g, u);
        }
        const int H = p.N / 2;
        float lbg = 0.0f, lbu = 0.0f;
        if (p.lbias) {
            lbg = elem_to_f32<F16>(((const uint16_t*)p.lbias)[t * 16 + n]);
            lbu = elem_to_f32<F16>(((const uint16_t*)p.lbias)[t * 16 + n + 8]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * q + r;
            if (go[r >> 1] && m < p.M)
                put16((uint16_t*)p.y + (size_t)m * H + t * 8 + n,
                      silu_mul_round<F16>(g[r] + lbg, u[r] + lbu));
        }
        return;
    }
    if (p.epi) {
        /* 9..16 rows.  Lane n < 8 of a 16-lane row holds g of column n for its four rows,
         * lane n + 8 the u of that column.  Each takes its partner's four values (row_ror:8), and each pair
         * of lanes splits the rows: the g lane carries rows 0 and 1 of the four, the u lane
         * rows 2 and 3, each element as one (g, u) word of the plain exchange.  Every lane
         * of the tile then exchanges two words in one round trip, and the party that
         * completes an element has its g and u together.  With the u words exchanged first
         * and then the g words on half the lanes (two round trips), 16 rows at
         * 2 x 17408 x 5120 (every tile exchanged) measured 40.0 us; with one (g, u) word per
         * element on half the lanes, 35.4 us; this form 32.8 us. */
        f32x4_t o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = dpp_f32<0x128>(v[r]);
        if (!act) return;
        const bool gl = n < 8;
        const int e0 = gl ? 0 : 2;  // the first of this lane's two rows (of four)
        f32x4_t w = gl ? f32x4_t{v[0], o[0], v[1], o[1]} : f32x4_t{o[2], v[2], o[3], v[3]};
#pragma unroll
        for (int L = 1; L <= kTreeLevels; ++L) {
            const int r = ((leaf >> L) * 2 + 1) << (L - 1);
            if (r >= nparts || !(go[0] || go[1])) continue;
            uint64_t* sj = tb + (lw + (uint32_t)((r - 1) * 64 * p.mt));
            if (l2) pair_exchange<kL2Scope>(sj, go, w);
            else pair_exchange<kDeviceScope>(sj, go, w);
        }
        const int H = p.N / 2, j = n & 7;
        float lbg = 0.0f, lbu = 0.0f;
        if (p.lbias) {
            lbg = elem_to_f32<F16>(((const uint16_t*)p.lbias)[t * 16 + j]);
            lbu = elem_to_f32<F16>(((const uint16_t*)p.lbias)[t * 16 + 8 + j]);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int m = 4 * q + e0 + h;
            if (go[h] && m < p.M)
                put16((uint16_t*)p.y + (size_t)m * H + t * 8 + j,
                      silu_mul_round<F16>(w[2 * h] + lbg, w[2 * h + 1] + lbu));
        }
        return;
    }
    if (!act) return;
    f32x4_t w = v;
#pragma unroll
    for (int L = 1; L <= kTreeLevels; ++L) {
        const int r = ((leaf >> L) * 2 + 1) << (L - 1);
        if (r >= nparts || !(go[0] || go[1])) continue;
        uint64_t* sj = tb + (lw + (uint32_t)((r - 1) * 64 * p.mt));
        if (l2) pair_exchange<kL2Scope>(sj, go, w);
        else pair_exchange<kDeviceScope>(sj, go, w);
    }
    const int col = t * 16 + n;
    float lb = 0.0f;
    if (p.lbias && col < p.N) lb = elem_to_f32<F16>(((const uint16_t*)p.lbias)[col]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * q + r;
        if (go[r >> 1] && m < p.M && col < p.N) {
            const uint16_t o = f32_to_out<F16>(w[r] + lb);
            if (!AM || p.y) put16((uint16_t*)p.y + (size_t)m * p.N + col, o);
            if constexpr (AM) fold_key<F16>(best[r], o, col);
        }
    }
}

/* Whether tile t of the range [a, b) (k-block of SS chunks) is finished by the pair exchange
 * while the streaming goes on: it has exactly two parts in the whole split (a tile cut by the
 * range, or any tile of a two-k-block split without a second pass).  Every other tile is
 * written at the end of the workgroup: a whole tile to y, a part of a reduce split to its
 * workspace slot. */
__device__ __forceinline__ bool exchange_tile(const QmmParams& p, int t, int a, int b, int SS) {
    const bool whole = max(a, t * SS) == t * SS && min(b, (t + 1) * SS) == (t + 1) * SS &&
                       p.nkb == 1;
    return !whole && !p.reduce;
}

/* Greedy-accept mode, once every output of the workgroup has been folded into its row's key
 * in LDS (keys[m], zero at the start): wave 0 folds them into the workgroup group's keys with
 * an agent-scope atomic max (16 groups of workgroups, so that no key takes more than a
 * sixteenth of the atomics), waits for the maxima to complete (vmcnt) and counts the
 * workgroup on one device-wide counter.  The last workgroup takes every group's keys
 * (exchanging them with zero), writes each row's token (the column of its key, -1 for a row
 * of NaN) and the accepted run -- the first verify row i < M-1 whose token differs from
 * proposals[i], or M-1 -- and re-arms the counter.  The keys and the counter are only
 * touched by agent-scope atomics, which complete before the arrival is counted: no cache
 * write-back or invalidate. */
__device__ void accept_finish(const QmmParams& p, const uint64_t* keys, int lane) {
    const int G = (int)gridDim.x, ng = min(16, G), grp = (int)blockIdx.x % ng;
    if (lane < p.M) {
        const uint64_t k = keys[lane];
        if (k)
            __hip_atomic_fetch_max(p.am_keys + (size_t)grp * p.M + lane, k, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the maxima have completed
    uint32_t last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(p.am_count + 16 * 32, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) + 1u == (uint32_t)G;
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    bool bad = false;
    if (lane < p.M) {
        /* every group's key and the proposal in flight together: one round trip, not one
         * per group */
        const int32_t prop = (p.am_proposals && lane < p.M - 1) ? p.am_proposals[lane] : 0;
        uint64_t kk[16];  // groups past ng hold zero keys (never raised): read them too
#pragma unroll
        for (int g = 0; g < 16; ++g)
            kk[g] = __hip_atomic_exchange(p.am_keys + (size_t)g * p.M + lane, 0ull,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint64_t k = 0;
#pragma unroll
        for (int g = 0; g < 16; ++g) k = kk[g] > k ? kk[g] : k;
        const int32_t tok = k ? (int32_t)~(uint32_t)k : -1;
        if (p.am_tokens) p.am_tokens[lane] = tok;
        bad = lane < p.M - 1 && !(p.am_proposals && prop == tok);
    }
    const uint64_t badm = __builtin_amdgcn_ballot_w64(bad);
    if (lane == 0) {
        if (p.am_accepted) *p.am_accepted = badm ? (int32_t)__builtin_ctzll(badm) : p.M - 1;
        __hip_atomic_store(p.am_count + 16 * 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

/* The publisher wave of a qmm_mt8 workgroup: it finishes the pair-exchange tiles (a device-
 * scope round trip each) while the streaming continues, and, unless the split writes its
 * outputs at the end ("burst"), writes every other tile as it finishes.  The streaming waves
 * only sum a finished tile into the LDS output area and mark it kTileDone.  Global stores and
 * atomics in the streaming waves would sit in the same in-order vmcnt queue as their prefetch
 * and make every later wait cover them.
 *
 * Tiles are taken in the order the take order completes them (the tile shared with the next
 * workgroup first, then the first tile, ...), publisher pi taking ranks pi, pi + kPublishers,
 * ..., so that the two shared tiles' exchanges run side by side.  It polls their counters (one
 * lane per tile, sleeping between empty polls) until each has been published: every unit of
 * [a, b) is taken by exactly one streaming wave, so every tile reaches kTileDone.  In greedy-
 * accept mode its outputs' keys go to the rows' keys in LDS. */
template <bool F16, int MT, bool AM>
__device__ void publisher_wave(const QmmParams& p, int kb, int cl, int a, int b,
                               const KBlock& kbk, int lane, int pi) {
    const int SS = kbk.SS;
    const int q = lane >> 4, n = lane & 15;
    const int ta = a / SS;
    const int ntl = (b > a) ? (b - 1) / SS - ta + 1 : 0;
    uint32_t* tcnt = (uint32_t*)(lds_base() + p.lds_cnt_off);
    const float* tout = (const float*)(lds_base() + p.lds_tout_off);
    __syncthreads();  // the staging barrier of the streaming waves (tile counters zeroed)
    uint64_t best[4] = {0, 0, 0, 0};  // greedy-accept keys of rows 4q..4q+3
    auto tile_of = [&](int rk) { return rk == 0 ? ntl - 1 : rk - 1; };
    const int nrank = ntl > pi ? (ntl - pi + kPublishers - 1) / kPublishers : 0;
    int remaining = 0;
    for (int base = 0; base < nrank; base += 64) {
        const int rk = pi + (base + lane) * kPublishers;
        const bool own = base + lane < nrank &&
                         (!p.burst || exchange_tile(p, ta + tile_of(rk), a, b, SS));
        remaining += __builtin_popcountll(__builtin_amdgcn_ballot_w64(own));
    }
    while (remaining > 0) {
        int found = 0;
        for (int base = 0; base < nrank; base += 64) {
            const int rk = pi + (base + lane) * kPublishers;
            bool ready = false;
            if (base + lane < nrank && (!p.burst || exchange_tile(p, ta + tile_of(rk), a, b, SS)))
                ready = __hip_atomic_load(tcnt + tile_of(rk), __ATOMIC_ACQUIRE,
                                          __HIP_MEMORY_SCOPE_WORKGROUP) == kTileDone;
            uint64_t m = __builtin_amdgcn_ballot_w64(ready);
            while (m) {
                const int bit = __builtin_ctzll(m);
                m &= m - 1;
                const int tlb = tile_of(pi + (base + bit) * kPublishers);
                const int t = ta + tlb;
                f32x4_t v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (lane < 32 * MT) v = *(const f32x4_t*)(tout + tlb * (MT * 128) + tile_off(lane));
                if (!exchange_tile(p, t, a, b, SS)) {
                    if (!p.reduce || (max(a, t * SS) == t * SS && min(b, (t + 1) * SS) == (t + 1) * SS &&
                                      p.nkb == 1))
                        store_y<F16, AM>(p, t, lane, v, best);
                    else if (lane < 32 * MT)  /* summed by the second pass: no round trip here */
                        put_tile4(tile_slot(p, t, kb, cl - tile_first_owner(kbk, t), lane), v);
                } else {
                    publish<F16, MT, AM>(p, kbk, t, kb, lane, v, best);
                }
                if (lane == 0) tcnt[tlb] = kTileOut;
                ++found;
            }
        }
        remaining -= found;
        if (!found) __builtin_amdgcn_s_sleep(1);
    }
    if constexpr (AM) {
        /* the lane keys of rows 4q..4q+3, reduced over the 16 columns of the lane group,
         * into the rows' keys in LDS */
        uint64_t* keys = (uint64_t*)(lds_base() + p.lds_key_off);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int s = 8; s > 0; s >>= 1) {
                const uint32_t lo = __shfl_xor((uint32_t)best[r], s, 16);
                const uint32_t hi = __shfl_xor((uint32_t)(best[r] >> 32), s, 16);
                const uint64_t o = ((uint64_t)hi << 32) | lo;
                best[r] = o > best[r] ? o : best[r];
            }
        if (n == 0 && lane < 32 * MT)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (4 * q + r < p.M && best[r])
                    __hip_atomic_fetch_max(keys + 4 * q + r, best[r], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

/* The end of a workgroup, reached by every wave once its work is done: after a barrier (every
 * tile summed into the LDS output area, every exchange tile published), all waves write the
 * remaining tiles.  A whole tile goes to y as 16-byte rows of 8 outputs (plus the linear
 * bias; the gate|up epilogue writes 8 outputs h = silu(g)*u per row), and, in greedy-accept
 * mode, each row's outputs are folded into its key; a tile's part of a reduce split goes to
 * its workspace slot.  Output stores happen here, after the streaming, so that they neither
 * queue behind the weight loads nor hold ring slots. */
template <bool F16, int MT, bool AM>
__device__ void finish_wg(const QmmParams& p, const KBlock& kbk, int kb, int cl, int a, int b,
                          int tid) {
    __syncthreads();
    /* opaque: nothing of the write-out is computed (and held in registers) before this point */
    __asm__ volatile("" : "+v"(tid));
    const int SS = kbk.SS;
    uint64_t* keys = (uint64_t*)(lds_base() + p.lds_key_off);
    if (b > a && p.burst) {
        const int ta = a / SS, ntl = (b - 1) / SS - ta + 1;
        const float* tout = (const float*)(lds_base() + p.lds_tout_off);
        const int M = p.M;
        const uint16_t* lb16 = (const uint16_t*)p.lbias;
        /* whole tiles: items (tile, row, half of 8 columns), or (tile, row) for the epilogue */
        const int per = p.epi ? M : 2 * M;
        for (int i = tid; i < ntl * per; i += kBlock) {
            const int tl = i / per, r = i - tl * per;
            const int t = ta + tl;
            if (!(max(a, t * SS) == t * SS && min(b, (t + 1) * SS) == (t + 1) * SS && p.nkb == 1))
                continue;
            const float* tb = tout + tl * (MT * 128);
            uint16_t o[8];
            if (p.epi) {
                const int m = r;
                const float* tr = tb + (m >> 3) * 128 + (m & 7);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float g = tr[j * 8], u = tr[(8 + j) * 8];
                    if (lb16) {
                        g += elem_to_f32<F16>(lb16[t * 16 + j]);
                        u += elem_to_f32<F16>(lb16[t * 16 + 8 + j]);
                    }
                    o[j] = silu_mul_round<F16>(g, u);
                }
                uint16_t* dst = (uint16_t*)p.y + (size_t)m * (p.N / 2) + t * 8;
                if (((uintptr_t)dst & 15) == 0) {
                    u32x4_t w;
#pragma unroll
                    for (int j = 0; j < 4; ++j) w[j] = (uint32_t)o[2 * j] | ((uint32_t)o[2 * j + 1] << 16);
                    *(u32x4_t*)dst = w;
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) put16(dst + j, o[j]);
                }
            } else {
                const int m = r >> 1, hh = r & 1;
                const int c0 = t * 16 + hh * 8;
                if (c0 >= p.N) continue;
                const float* tr = tb + (m >> 3) * 128 + (hh * 8) * 8 + (m & 7);
                uint64_t kbest = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int col = c0 + j;
                    float v = tr[j * 8];
                    if (lb16 && col < p.N) v += elem_to_f32<F16>(lb16[col]);
                    o[j] = f32_to_out<F16>(v);
                    if constexpr (AM)
                        if (col < p.N) fold_key<F16>(kbest, o[j], col);
                }
                if (!AM || p.y) {
                    uint16_t* dst = (uint16_t*)p.y + (size_t)m * p.N + c0;
                    if (c0 + 8 <= p.N && ((uintptr_t)dst & 15) == 0) {
                        u32x4_t w;
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            w[j] = (uint32_t)o[2 * j] | ((uint32_t)o[2 * j + 1] << 16);
                        *(u32x4_t*)dst = w;
                    } else {
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            if (c0 + j < p.N) put16(dst + j, o[j]);
                    }
                }
                if constexpr (AM)
                    if (kbest)
                        __hip_atomic_fetch_max(keys + m, kbest, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        /* parts of a reduce split: each tile's fp32 part to its workspace slot */
        if (p.reduce) {
            for (int i = tid; i < ntl * 32 * MT; i += kBlock) {
                const int tl = i / (32 * MT), li = i - tl * (32 * MT);
                const int t = ta + tl;
                if (max(a, t * SS) == t * SS && min(b, (t + 1) * SS) == (t + 1) * SS && p.nkb == 1)
                    continue;  // whole: written to y above
                put_tile4(tile_slot(p, t, kb, cl - tile_first_owner(kbk, t), li),
                          *(const f32x4_t*)(tout + tl * (MT * 128) + tile_off(li)));
            }
        }
    }
    if constexpr (AM) {
        __syncthreads();  // every output folded into its row's key
        if ((tid >> 6) == 0) accept_finish(p, keys, tid & 63);
    }
}

/* ---------------------------------------------------------------------------------- */
/* The fast kernel                                                                      */
/* ---------------------------------------------------------------------------------- */

/* CH super-steps form one work unit ("chunk").  With CH = 8 / GPS a chunk spans exactly 8
 * quantisation groups, so each lane fetches the chunk's scales (and biases) of its row as
 * one 16-byte load; CH = 1 is the general form (one 4-byte scale load per super-step). */
/* One tile of a reduce split's second pass: the tile's partial slots summed in (k-block,
 * workgroup) order -- a fixed order, so the result does not depend on timing -- plus the
 * linear bias, to y; the slots are zeroed, which leaves the workspace zero at rest.  Tiles
 * with one contributor were written by the main kernel.
 *
 * All nkb * nslot_kb slots of the tile are read, eight loads in flight
 * before any use: the slots a k-block leaves unused are zero, and adding +0.0f to a sum
 * that is never -0.0f (it starts at +0.0f) leaves it unchanged, so the result equals the
 * sum of the used slots alone.  One memory latency per eight slots instead of one per
 * slot. */
template <bool F16>
__device__ __forceinline__ void reduce_tile(const QmmParams& p, int t, int lane) {
    /* A tile of a several-k-block split has a part in every k-block.  With one k-block, a tile
     * inside one workgroup's range was written by the main kernel.  (Counting the parts over
     * every k-block put each k-block's split arithmetic, several integer divisions, before
     * the first load: C3 19.7-20.3 -> 18.6-19.0 us.) */
    if (p.nkb == 1 && tile_owners(kblock(p, 0), t) <= 1) return;
    f32x4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
    if (lane < 32 * p.mt) {
        const int S = p.nkb * p.nslot_kb, stride = p.mt * 128;
        float* s0 = tile_slot(p, t, 0, 0, lane);  // slot i = kb * nslot_kb + j at s0 + i * stride
        constexpr int NB = 8;
        for (int b = 0; b < S; b += NB) {
            f32x4_t v[NB];
#pragma unroll
            for (int i = 0; i < NB; ++i)
                if (b + i < S) v[i] = *(const f32x4_t*)(s0 + (size_t)(b + i) * stride);
#pragma unroll
            for (int i = 0; i < NB; ++i)
                if (b + i < S) {
                    sum += v[i];
                    put_tile4(s0 + (size_t)(b + i) * stride, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
                }
        }
    }
    uint64_t unused[4] = {0, 0, 0, 0};  // a reduce split never runs in greedy-accept mode
    store_y<F16>(p, t, lane, sum, unused);
}

template <int BITS, int GS, bool F16, int CH, int PF, int MT, bool AM = false, bool PK = false>
__device__ __forceinline__ void qmm_mt8(const QmmParams& p, int wg) {
    using C = Cfg<BITS, GS>;
    static_assert(!PK || CH > 1, "the packed layout holds 8-group chunks");
    constexpr int XR = 8 * MT;  // rows of x sums per group in LDS
    static_assert(CH == 1 || CH * C::GPS == 8 || CH * C::GPS == C::CG,
                  "chunk = one super-step, 8 groups or CG groups");
    constexpr int SB = (CH > 1) ? CH * C::GPS / 8 : 1;  // 16-byte scale (bias) loads a unit
    uint8_t* lds = lds_base();

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4;  // lane group: k slot for A/B, row block for the result
    const int n = lane & 15;  // B column / A row / result column

    const int kb = wg / p.Gkb;          // the launch has nkb * Gkb workgroups
    const int cl = wg - kb * p.Gkb;
    const KBlock kbk = kblock(p, kb);
    const int SS = kbk.SS;    // chunks per tile in this k-block
    const int a = range_start(kbk, cl);
    const int b = range_start(kbk, cl + 1);

    if (wave >= kWaves) {
        publisher_wave<F16, MT, AM>(p, kb, cl, a, b, kbk, lane, wave - kWaves);
        finish_wg<F16, MT, AM>(p, kbk, kb, cl, a, b, tid);
        return;
    }

    const int RB = p.K * BITS / 8;        // bytes per weight row
    const int GPR = p.K / GS;             // groups per row
    const int kr = SS * (CH * C::KSS);    // k elements in this k-block
    const int k0 = kbk.c0 * (CH * C::KSS);  // first k of this k-block

    /* ---- x staging loads go out first (their wait must not cover the weight prefetch).
     * Row sr of the k-block's x goes to the TPR threads sr*TPR .. +TPR-1 (a multiple of GS/8,
     * M*TPR <= kStageThreads): thread sr*TPR + sc takes the 16-byte chunks sc, sc + TPR,
     * sc + 2 TPR, ... of the row, so an item's global and LDS addresses and its group-sum
     * slot step by constants, and a group's GS/8 chunks sit in aligned neighbouring lanes.
     * A thread's last item past the row's end reloads the row's last chunk (and stores the
     * same value again); threads past row M stage nothing. */
    const int CPR = kr / 8;                  // 16-byte chunks per row of the k-block
    const int TPR = DFQ_STAGE_TPR(p.M, GS);  // wave-uniform
    constexpr int kMaxStageItems = DFQ_STAGE_ITEMS(MT);  // 16-byte x chunks a thread at most
    const int NI = (CPR + TPR - 1) / TPR;    // items per staging thread (the host plan
                                             // keeps it within kMaxStageItems)
    const int sr = tid / TPR;
    const int sc = tid - sr * TPR;
    const bool stager = tid < kStageThreads && sr < p.M;
    /* the k-block's x as a uniform base plus 32-bit per-lane offsets (24-bit multiplies:
     * staging is VALU-bound, so no 64-bit address arithmetic per item) */
    const uint8_t* xb = (const uint8_t*)p.x + (size_t)k0 * 2;
    const uint32_t xrow_off = __umul24((uint32_t)sr, (uint32_t)p.K * 2u);
    u32x4_t xv[kMaxStageItems];
    auto stage_loads = [&]() {
        if (!stager) return;
#pragma unroll
        for (int i = 0; i < kMaxStageItems; ++i)
            if (i < NI) {
                const uint32_t c = (uint32_t)min(sc + i * TPR, CPR - 1);
                xv[i] = *(const u32x4_t*)(xb + (xrow_off + c * 16u));
            }
        __builtin_amdgcn_sched_barrier(0);
    };
    /* x goes out before the split's scalar arithmetic, which overlaps its latency */
    stage_loads();

    /* ---- units of this workgroup, in the order its waves take them: the tile it shares
     * with the next workgroup first ([s1, b)), then the rest from a (which starts with the
     * tile shared with the previous one), so that cross-workgroup fix-ups happen early.
     * Waves take the first kWaves*PF units by index and the rest from an LDS counter. */
    const int L = b - a;
    const int tlast = (b - 1) / SS;
    const int s1 = max(a, tlast * SS);
    const int nrot = b - s1;
    auto unit_of = [&](int g) { return g < nrot ? s1 + g : a + (g - nrot); };

    /* ---- weight / scale / bias prefetch ring, one unit per slot.  Loads take a scalar
     * base (tile row 0, chunk k) plus a per-lane 32-bit offset; a lane whose row is past N
     * re-reads row N-1 (its result is never stored).  Every issue loads its slot: past the
     * end of the range it fetches the last unit it had again (an L2 hit), so the number of
     * loads in flight is the same on every path through the loop and the compiler's vmcnt
     * waits name exactly the slot being consumed. */
    const uint32_t lane_w = (uint32_t)q * 16u;
    const uint32_t lane_s = (CH > 1) ? 0u : (C::GPS == 4 ? 4u * (q >> 1) : 0u);
    using SV = typename std::conditional<(CH > 1), u32x4_t, uint32_t>::type;
    u32x4_t rw[PF][CH][C::NS];
    SV rsb[PF][SB];  // scale words (lane rows 0, 2) or bias words (rows 1, 3) of the slot's unit
    int sg[PF];  // the unit (as a take index) each slot holds; >= L: none
    const uint8_t* wbytes = (const uint8_t*)p.w;
    const uint8_t* sbytes = (const uint8_t*)p.scales;
    const uint8_t* bbytes = (const uint8_t*)p.biases;

    /* last unit fetched.  A wave that gets no unit still fetches one, never used: the first
     * unit of the range, or the k-block's last unit for an empty range (which can sit past
     * the last unit when a small k-block has fewer units than workgroups).  Skipping that
     * fetch measured 1.1 us slower at 16 rows and 0.2 us at 8 (the loop's code changes),
     * for 0.18 us at one row and N = K = 4096 (eight units a workgroup). */
    int lu = min(a, p.T * SS - 1);
    auto issue = [&](int slot, int g) {
        sg[slot] = g;
        const int u = g < L ? unit_of(g) : lu;
        lu = u;
        const int t = u / SS, c = u - t * SS;
        const int row0 = t * 16;
        const int rl = (row0 + 16 <= p.N) ? n : min(n, p.N - 1 - row0);
        const uint32_t vw = (uint32_t)rl * RB + lane_w;
        const uint32_t vs = (uint32_t)rl * GPR * 2u + lane_s;
        if constexpr (PK) {
            /* the packed unit of CG groups, which holds RH of this kernel's chunks (part hh
             * of it is this chunk): its codes as pieces of 1 KB (this lane's 16 bytes of piece
             * i at i * 1024 + lane * 16; the chunk's pieces from hh * CH * NS), then its rows'
             * scales and biases, 16 * PSB bytes a row (this lane's h-th 16 bytes of the chunk
             * at (q & 1) * 256 PSB + n * 16 PSB + 16 (hh SB + h)); past row N the pack holds
             * zeros */
            constexpr int RH = C::CG / (CH * C::GPS);
            constexpr int PSB = C::CG / 8;
            constexpr uint32_t kCodeBytes = 16u * C::CG * GS * BITS / 8u;
            const int kc = kbk.c0 + c;
            const int hh = kc % RH;
            const uint8_t* ub = wbytes + ((size_t)t * (p.chunks / RH) + kc / RH) *
                                             (kCodeBytes + 512u * PSB);
#pragma unroll
            for (int h = 0; h < SB; ++h)
                rsb[slot][h] = *(const SV*)(ub + kCodeBytes +
                                            (uint32_t)((q & 1) * 256 * PSB + n * 16 * PSB +
                                                       16 * (hh * SB + h)));
#pragma unroll
            for (int j = 0; j < CH; ++j)
#pragma unroll
                for (int s = 0; s < C::NS; ++s)
                    rw[slot][j][s] = *(const u32x4_t*)(ub + (hh * CH * C::NS + j * C::NS + s) * 1024 +
                                                       (uint32_t)lane * 16u);
            return;
        }
        const uint8_t* sbb = (q & 1) ? bbytes : sbytes;
        const int kc = k0 + c * (CH * C::KSS);  // first k of the chunk
        const uint8_t* wb = wbytes + (size_t)row0 * RB + kc * BITS / 8;
        const size_t so = ((size_t)row0 * GPR + kc / GS) * 2;
        /* scales / biases first: they are split (a cross-lane swap) before the first MFMA */
#pragma unroll
        for (int h = 0; h < SB; ++h) rsb[slot][h] = *(const SV*)(sbb + so + vs + 16u * h);
#pragma unroll
        for (int j = 0; j < CH; ++j)
#pragma unroll
            for (int s = 0; s < C::NS; ++s)
                rw[slot][j][s] = *(const u32x4_t*)(wb + vw + (j * C::NS + s) * 64);
    };

    /* ---- LDS layout: row 0 zeros, rows 1..M x; per-group x sums; a ring of p.ring partial
     * tiles ([n][8] fp32, 512 bytes each), the unit with take index g using slot g % ring,
     * and each slot's generation (the take index allowed to write it next); tile arrival
     * counters; the take counter */
    const int RS = p.lds_row_stride;
    const int R = p.ring;
    float* xsum = (float*)(lds + p.lds_xsum_off);
    float* part = (float*)(lds + p.lds_part_off);
    float* tout = (float*)(lds + p.lds_tout_off);
    uint32_t* gen = (uint32_t*)(lds + p.lds_gen_off);
    uint32_t* tcnt = (uint32_t*)(lds + p.lds_cnt_off);
    const int ta = a / SS;               // first tile touched by this workgroup
    const int ntl = tlast - ta + 1;      // tiles touched
    uint32_t* gcnt = tcnt + ntl;
    const int GK = kr / GS;  // groups in the k-block
    /* per item: pre-permute into the MFMA k order, and sum its 8 elements; the GS/8 items
     * of a group sit in aligned neighbouring lanes of one row (all real or all past the
     * row's end, as CPR and TPR are multiples of GS/8) and are summed with DPP; the group's
     * first lane stores the sum. */
    const bool leader = (tid & (GS / 8 - 1)) == 0;
    auto stage_finish = [&]() {
    if (stager) {
        const uint32_t lrow = __umul24((uint32_t)(1 + sr), (uint32_t)p.lds_row_stride);
#pragma unroll
        for (int i = 0; i < kMaxStageItems; ++i) {
            if (i < NI) {
                const int c = sc + i * TPR;
                float sm = chunk_dot<F16>(xv[i], 0.0f);
                sm += dpp_f32<0xB1>(sm);             // lanes ^1 (quad_perm 1,0,3,2)
                sm += dpp_f32<0x4E>(sm);             // lanes ^2 (quad_perm 2,3,0,1)
                if constexpr (GS >= 64) sm += dpp_f32<0x104>(sm);   // + lane+4 (row_shl:4)
                if constexpr (GS >= 128) sm += dpp_f32<0x108>(sm);  // + lane+8 (row_shl:8)
                const u32x4_t v = (BITS == 4) ? nibble_permute(xv[i]) : xv[i];
                *(u32x4_t*)(lds + lrow + (uint32_t)min(c, CPR - 1) * 16u) = v;
                if (leader && c < CPR) xsum[(c / (GS / 8)) * XR + sr] = sm;
            }
        }
    }
    for (int c = tid; c < CPR; c += kThreads) *(u32x4_t*)(lds + c * 16) = u32x4_t{0, 0, 0, 0};
    for (int i = tid; i < GK * XR; i += kThreads)
        if ((i & (XR - 1)) >= p.M) xsum[i] = 0.0f;
    for (int i = tid; i < ntl; i += kThreads) tcnt[i] = 0u;
    for (int i = tid; i < R; i += kThreads) gen[i] = (uint32_t)i;
    if (tid < 16) ((uint64_t*)(lds + p.lds_key_off))[tid] = 0ull;  // greedy-accept row keys
    if (tid == 0) {
        *gcnt = (uint32_t)(kWaves * PF);
        gcnt[1] = 0u;  // the publishers' arrival count (greedy-accept mode)
    }
    __builtin_amdgcn_sched_barrier(0);
    };
    auto issue_first = [&]() {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            issue(i, wave * PF + i);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    /* x first (issued above): issued after the weights, its wait would cover them */
    stage_finish();
    issue_first();
    __syncthreads();

    /* ---- per-lane A / x-sum addresses.  Up to 8 rows: the A operand is block-diagonal,
     * x rows 0-7 against the lane groups 0-1 (one quantisation group) in rows 0-7 and against
     * lane groups 2-3 (the other) in rows 8-15, zeros elsewhere (LDS row 0); the two halves
     * are folded at the end.  9..16 rows: x rows 0-15 against every lane group (operand words
     * in the 16-row form). */
    const bool diag = (n < 8) == (q < 2);
    const int arow = (MT == 1) ? ((diag && (n & 7) < p.M) ? 1 + (n & 7) : 0)
                               : (n < p.M ? 1 + n : 0);
    constexpr int HO = C::NOPS / 2;
    constexpr int DH = C::delta_chunk(HO);
    static_assert(wide_layout_holds<C>(), "16-row operand layout");
    const uint32_t abase =
        (uint32_t)arow * RS +
        (uint32_t)((MT == 1) ? C::base_chunk(q) : C::base_chunk(q & 1) + (q >> 1) * DH) * 16u;
    const uint32_t abase_hi =
        (uint32_t)arow * RS + (uint32_t)(C::base_chunk((q & 1) + 2) + (q >> 1) * DH) * 16u;
    const uint32_t xbase =
        (MT == 1) ? (uint32_t)p.lds_xsum_off + (uint32_t)C::group_of(0, q) * (XR * 4u) +
                        (uint32_t)(q & 1) * 16u
                  : (uint32_t)p.lds_xsum_off + (uint32_t)q * 16u;
    const uint32_t sel_half = (q >> 1) ? kSelHi : kSelLo;
    constexpr float kOff = (BITS == 4) ? (F16 ? 1024.0f : 128.0f) : 0.0f;
    uint32_t magic = F16 ? 0x64006400u : 0x43004300u;
    uint32_t nmask = 0x000F000Fu;
    __asm__ volatile("" : "+v"(magic));  // opaque: keep in a VGPR (see nibble_operand)
    __asm__ volatile("" : "+s"(nmask));  // opaque: keep in an SGPR

    /* One unit: CH super-steps of MFMA on the operands in slot i, the scale / bias epilogue,
     * the fold of the two group halves, and the arrival at the unit's tile. */
    auto process = [&](const int i, const int g) {
        const int u = unit_of(g);
        const int t = u / SS, cc = u - t * SS;
        /* The scale (bias) words of the super-steps in hand: load h serves super-steps
         * [h * JPH, (h + 1) * JPH) and is split as the first of them begins, so that only one
         * load's words are live at a time.  Word w of the chunk covers its groups 2w, 2w + 1. */
        constexpr int JPH = CH / SB;
        SV rs_i, rb_i;
        auto sw_of = [&](const SV& a, int w) -> uint32_t {
            if constexpr (CH > 1) return a[w & 3];
            else return a;
        };
        auto split_for = [&](int j) {
            if (j % JPH == 0) split_scale_bias(rsb[i][j / JPH], rs_i, rb_i);
        };
        f32x4_t v;  // lanes 0-31: rows 0-7 (MT 1); all lanes: rows 4q..4q+3 (MT 2)
        if constexpr (MT == 1) {
            f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int css = cc * CH + j;  // super-step within the k-block
                split_for(j);
                uint32_t OW[C::NOW];
                build_operand_words<BITS, GS>(rw[i][j], OW);
                const uint32_t aoff = abase + (uint32_t)css * (C::CPS * 16);
                f32x4_t P[C::NP];
#pragma unroll
                for (int pp = 0; pp < C::NP; ++pp) P[pp] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int o = 0; o < C::NOPS; ++o) {
                    const u32x4_t A = *(const u32x4_t*)(lds + aoff + C::delta_chunk(o) * 16);
                    u32x4_t B;
                    if constexpr (BITS == 4) B = nibble_operand<F16>(OW[o], nmask, magic);
                    else B = byte_operand<F16>(OW[2 * o], OW[2 * o + 1]);
                    P[C::partial_of(o)] = mfma<F16>(A, B, P[C::partial_of(o)]);
                }
                const uint32_t xo = xbase + (uint32_t)css * (C::GPS * XR * 4);
#pragma unroll
                for (int pp = 0; pp < C::NP; ++pp) {
                    uint32_t sw, bw2, sel;
                    if constexpr (CH > 1) {
                        if constexpr (C::GPS == 4) {
                            sw = (q >> 1) ? sw_of(rs_i, 2 * j + 1) : sw_of(rs_i, 2 * j);
                            bw2 = (q >> 1) ? sw_of(rb_i, 2 * j + 1) : sw_of(rb_i, 2 * j);
                            sel = pp ? kSelHi : kSelLo;
                        } else {
                            sw = sw_of(rs_i, j);
                            bw2 = sw_of(rb_i, j);
                            sel = sel_half;
                        }
                    } else {
                        sw = rs_i;
                        bw2 = rb_i;
                        sel = (C::GPS == 4) ? (pp ? kSelHi : kSelLo) : sel_half;
                    }
                    const float s = half_sel<F16>(sw, sel);
                    const float bb = half_sel<F16>(bw2, sel);
                    const float bp = (kOff != 0.0f) ? __builtin_fmaf(-kOff, s, bb) : bb;
                    const f32x4_t X = *(const f32x4_t*)(lds + xo + pp * (XR * 4));
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        acc[r] = __builtin_fmaf(s, P[pp][r], acc[r]);
                        acc[r] = __builtin_fmaf(bp, X[r], acc[r]);
                    }
                }
            }
            /* fold the two group halves: lanes 0-31 hold the 8x16 partial */
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                uint32_t lo = __float_as_uint(acc[r]), hi = lo;
                permlane32_swap(lo, hi);
                /* lanes 0-31: own value + the value of lane + 32 */
                v[r] = __uint_as_float(lo) + __uint_as_float(hi);
            }
        } else {
            static_assert(CH > 1, "the 16-row form takes 8-group chunks");
            v = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int css = cc * CH + j;
                split_for(j);
                uint32_t OW[C::NOW];
                build_operand_words_wide<BITS, GS>(rw[i][j], OW);
                f32x4_t P[C::GPS];  // one partial per group of the super-step
#pragma unroll
                for (int gg = 0; gg < C::GPS; ++gg) P[gg] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int o = 0; o < C::NOPS; ++o) {
                    const int h = o >= HO ? 1 : 0;
                    const uint32_t aoff = (h ? abase_hi : abase) + (uint32_t)css * (C::CPS * 16) +
                                          C::delta_chunk(o - h * HO) * 16;
                    const u32x4_t A = *(const u32x4_t*)(lds + aoff);
                    u32x4_t B;
                    if constexpr (BITS == 4) B = nibble_operand<F16>(OW[o], nmask, magic);
                    else B = byte_operand<F16>(OW[2 * o], OW[2 * o + 1]);
                    const int gg = C::group_of(C::partial_of(o), 2 * h);
                    P[gg] = mfma<F16>(A, B, P[gg]);
                }
                const uint32_t xo = xbase + (uint32_t)css * (C::GPS * XR * 4);
#pragma unroll
                for (int gg = 0; gg < C::GPS; ++gg) {
                    const int gi = j * C::GPS + gg;  // group within the chunk
                    const uint32_t sel = (gi & 1) ? kSelHi : kSelLo;
                    const float s = half_sel<F16>(sw_of(rs_i, gi >> 1), sel);
                    const float bb = half_sel<F16>(sw_of(rb_i, gi >> 1), sel);
                    const float bp = (kOff != 0.0f) ? __builtin_fmaf(-kOff, s, bb) : bb;
                    const f32x4_t X = *(const f32x4_t*)(lds + xo + gg * (XR * 4));
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        v[r] = __builtin_fmaf(s, P[gg][r], v[r]);
                        v[r] = __builtin_fmaf(bp, X[r], v[r]);
                    }
                }
            }
        }
        /* the slot of take g: wait until the unit that held it last (take g - R) is
         * released (never, when the range fits the ring) */
        const int sl = g % R;
        if (L > R) {
            while ((int)__hip_atomic_load(gen + sl, __ATOMIC_ACQUIRE,
                                          __HIP_MEMORY_SCOPE_WORKGROUP) != g)
                __builtin_amdgcn_s_sleep(1);
        }
        if (lane < 32 * MT) *(f32x4_t*)(part + sl * (MT * 128) + tile_off(lane)) = v;
        /* arrive at tile t; the wave that completes its units here sums them (in unit order)
         * into the tile's block of the output area, releases all the tile's slots, and marks
         * the tile done (for the publisher wave, or the write-out at the end) */
        const int u0 = max(a, t * SS), u1 = min(b, (t + 1) * SS);
        uint32_t old = 0;
        if (lane == 0)
            old = __hip_atomic_fetch_add(tcnt + (t - ta), 1u, __ATOMIC_ACQ_REL,
                                         __HIP_MEMORY_SCOPE_WORKGROUP);
        old = __builtin_amdgcn_readfirstlane(old);
        if ((int)old + 1 == u1 - u0) {
            const int g0 = u0 >= s1 ? u0 - s1 : nrot + (u0 - a);  // the tile's takes: g0..
            const int sl0 = g0 % R;
            if (lane < 32 * MT) {
                f32x4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int i = 0, s2 = sl0; i < u1 - u0; ++i, s2 = (s2 + 1 == R) ? 0 : s2 + 1)
                    sum += *(const f32x4_t*)(part + s2 * (MT * 128) + tile_off(lane));
                *(f32x4_t*)(tout + (t - ta) * (MT * 128) + tile_off(lane)) = sum;
            }
            /* The slots' reads above complete before any slot is handed on.  Then each lane
             * releases one slot (a tile has at most R units in a range, so its slots wrap
             * at most once): one store instruction instead of a per-slot loop of modulo
             * arithmetic and waits on the completing wave, which issues its next unit only
             * after this (the headline call measured 16.25-16.47 -> 16.06-16.09 us, the LM
             * head 82.9 -> 82.1 us). */
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            for (int i = lane; i < u1 - u0; i += 64) {
                const int s2 = sl0 + i;
                __hip_atomic_store(gen + (s2 >= R ? s2 - R : s2), (uint32_t)(g0 + i + R),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            if (lane == 0)
                __hip_atomic_store(tcnt + (t - ta), kTileDone, __ATOMIC_RELEASE,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    };

    if constexpr (PF == 1) {
        /* One slot: take the next unit, compute this one, and refill the slot only if there
         * is a next unit.  Both edges into the loop header carry exactly the slot's loads,
         * and the last pass issues nothing (no reload past the end to drain before exit). */
        int g = sg[0];
        if constexpr (MT == 2 && BITS == 8 && GS == 128) {
            /* The same loop written over a lambda: the register allocation it gets keeps
             * this kernel at 100 VGPRs with no spills, instead of 128 VGPRs and 164 bytes
             * of scratch (16 rows: 16.7 us against 27.4 us at N = K = 5120).  For the other
             * formats it measured equal or up to 3 % slower, so they keep the plain form. */
            auto stream = [&](int end) {
                while (g < end) {
                    uint32_t gn = 0;
                    if (lane == 0)
                        gn = __hip_atomic_fetch_add(gcnt, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_WORKGROUP);
                    process(0, g);
                    gn = __builtin_amdgcn_readfirstlane(gn);
                    g = (int)gn;
                    if (g >= end) break;
                    __builtin_amdgcn_sched_barrier(0);
                    issue(0, g);
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            stream(L);
        } else {
            while (g < L) {
                uint32_t gn = 0;
                if (lane == 0)
                    gn = __hip_atomic_fetch_add(gcnt, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_WORKGROUP);
                process(0, g);
                gn = __builtin_amdgcn_readfirstlane(gn);
                if ((int)gn >= L) break;
                __builtin_amdgcn_sched_barrier(0);
                issue(0, (int)gn);
                __builtin_amdgcn_sched_barrier(0);
                g = (int)gn;
            }
        }
    } else {
    /* The only exit is at the top: takes grow monotonically, so once slot 0 holds no unit no
     * slot does.  Every pass refills every slot (past the end with a clamped reload), so no
     * path reaches the back edge with fewer loads in flight. */
    while (sg[0] < L) {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            const int g = sg[i];
            /* take the next unit now; its index is needed when slot i is refilled */
            uint32_t gn = 0;
            if (lane == 0)
                gn = __hip_atomic_fetch_add(gcnt, 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_WORKGROUP);
            if (g < L) process(i, g);
            gn = __builtin_amdgcn_readfirstlane(gn);
            __builtin_amdgcn_sched_barrier(0);
            issue(i, (int)gn);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    }
    finish_wg<F16, MT, AM>(p, kbk, kb, cl, a, b, tid);
}


/* ---------------------------------------------------------------------------------- */
/* Generic kernel: the stock-op stand-in                                                */
/* ---------------------------------------------------------------------------------- */

__device__ __forceinline__ float load_any(const void* ptr, int dt, size_t i) {
    if (dt == 2) return ((const float*)ptr)[i];
    const uint16_t h = ((const uint16_t*)ptr)[i];
    if (dt == 1) return (float)__builtin_bit_cast(_Float16, h);
    return __uint_as_float((uint32_t)h << 16);
}

__device__ __forceinline__ void store_any(void* ptr, int dt, size_t i, float f) {
    if (dt == 2) ((float*)ptr)[i] = f;
    else if (dt == 1) ((uint16_t*)ptr)[i] = f32_to_out<true>(f);
    else ((uint16_t*)ptr)[i] = f32_to_out<false>(f);
}

/* ---------------------------------------------------------------------------------- */
/* The stock path for few rows: a GEMV (qmv)                                            */
/* ---------------------------------------------------------------------------------- */

/* MLX's stock op runs a GEMV (qmv) below about 13 rows (README.md:19-21 of the reference):
 * one pass over each weight row per call, at HBM speed for one row.  This is that path for
 * up to 4 rows a launch (more rows take one launch per 4), written for CDNA4: no MFMA, no
 * split of K across workgroups, nothing shared between workgroups.
 *
 *  - x (all M rows, pre-permuted into the nibble order of the codes, as the fast kernel keeps
 *    it) and its per-chunk sums are staged in LDS once per workgroup, one workgroup per CU.
 *  - A wave takes 4 weight rows at a time (groups of the workgroup's rows, the first by wave
 *    index, then from an LDS counter) and walks K in steps: lane l holds the 16 bytes of codes
 *    of chunk l + 64 j of each row (32 k at 4 bits, 16 at 8), so each load instruction reads
 *    1 KB of one row.  The next step's codes, scales and biases are in flight while a step is
 *    computed (two register sets).
 *  - A chunk lies in one quantisation group: acc += s * sum x (MAGIC + q) + (b - MAGIC s) *
 *    sum x, with sum x (MAGIC + q) from v_dot2 on the exact 16-bit codes and the chunk's
 *    staged x sum.
 *  - At the end of a row group every lane holds partial sums; a DPP and cross-row reduction
 *    gives each output, which goes to an LDS block; the workgroup writes its rows' outputs
 *    after all its groups, so no store joins the loads' queue. */
constexpr int kQmvWaves = 8;  // waves per workgroup
constexpr int kQmvRows = 4;   // weight rows a wave works on at once

template <bool F16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    if constexpr (F16)
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a),
                                      __builtin_bit_cast(f16x2_t, b), c, false);
    else
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                               __builtin_bit_cast(bf16x2_t, b), c, false);
}

/* The sum of v over the 64 lanes, in every lane: the four DPP steps of a 16-lane row, then
 * the rows combined. */
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm 1,0,3,2
    v += dpp_f32<0x4E>(v);   // quad_perm 2,3,0,1
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

template <int BITS, int GS, bool F16, int MM>
__device__ __forceinline__ void qmv(const QmvParams& p) {
    constexpr int KPL = 128 / BITS;  // k a lane covers per step (16 bytes of codes)
    constexpr int IPC = KPL / 8;     // 16-byte x items per lane chunk
    constexpr int R = kQmvRows;
    static_assert(KPL <= GS, "a lane chunk lies in one group");
    uint8_t* lds = lds_base();
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = p.M, N = p.N, K = p.K;
    const int nchunk = K / KPL;
    const int nsteps = (nchunk + 63) / 64;
    const int bid = blockIdx.x;
    const int base = N / p.G, rem = N - base * p.G;
    const int row_lo = bid * base + min(bid, rem);
    const int nrows = base + (bid < rem ? 1 : 0);
    const int ngroups = (nrows + R - 1) / R;
    float* xsum = (float*)(lds + p.lds_xsum_off);
    float* out = (float*)(lds + p.lds_out_off);
    uint32_t* gcnt = (uint32_t*)(lds + p.lds_cnt_off);

    /* x to LDS (item = 8 consecutive k), pre-permuted, and each lane chunk's sum: the IPC
     * items of a chunk sit in aligned neighbouring lanes */
    {
        const int ipr = K / 8;
        const uint8_t* xg = (const uint8_t*)p.x;
        for (int it = tid; it < M * ipr; it += kQmvWaves * 64) {
            const int m = it / ipr, kk = it - m * ipr;
            const uint32_t off = ((uint32_t)m * (uint32_t)K + (uint32_t)kk * 8u) * 2u;
            const u32x4_t v = *(const u32x4_t*)(xg + off);
            float sm = chunk_dot<F16>(v, 0.0f);
            sm += dpp_f32<0xB1>(sm);                         // lanes ^1
            if constexpr (IPC == 4) sm += dpp_f32<0x4E>(sm);  // lanes ^2
            *(u32x4_t*)(lds + off) = (BITS == 4) ? nibble_permute(v) : v;
            if ((it & (IPC - 1)) == 0) xsum[m * nchunk + kk / IPC] = sm;
        }
        if (tid == 0) *gcnt = (uint32_t)kQmvWaves;  // groups below kQmvWaves go by wave index
    }
    __syncthreads();

    uint32_t magic = F16 ? 0x64006400u : 0x43004300u;
    uint32_t nmask = 0x000F000Fu;
    __asm__ volatile("" : "+v"(magic));  // opaque: keep in a VGPR (see nibble_operand)
    __asm__ volatile("" : "+s"(nmask));  // opaque: keep in an SGPR
    constexpr float kOff = (BITS == 4) ? (F16 ? 1024.0f : 128.0f) : 0.0f;
    const uint8_t* wg = (const uint8_t*)p.w;
    const uint16_t* sg = (const uint16_t*)p.scales;
    const uint16_t* bg = (const uint16_t*)p.biases;
    const uint32_t RB = (uint32_t)K * BITS / 8u;
    const uint32_t GPR = (uint32_t)(K / GS);

    int grp = wave;
    while (grp < ngroups) {
        /* the next group's index, taken now and needed after this group */
        uint32_t gn = 0;
        if (lane == 0)
            gn = __hip_atomic_fetch_add(gcnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        uint32_t rowoff[R], sboff[R];  // a row's first code byte and first scale (clamped rows)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = (uint32_t)(row_lo + min(grp * R + r, nrows - 1));
            rowoff[r] = row * RB;
            sboff[r] = row * GPR;
        }
        float acc[R][MM];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MM; ++m) acc[r][m] = 0.0f;
        u32x4_t wA[R], wB[R];
        uint32_t sA[R], bA[R], sB[R], bB[R];
        /* step j's codes, scales and biases; a lane past the row's last chunk reloads it */
        auto load = [&](u32x4_t (&wv)[R], uint32_t (&sv)[R], uint32_t (&bv)[R], int j) {
            const uint32_t c = (uint32_t)min(lane + 64 * j, nchunk - 1);
            const uint32_t g = c * KPL / GS;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                wv[r] = *(const u32x4_t*)(wg + rowoff[r] + c * 16u);
                sv[r] = sg[sboff[r] + g];
                bv[r] = bg[sboff[r] + g];
            }
        };
        auto compute = [&](const u32x4_t (&wv)[R], const uint32_t (&sv)[R],
                           const uint32_t (&bv)[R], int j) {
            const int c0 = lane + 64 * j;
            const bool act = c0 < nchunk;
            const int c = act ? c0 : nchunk - 1;
            float s[R], bp[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                s[r] = act ? elem_to_f32<F16>(sv[r]) : 0.0f;
                const float b = act ? elem_to_f32<F16>(bv[r]) : 0.0f;
                bp[r] = (kOff != 0.0f) ? __builtin_fmaf(-kOff, s[r], b) : b;
            }
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                if (m >= M) break;
                const uint8_t* xp = lds + ((uint32_t)m * (uint32_t)K + (uint32_t)c * KPL) * 2u;
                u32x4_t xv[IPC];
#pragma unroll
                for (int i = 0; i < IPC; ++i) xv[i] = *(const u32x4_t*)(xp + i * 16);
                const float X = xsum[m * nchunk + c];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float P = 0.0f;
#pragma unroll
                    for (int i = 0; i < IPC; ++i) {
                        u32x4_t B;
                        if constexpr (BITS == 4) B = nibble_operand<F16>(wv[r][i], nmask, magic);
                        else B = byte_operand<F16>(wv[r][2 * i], wv[r][2 * i + 1]);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t xe = xv[i][e], be = B[e];
                            P = dot2<F16>(xe, be, P);
                        }
                    }
                    acc[r][m] = __builtin_fmaf(s[r], P, acc[r][m]);
                    acc[r][m] = __builtin_fmaf(bp[r], X, acc[r][m]);
                }
                __builtin_amdgcn_sched_barrier(0);  // one x row at a time
            }
        };
        load(wA, sA, bA, 0);
        for (int j = 0; j < nsteps; j += 2) {
            __builtin_amdgcn_sched_barrier(0);
            load(wB, sB, bB, min(j + 1, nsteps - 1));  // always issued: exact vmcnt waits
            __builtin_amdgcn_sched_barrier(0);
            compute(wA, sA, bA, j);
            if (j + 1 >= nsteps) break;
            __builtin_amdgcn_sched_barrier(0);
            load(wA, sA, bA, min(j + 2, nsteps - 1));
            __builtin_amdgcn_sched_barrier(0);
            compute(wB, sB, bB, j + 1);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int rr = grp * R + r;
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                if (m >= M) break;
                const float v = wave_sum(acc[r][m]);
                if (lane == 0 && rr < nrows) out[m * p.rows_max + rr] = v;
            }
        }
        grp = (int)__builtin_amdgcn_readfirstlane(gn);
    }
    __syncthreads();
    /* the workgroup's outputs, plus the linear bias, rounded once */
    const uint16_t* lb = (const uint16_t*)p.lbias;
    uint16_t* y = (uint16_t*)p.y;
    for (int i = tid; i < M * nrows; i += kQmvWaves * 64) {
        const int m = i / nrows, rr = i - m * nrows;
        float v = out[m * p.rows_max + rr];
        if (lb) v += elem_to_f32<F16>(lb[row_lo + rr]);
        y[(size_t)m * N + row_lo + rr] = f32_to_out<F16>(v);
    }
}

}  // namespace

/* One 64-lane wave per output element (blockIdx.x = column n, blockIdx.y = row m). */
extern "C" __global__ void __launch_bounds__(64) dfq_qmm_generic(QmmGenericParams p) {
    const int n = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
    const int per = 32 / p.bits;
    const uint32_t mask = (1u << p.bits) - 1u;
    const int wpr = p.K / per, gpr = p.K / p.gs;
    const uint32_t* wr = p.w + (size_t)n * wpr;
    float acc = 0.0f;
    for (int j = lane; j < wpr; j += 64) {
        const uint32_t word = wr[j];
        const int g = (j * per) / p.gs;
        const float s = load_any(p.scales, p.sdt, (size_t)n * gpr + g);
        const float b = load_any(p.biases, p.sdt, (size_t)n * gpr + g);
        for (int t = 0; t < per; ++t) {
            const float wq = (float)((word >> (p.bits * t)) & mask) * s + b;
            acc += load_any(p.x, p.xdt, (size_t)m * p.K + (size_t)j * per + t) * wq;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) {
        if (p.lbias) acc += load_any(p.lbias, p.sdt, n);
        store_any(p.y, p.ydt, (size_t)m * p.N + n, acc);
    }
}

/* The packed layout of a 4/8-bit weight with its scales and biases, for the c8 kernels'
 * chunks of cg groups (8; 16 at 4-bit group 32), sb = cg / 8: unit (t, c) -- 16 rows of
 * tile t, chunk c of K -- at (t * chunks + c) * ub bytes, ub = cb + 512 sb.  Its codes are
 * cb / 1024 pieces of 1 KB: byte 16 * l of piece i holds the 16 bytes lane l = 16 q + n loads
 * for piece i from the MLX layout (row 16 t + n, bytes 64 i + 16 q of the chunk's codes).
 * Then 512 sb bytes: for qq = 0 (scales) and 1 (biases) and each row n, the chunk's groups
 * (16 sb bytes) at (16 qq + n) * 16 sb.  Rows past N are zeros.  One thread per 16-byte
 * piece; a pure byte permutation of the MLX arrays. */
extern "C" __global__ void __launch_bounds__(256) dfq_pack_weights(
    const uint8_t* w, const uint8_t* scales, const uint8_t* biases, uint8_t* packed, int N,
    int K, int bits, int gs, uint64_t pieces) {
    const uint32_t sbu = (bits == 4 && gs == 32) ? 2u : 1u;  // 16-byte scale pieces a row
    const uint32_t chunk_k = 8u * sbu * (uint32_t)gs;      // k of a chunk
    const uint32_t cb = 16u * chunk_k * (uint32_t)bits / 8u;  // code bytes of a unit
    const uint32_t ppu = (cb + 512u * sbu) / 16u;          // 16-byte pieces of a unit
    const uint32_t chunks = (uint32_t)K / chunk_k;
    const size_t rb = (size_t)K * bits / 8;                // bytes per weight row
    const size_t sb = (size_t)(K / gs) * 2;                // bytes per scale row
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < pieces;
         i += (uint64_t)gridDim.x * 256) {
        const uint64_t u = i / ppu;
        const uint32_t r = (uint32_t)(i - u * ppu);
        const uint32_t t = (uint32_t)(u / chunks), c = (uint32_t)(u - (uint64_t)t * chunks);
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (r < cb / 16u) {
            const uint32_t piece = r / 64u, l = r % 64u, q = l >> 4, n = l & 15u;
            const uint32_t row = t * 16u + n;
            if ((int)row < N)
                v = *(const u32x4_t*)(w + row * rb + (size_t)c * chunk_k * bits / 8 +
                                      piece * 64u + q * 16u);
        } else {
            const uint32_t k = r - cb / 16u, qq = k / (16u * sbu), rem = k - qq * 16u * sbu;
            const uint32_t n = rem / sbu, h = rem - n * sbu;
            const uint32_t row = t * 16u + n;
            if ((int)row < N)
                v = *(const u32x4_t*)((qq ? biases : scales) + row * sb +
                                      ((size_t)c * sbu + h) * 16u);
        }
        *(u32x4_t*)(packed + i * 16u) = v;
    }
}

/* Fill n uint32 words with v (workspace re-arm; no memset node is ever captured). */
extern "C" __global__ void __launch_bounds__(256) dfq_fill_u32(uint32_t* ptr, uint32_t v,
                                                                uint64_t count) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < count;
         i += (uint64_t)gridDim.x * 256)
        ptr[i] = v;
}

/* The fast kernel's own read, with no compute: the units of a one-k-block 4-bit group-64
 * split -- the same ranges, and per unit the same loads: one 16-byte scale-or-bias load a
 * lane and four 16-byte weight loads of 16 rows x 64 bytes -- taken in order by 12 waves, one
 * unit in flight each, XORed into one word per wave (sink[12 * range + wave]).  It is
 * the weight stream the matmul would reach if its x staging, arithmetic and output cost
 * nothing: the bound its own access pattern sets.  A wave issues nothing past its last unit
 * (a re-read of it there would hold the wave, and the launch's end, for one more round
 * trip). */
extern "C" __global__ void __launch_bounds__(768) dfq_read_units_b4_g64(QmmParams p,
                                                                         uint32_t* sink) {
    using C = Cfg<4, 64>;
    constexpr int CH = 8 / C::GPS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane >> 4, n = lane & 15;
    const KBlock kbk = kblock(p, 0);
    const int wr = xcd_order((int)blockIdx.x, (int)gridDim.x);  // this workgroup's range
    const int a = range_start(kbk, wr), b = range_start(kbk, wr + 1);
    const int SS = kbk.SS;
    const int RB = p.K / 2, GPR = p.K / 64;
    const uint8_t* wbytes = (const uint8_t*)p.w;
    const uint8_t* sbb = (const uint8_t*)((q & 1) ? p.biases : p.scales);
    u32x4_t acc = {0u, 0u, 0u, 0u};
    u32x4_t r[1 + CH];
    auto load = [&](int u) {
        const int t = u / SS, c = u - t * SS;
        const int row0 = t * 16;
        const int rl = (row0 + 16 <= p.N) ? n : min(n, p.N - 1 - row0);
        const int kc = c * (CH * C::KSS);
        r[0] = *(const u32x4_t*)(sbb + ((size_t)row0 * GPR + kc / 64) * 2 + (uint32_t)rl * GPR * 2u);
        const uint8_t* wb = wbytes + (size_t)row0 * RB + kc / 2 + (uint32_t)rl * RB + q * 16u;
#pragma unroll
        for (int j = 0; j < CH; ++j) r[1 + j] = *(const u32x4_t*)(wb + j * 64);
    };
    int u = a + wave;
    if (u < b) {
        load(u);
        for (; u < b; u += 12) {
#pragma unroll
            for (int j = 0; j < 1 + CH; ++j) acc ^= r[j];
            if (u + 12 >= b) break;
            __builtin_amdgcn_sched_barrier(0);
            load(u + 12);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (lane == 0) sink[wr * 12 + wave] = v;
}

/* The same read over a packed weight array: unit (t, c) is 4608 contiguous bytes at
 * (t * chunks + c) * 4608 -- its codes as four 1 KB pieces (load j of lane l at j * 1024 +
 * l * 16), then its 16 rows' scales and biases (512 bytes: lane (q, n) at ((q & 1) * 16 + n) *
 * 16) -- in the unpacked read's ranges, order and depth. */
extern "C" __global__ void __launch_bounds__(768) dfq_read_units_packed_b4_g64(QmmParams p,
                                                                                uint32_t* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane >> 4, n = lane & 15;
    const KBlock kbk = kblock(p, 0);
    const int wr = xcd_order((int)blockIdx.x, (int)gridDim.x);  // this workgroup's range
    const int a = range_start(kbk, wr), b = range_start(kbk, wr + 1);
    const uint8_t* pk = (const uint8_t*)p.w;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    u32x4_t r[5];
    auto load = [&](int u) {
        const uint8_t* ub = pk + (size_t)u * 4608;  // one k-block: u = t * chunks + c
        r[0] = *(const u32x4_t*)(ub + 4096 + ((q & 1) * 16 + n) * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) r[1 + j] = *(const u32x4_t*)(ub + j * 1024 + lane * 16);
    };
    int u = a + wave;
    if (u < b) {
        load(u);
        for (; u < b; u += 12) {
#pragma unroll
            for (int j = 0; j < 5; ++j) acc ^= r[j];
            if (u + 12 >= b) break;
            __builtin_amdgcn_sched_barrier(0);
            load(u + 12);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (lane == 0) sink[wr * 12 + wave] = v;
}

/* The read ceiling: a plain streaming read of `units` 4 KB blocks, the best single-launch
 * read this memory system does with nothing else in the kernel.  The blocks are dealt to
 * the waves round-robin (wave w of the grid reads blocks w, w + 8G, ...), so that at any
 * moment the whole GPU reads one window of neighbouring blocks; each wave keeps one block
 * (four 16-byte loads a lane, 1 KB per instruction; 32 KB a CU) in flight and XORs what it
 * read into one word per wave (sink[8 * blockIdx.x + wave]) so that no load is dead.  Past
 * its last block a wave re-reads that block (an L2 hit), so every pass of the loop has the
 * same loads in flight.  Measured on MI355X for 50.5 MB per launch: 9.47 us, against 10.23
 * us when each wave reads a contiguous range (2048 streams far apart) and 10.30 us with
 * 64 KB a CU in flight. */
extern "C" __global__ void __launch_bounds__(512) dfq_read_stream(const u32x4_t* src,
                                                                  uint64_t units,
                                                                  uint32_t* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t nw = (uint64_t)gridDim.x * 8, gw = (uint64_t)blockIdx.x * 8 + wave;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    if (gw < units) {
        u32x4_t buf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) buf[j] = src[gw * 256 + j * 64 + lane];
        for (uint64_t u = gw; u < units; u += nw) {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc ^= buf[j];
            const uint64_t nu = (u + nw < units) ? u + nw : u;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j) buf[j] = src[nu * 256 + j * 64 + lane];
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (lane == 0) sink[gw] = v;
}

/* h[m][n] = silu(g) * u with g = gu[m][n], u = gu[m][N + n] (gu row pitch 2N), in fp32,
 * rounded once to the output dtype. */
template <bool F16>
__device__ __forceinline__ void silu_mul(const uint16_t* gu, uint16_t* h, int M, int N,
                                         int64_t first, int64_t stride) {
    const int64_t total = (int64_t)M * N;
    for (int64_t i = first; i < total; i += stride) {
        const int64_t m = i / N, n = i - m * N;
        const float g = elem_to_f32<F16>(gu[m * 2 * N + n]);
        const float u = elem_to_f32<F16>(gu[m * 2 * N + N + n]);
        put16(h + i, silu_mul_round<F16>(g, u));
    }
}
extern "C" __global__ void __launch_bounds__(256) dfq_silu_mul_bf16(const uint16_t* gu,
                                                                    uint16_t* h, int M, int N) {
    silu_mul<false>(gu, h, M, N, (int64_t)blockIdx.x * 256 + threadIdx.x,
                    (int64_t)gridDim.x * 256);
}
extern "C" __global__ void __launch_bounds__(256) dfq_silu_mul_f16(const uint16_t* gu,
                                                                   uint16_t* h, int M, int N) {
    silu_mul<true>(gu, h, M, N, (int64_t)blockIdx.x * 256 + threadIdx.x,
                   (int64_t)gridDim.x * 256);
}

/* Greedy accept of a verify pass (the reference's acceptedPrefix).  Blocks of one row cover
 * DFQ_ACCEPT_CHUNK of its V logits; each folds its chunk's maximum into the row's 64-bit key
 * with an agent-scope atomic max: the high word is the logit's bits made order-preserving
 * (sign flip or full flip for negatives), the low word is ~index, so the largest key is the
 * largest logit and, among equal logits, the first index (MLX's argMax).  NaN logits are
 * skipped.  The last block to arrive (counter) turns the keys into tokens, finds the leading
 * run of tokens[i] == proposals[i] (i < M-1), writes both, and re-arms keys and counter.
 *
 * A thread issues all of its 16-byte loads before using any (rows 16-byte aligned: V a
 * multiple of 8); other rows take 2-byte loads, four in flight.  Keys are only touched by
 * agent-scope atomics, so a block's max is visible to the last block once it has completed
 * (vmcnt) before the block's relaxed counter increment: no cache write-back or invalidate. */
template <bool F16>
__device__ __forceinline__ void argmax_accept(const uint16_t* logits, int M, int V,
                                              const int32_t* proposals, int32_t* tokens,
                                              int32_t* accepted, uint64_t* keys,
                                              uint32_t* counter) {
    constexpr int C = DFQ_ACCEPT_CHUNK;
    const int tid = threadIdx.x;
    const int per_row = (V + C - 1) / C;
    const int row = blockIdx.x / per_row, c = blockIdx.x - row * per_row;
    const int lo = c * C, hi = min(V, lo + C);
    const uint16_t* lr = logits + (size_t)row * V;
    uint64_t best = 0;
    if ((V & 7) == 0 && ((uintptr_t)logits & 15) == 0) {
        constexpr int UN = C / 2048;  // 16-byte loads a thread, all in flight before any use
        u32x4_t v[UN];
#pragma unroll
        for (int u = 0; u < UN; ++u) {
            const int i = lo + (u * 256 + tid) * 8;
            if (i < hi) v[u] = *(const u32x4_t*)(lr + i);
        }
#pragma unroll
        for (int u = 0; u < UN; ++u) {
            const int i = lo + (u * 256 + tid) * 8;
            if (i >= hi) continue;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f = elem_to_f32<F16>((uint16_t)(v[u][e >> 1] >> (16 * (e & 1))));
                if (f != f) continue;
                const uint64_t k = argmax_key(f, i + e);
                best = k > best ? k : best;
            }
        }
    } else {
#pragma unroll 4
        for (int i = lo + tid; i < hi; i += 256) {
            const float f = elem_to_f32<F16>(lr[i]);
            if (f != f) continue;
            const uint64_t k = argmax_key(f, i);
            best = k > best ? k : best;
        }
    }
    best = max_key_wave(best);
    __shared__ uint64_t wbest[4];
    __shared__ uint32_t last;
    __shared__ int first_bad;
    if ((tid & 63) == 0) wbest[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        uint64_t b = wbest[0];
        for (int w = 1; w < 4; ++w) b = wbest[w] > b ? wbest[w] : b;
        if (b) __hip_atomic_fetch_max(keys + row, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const uint32_t n = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        last = (n + 1 == gridDim.x) ? 1u : 0u;
        first_bad = M - 1;
    }
    __syncthreads();
    if (!last) return;
    for (int m = tid; m < M; m += 256) {
        /* the proposal and the key in flight together */
        const int32_t prop = (proposals && m < M - 1) ? proposals[m] : 0;
        const uint64_t k = __hip_atomic_exchange(keys + m, 0ull, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
        const int32_t tok = k ? (int32_t)~(uint32_t)k : -1;
        if (tokens) tokens[m] = tok;
        if (m < M - 1 && !(proposals && prop == tok)) atomicMin(&first_bad, m);
    }
    __syncthreads();
    if (tid == 0) {
        if (accepted) *accepted = first_bad;
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

extern "C" __global__ void __launch_bounds__(256) dfq_argmax_accept_bf16(
    const uint16_t* logits, int M, int V, const int32_t* proposals, int32_t* tokens,
    int32_t* accepted, uint64_t* keys, uint32_t* counter) {
    argmax_accept<false>(logits, M, V, proposals, tokens, accepted, keys, counter);
}
extern "C" __global__ void __launch_bounds__(256) dfq_argmax_accept_f16(
    const uint16_t* logits, int M, int V, const int32_t* proposals, int32_t* tokens,
    int32_t* accepted, uint64_t* keys, uint32_t* counter) {
    argmax_accept<true>(logits, M, V, proposals, tokens, accepted, keys, counter);
}

/* The second pass of a split whose tiles can have more than two contributors (several
 * k-blocks, or tiles spread over three or more workgroups): one wave per 16-column tile. */
template <bool F16>
__device__ __forceinline__ void qmm_reduce(const QmmParams& p) {
    /* Every parameter the pass reads, fetched in one go: left to itself the compiler fetches
     * each where it is first used, three dependent scalar round trips before the first slot
     * load (C3 18.6 -> 18.5 us, M=16 20.9 -> 20.2 us). */
    int nkb = p.nkb, nslot = p.nslot_kb, mt = p.mt, M = p.M, N = p.N, epi = p.epi, T = p.T;
    int chunks = p.chunks, Gkb = p.Gkb, al = p.aligned;
    const void* y = p.y;
    const void* lb = p.lbias;
    const float* sl = p.slots;
    __asm__ volatile("" ::"s"(nkb), "s"(nslot), "s"(mt), "s"(M), "s"(N), "s"(epi), "s"(T),
                     "s"(chunks), "s"(Gkb), "s"(al), "s"(y), "s"(lb), "s"(sl));
    reduce_tile<F16>(p, blockIdx.x, threadIdx.x);
}

extern "C" __global__ void __launch_bounds__(64) dfq_qmm_reduce_bf16(QmmParams p) {
    qmm_reduce<false>(p);
}
extern "C" __global__ void __launch_bounds__(64) dfq_qmm_reduce_f16(QmmParams p) {
    qmm_reduce<true>(p);
}

/* Chunks in flight per wave: enough to keep DFQ_PF_LOADS weight loads per lane
 * outstanding, at least 1 and at most 8.  Measured on the headline shape, one 4 KB chunk per
 * wave (about 48 KB per CU with scales and biases) streams faster than two or more: deeper
 * queues only add latency. */
template <int BITS, int GS, int CH>
constexpr int prefetch_depth() {
    constexpr int loads = CH * Cfg<BITS, GS>::NS;
    constexpr int d = DFQ_PF_LOADS / loads;
    return d < 1 ? 1 : (d > 8 ? 8 : d);
}

#define DFQ_MT8_KERNEL(BITS, GS, F16, NAME, CHN, CH, MTN, MT, AM, PK, SFX)                 \
    extern "C" __global__ void __launch_bounds__(kBlock)                                     \
        dfq_qmm_##MTN##_b##BITS##_g##GS##_##NAME##_##CHN##SFX(QmmParams p) {                  \
        qmm_mt8<BITS, GS, F16, CH, prefetch_depth<BITS, GS, CH>(), MT, AM, PK>(               \
            p, launch_order(p, (int)blockIdx.x, (int)gridDim.x));                             \
    }
/* per format: one super-step or 8-group chunks at up to 8 rows; 8-group chunks at up to 16;
 * the greedy-accept forms (_am) of the 8-group-chunk kernels; and all of the 8-group-chunk
 * kernels again over the packed layout (_pk).  4-bit group 32 also has 16-group chunks at up
 * to 8 rows (c16, in every form); at 16 rows they would need more than the 128 VGPRs a
 * 14-wave workgroup allows (about 90 spilled), so 9..16 rows keep 8-group chunks. */
#define DFQ_MT8_FORMAT(BITS, GS, F16, NAME)                                                    \
    DFQ_MT8_KERNEL(BITS, GS, F16, NAME, c1, 1, mt8, 1, false, false, )                        \
    DFQ_MT8_KERNEL(BITS, GS, F16, NAME, c8, (8 / Cfg<BITS, GS>::GPS), mt8, 1, false, false, ) \
    DFQ_MT8_KERNEL(BITS, GS, F16, NAME, c8, (8 / Cfg<BITS, GS>::GPS), mt16, 2, false, false, )\
    DFQ_MT8_KERNEL(BITS, GS, F16, NAME, c8, (8 / Cfg<BITS, GS>::GPS), mt8, 1, true, false, _am)\
    DFQ_MT8_KERNEL(BITS, GS, F16, NAME, c8, (8 / Cfg<BITS, GS>::GPS), mt16, 2, true, false,    \
                   _am)                                                                        \
    DFQ_MT8_KERNEL(BITS, GS, F16, NAME, c8, (8 / Cfg<BITS, GS>::GPS), mt8, 1, false, true, _pk)\
    DFQ_MT8_KERNEL(BITS, GS, F16, NAME, c8, (8 / Cfg<BITS, GS>::GPS), mt16, 2, false, true,    \
                   _pk)                                                                        \
    DFQ_MT8_KERNEL(BITS, GS, F16, NAME, c8, (8 / Cfg<BITS, GS>::GPS), mt8, 1, true, true,      \
                   _am_pk)                                                                     \
    DFQ_MT8_KERNEL(BITS, GS, F16, NAME, c8, (8 / Cfg<BITS, GS>::GPS), mt16, 2, true, true,     \
                   _am_pk)

#define DFQ_MT8_C16(F16, NAME)                                                                 \
    DFQ_MT8_KERNEL(4, 32, F16, NAME, c16, 4, mt8, 1, false, false, )                          \
    DFQ_MT8_KERNEL(4, 32, F16, NAME, c16, 4, mt8, 1, true, false, _am)                        \
    DFQ_MT8_KERNEL(4, 32, F16, NAME, c16, 4, mt8, 1, false, true, _pk)                        \
    DFQ_MT8_KERNEL(4, 32, F16, NAME, c16, 4, mt8, 1, true, true, _am_pk)

DFQ_MT8_C16(false, bf16)
DFQ_MT8_C16(true, f16)
DFQ_MT8_FORMAT(4, 32, false, bf16)
DFQ_MT8_FORMAT(4, 64, false, bf16)
DFQ_MT8_FORMAT(4, 128, false, bf16)
DFQ_MT8_FORMAT(8, 32, false, bf16)
DFQ_MT8_FORMAT(8, 64, false, bf16)
DFQ_MT8_FORMAT(8, 128, false, bf16)
DFQ_MT8_FORMAT(4, 32, true, f16)
DFQ_MT8_FORMAT(4, 64, true, f16)
DFQ_MT8_FORMAT(4, 128, true, f16)
DFQ_MT8_FORMAT(8, 32, true, f16)
DFQ_MT8_FORMAT(8, 64, true, f16)
DFQ_MT8_FORMAT(8, 128, true, f16)

/* The stock path's few-row GEMV, per format: one row (decode) and up to four. */
#define DFQ_QMV_KERNEL(BITS, GS, F16, NAME, MM)                                                \
    extern "C" __global__ void __launch_bounds__(kQmvWaves * 64)                               \
        dfq_qmv_b##BITS##_g##GS##_##NAME##_m##MM(QmvParams p) {                               \
        qmv<BITS, GS, F16, MM>(p);                                                             \
    }
#define DFQ_QMV_FORMAT(BITS, GS, F16, NAME) \
    DFQ_QMV_KERNEL(BITS, GS, F16, NAME, 1)  \
    DFQ_QMV_KERNEL(BITS, GS, F16, NAME, 4)

DFQ_QMV_FORMAT(4, 32, false, bf16)
DFQ_QMV_FORMAT(4, 64, false, bf16)
DFQ_QMV_FORMAT(4, 128, false, bf16)
DFQ_QMV_FORMAT(8, 32, false, bf16)
DFQ_QMV_FORMAT(8, 64, false, bf16)
DFQ_QMV_FORMAT(8, 128, false, bf16)
DFQ_QMV_FORMAT(4, 32, true, f16)
DFQ_QMV_FORMAT(4, 64, true, f16)
DFQ_QMV_FORMAT(4, 128, true, f16)
DFQ_QMV_FORMAT(8, 32, true, f16)
DFQ_QMV_FORMAT(8, 64, true, f16)
DFQ_QMV_FORMAT(8, 128, true, f16)
