// Device primitives of the EXL3 trellis decoder for gfx950 (CDNA4, wave64).
//
// Format (reference docs/FORMAT.md:42-86, python/strix_trellis/codec.py:12-101):
//   * a 16x16 tile holds 256 states in a ring of 256*K bits = 8K little-endian
//     uint32 words (lo16 | hi16 << 16); the stream reads bit 31 of each word first;
//   * state p (p = 8t + f, t = 0..31, f = 0..7) is the 16 ring bits ending at
//     bit (p+1)*K, MSB first; state 0's window wraps to the end of the same tile;
//   * state p sits at row 2(t%4) + f%2 + 8((f/2)%2), column t/4 + 8(f/4).
//
// Work split used by every kernel here.  One lane owns a "chunk" of K
// consecutive words of a tile: chunk g (0..7) holds the states of fragment
// lanes t = 4g..4g+3.  Those 32 states cover all 16 rows of tile columns g and
// g+8, so a lane can finish a 16-deep dot product for two output columns
// without any cross-lane reduction.  Eight lanes cover one tile, a wave64
// covers eight tiles that are adjacent in memory (one 128-column output group
// of one 16-row input block): K*256 contiguous bytes per wave, K dwords per lane.
// The 16 - K ring bits before a chunk are the last word of the previous chunk
// (chunk 7 for chunk 0, the wrap), fetched with two DPP moves.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace stx {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum Codebook { CB_3INST = 0, CB_MCG = 1, CB_MUL1 = 2 };

// Raw buffer resource for gfx9-family loads: out-of-range offsets read zero
// instead of faulting, so a wrong index can never touch foreign memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Load through a global-address-space pointer.  Pointers that arrive through
// structs are generic to the compiler, which would emit FLAT loads; those
// count on both vmcnt and lgkmcnt and force full waits.
template <class T>
__device__ __forceinline__ T ld_global(const T* p) {
    return *(const __attribute__((address_space(1))) T*)(p);
}

// Keep an FP32 value in a register so that a later FP32->FP16 conversion is a
// separate rounding (stops LLVM from forming mixed-precision ops that round
// once from the wider value).
__device__ __forceinline__ float rn32(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ uint32_t as_u32(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// ---------------------------------------------------------------------------
// Chunk: the K words of one lane plus the word before them.
// ---------------------------------------------------------------------------
template <int K>
struct Chunk {
    uint32_t d[K];   // stream order: d[0] is read first
    uint32_t prev;   // ring word preceding d[0]

    // Word by position counted from the least significant end of the big
    // number prev:d[0]:...:d[K-1]; q = K is prev.
    template <int Q>
    __device__ __forceinline__ uint32_t lsb() const {
        if constexpr (Q < K) return d[K - 1 - Q];
        else return prev;
    }
};

// Load chunk g of the tile that starts at byte offset `tile_byte` of `rsrc`:
// the lane's byte offset is voff + soff, soff a wave-uniform part (an SGPR
// operand of the load, so a loop can advance it without vector arithmetic).
template <int K>
__device__ __forceinline__ void load_chunk(Chunk<K>& c, __amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff = 0) {
    // voff + soff = tile_byte + 4*K*g: 16-byte aligned for K = 4, 8; 4-byte otherwise.
    if constexpr (K == 1) {
        c.d[0] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, voff, soff, 0);
    } else if constexpr (K == 2) {
        u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rsrc, voff, soff, 0);
        c.d[0] = v.x; c.d[1] = v.y;
    } else if constexpr (K == 3) {
        u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(rsrc, voff, soff, 0);
        c.d[0] = v.x; c.d[1] = v.y; c.d[2] = v.z;
    } else {
        u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, soff, 0);
        c.d[0] = v.x; c.d[1] = v.y; c.d[2] = v.z; c.d[3] = v.w;
        if constexpr (K == 5) {
            c.d[4] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, voff + 16, soff, 0);
        } else if constexpr (K == 6) {
            u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rsrc, voff + 16, soff, 0);
            c.d[4] = w.x; c.d[5] = w.y;
        } else if constexpr (K == 7) {
            u32x3 w = __builtin_amdgcn_raw_buffer_load_b96(rsrc, voff + 16, soff, 0);
            c.d[4] = w.x; c.d[5] = w.y; c.d[6] = w.z;
        } else if constexpr (K == 8) {
            u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff + 16, soff, 0);
            c.d[4] = w.x; c.d[5] = w.y; c.d[6] = w.z; c.d[7] = w.w;
        }
    }
}

// prev = last word of chunk g-1 of the same tile, or of chunk 7 for g = 0.
// Lanes 8j..8j+7 hold the chunks of one tile, so both sources sit in the same
// DPP row of 16 lanes: row_shr:1 gives lane-1, row_shl:7 gives lane+7.
template <int K>
__device__ __forceinline__ void link_chunk(Chunk<K>& c, bool first_of_tile) {
    const uint32_t last = c.d[K - 1];
    const uint32_t left = __builtin_amdgcn_mov_dpp(last, 0x111, 0xf, 0xf, false);   // row_shr:1
    const uint32_t wrap = __builtin_amdgcn_mov_dpp(last, 0x107, 0xf, 0xf, false);   // row_shl:7
    c.prev = first_of_tile ? wrap : left;
}

// ---------------------------------------------------------------------------
// Window of the state at chunk position (V, F): fragment lane 4g+V, fragment F.
// Its 16 bits end (8V+F+1)*K bits after the chunk start.  Returns a register
// whose low (HI = false) or high (HI = true) 16 bits are the state; the other
// half is don't-care, because every consumer reads 16-bit operands.  Two
// windows 16 bits apart share one v_alignbit (K = 2, 4, 8).  Other widths have
// no such pairs, so their windows take the high half only where it is a word's
// own high half (no v_alignbit); a v_pk_* product of a high half counts as a
// high-half write for the compiler, whose next reader then waits a state.
// ---------------------------------------------------------------------------
template <int K, int V, int F>
struct Window {
    static constexpr int end = (8 * V + F + 1) * K;
    static constexpr int shift = 32 * K - end;   // distance of the window LSB from the chunk LSB
    static constexpr int q = shift / 32;
    static constexpr int r = shift % 32;
    static constexpr bool hi = r == 16 || (r > 16 && 16 % K == 0);
    static constexpr int align = hi ? r - 16 : r;

    __device__ __forceinline__ static uint32_t reg(const Chunk<K>& c) {
        if constexpr (align == 0) {
            return c.template lsb<q>();
        } else {
            return __builtin_amdgcn_alignbit(c.template lsb<q + 1>(), c.template lsb<q>(), align);
        }
    }
};

// ---------------------------------------------------------------------------
// Codebook products p = state * M (+ C) mod 2^32 on a 16-bit half-register
// operand: p = lo16(s)*M_lo + ((lo16(s)*M_hi mod 2^16) << 16) (+ C).
// v_pk_mul_lo_u16 with op_sel produces the shifted high product directly and
// v_mad_u32_u16 ignores the upper half of its 16-bit operands.
// ---------------------------------------------------------------------------
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

template <uint32_t M, bool HI>
__device__ __forceinline__ uint32_t product16(uint32_t src) {
    constexpr uint32_t mlo = M & 0xFFFFu;
    const u16x2 sv = __builtin_bit_cast(u16x2, src);
    const unsigned short s = HI ? sv.y : sv.x;
    const u16x2 splat = {s, s};
    const u16x2 mhi = {0, (unsigned short)(M >> 16)};
    // (0, s*M_hi mod 2^16): the compiler selects v_pk_mul_lo_u16 with op_sel.
    const uint32_t hs = __builtin_bit_cast(uint32_t, splat * mhi);
    uint32_t p;
    if constexpr (!HI) {
        asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(p) : "v"(src), "s"(mlo), "v"(hs));
    } else {
        asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(p) : "v"(src), "s"(mlo), "v"(hs));
    }
    return p;
}

constexpr uint32_t MUL1_M = 0x83DCD12Du;
constexpr uint32_t MCG_M = 0xCBAC1FEDu;
constexpr uint32_t INST3_M = 89226354u;
constexpr uint32_t INST3_C = 64248484u;

template <int CB, bool HI>
__device__ __forceinline__ uint32_t codebook_product(uint32_t src) {
    if constexpr (CB == CB_MUL1) return product16<MUL1_M, HI>(src);
    else if constexpr (CB == CB_MCG) return product16<MCG_M, HI>(src);
    else return product16<INST3_M, HI>(src) + INST3_C;
}

// mul1: b = sum of the four bytes of p; value = RN16((1024+b)*h(0x1EEE) + h(0xC931))
// with one rounding (reference docs/FORMAT.md:80-86).  The binary16 pattern of
// the integer 1024+b (b <= 1020) is 0x6400 + b, so v_sad_u8 / v_sad_hi_u8
// build both halves of a half2 and one v_pk_fma_f16 finishes two weights.
__device__ __forceinline__ half2_t mul1_pair(uint32_t pa, uint32_t pb) {
    const uint32_t lo = __builtin_amdgcn_sad_u8(pa, 0u, 0x64006400u);
    const uint32_t both = __builtin_amdgcn_sad_hi_u8(pb, 0u, lo);
    const half2_t scale = as_h2(0x1EEE1EEEu);
    const half2_t offset = as_h2(0xC931C931u);
    return __builtin_elementwise_fma(as_h2(both), scale, offset);
}

// 3inst / mcg: q = (p & 0x8FFF8FFF) ^ 0x3B603B60, value = RN16(h(q.lo) + h(q.hi)).
// Both halves are finite binary16 with exponents 12..15, so one FP16 add is
// the exact sum rounded once.
__device__ __forceinline__ _Float16 halves_value(uint32_t p) {
    const half2_t h = as_h2((p & 0x8FFF8FFFu) ^ 0x3B603B60u);
    return h.x + h.y;
}

// Decode the pair of states (V, F) and (V, F+1) of a chunk.
template <int K, int CB, int V, int F>
__device__ __forceinline__ half2_t decode_pair(const Chunk<K>& c) {
    using A = Window<K, V, F>;
    using B = Window<K, V, F + 1>;
    const uint32_t pa = codebook_product<CB, A::hi>(A::reg(c));
    const uint32_t pb = codebook_product<CB, B::hi>(B::reg(c));
    if constexpr (CB == CB_MUL1) {
        return mul1_pair(pa, pb);
    } else {
        half2_t r;
        r.x = halves_value(pa);
        r.y = halves_value(pb);
        return r;
    }
}

// All 32 weights of a chunk as 16 half2 registers, grouped for the dot:
//   w[V][0] = rows (2V, 2V+1),   column g      w[V][1] = rows (2V+8, 2V+9), column g
//   w[V][2] = rows (2V, 2V+1),   column g+8    w[V][3] = rows (2V+8, 2V+9), column g+8
template <int K, int CB>
__device__ __forceinline__ void decode_chunk(const Chunk<K>& c, half2_t (&w)[4][4]) {
#define STX_DECODE_V(V)                                   \
    w[V][0] = decode_pair<K, CB, V, 0>(c);                \
    w[V][1] = decode_pair<K, CB, V, 2>(c);                \
    w[V][2] = decode_pair<K, CB, V, 4>(c);                \
    w[V][3] = decode_pair<K, CB, V, 6>(c);
    STX_DECODE_V(0)
    STX_DECODE_V(1)
    STX_DECODE_V(2)
    STX_DECODE_V(3)
#undef STX_DECODE_V
}

// Pair q (0..15) of decode_chunk: w[q / 4][q % 4] (runtime-unrolled callers
// pass a constant q).
template <int K, int CB>
__device__ __forceinline__ void decode_pair_at(const Chunk<K>& c, half2_t (&w)[4][4], int q) {
#define STX_PAIR(Q) \
    if (q == Q) w[Q / 4][Q % 4] = decode_pair<K, CB, Q / 4, 2 * (Q % 4)>(c);
    STX_PAIR(0) STX_PAIR(1) STX_PAIR(2) STX_PAIR(3) STX_PAIR(4) STX_PAIR(5) STX_PAIR(6) STX_PAIR(7)
    STX_PAIR(8) STX_PAIR(9) STX_PAIR(10) STX_PAIR(11) STX_PAIR(12) STX_PAIR(13) STX_PAIR(14) STX_PAIR(15)
#undef STX_PAIR
}

// Bytes of one tile and of one 16-row block of tiles.
template <int K>
struct Geometry {
    static constexpr uint32_t tile_bytes = 32u * K;
    static constexpr uint32_t chunk_bytes = 4u * K;
};

}  // namespace stx
