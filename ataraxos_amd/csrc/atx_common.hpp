// Shared helpers of the gfx950 attention library: error reporting on the
// host, vector types and MFMA wrappers on the device.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ataraxos_attn.h"

namespace atx {

// ---------------------------------------------------------------------------
// Host: thread-local error text behind atx_last_error().
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Records `code` with a formatted message and returns it.
#define ATX_FAIL(code, ...)            \
    do {                               \
        ::atx::set_error(__VA_ARGS__); \
        return (code);                 \
    } while (0)

// Launch check: converts a HIP error after a launch into ATX_ERR_LAUNCH.
#define ATX_CHECK_LAUNCH(what)                                                \
    do {                                                                      \
        hipError_t e_ = hipGetLastError();                                    \
        if (e_ != hipSuccess)                                                 \
            ATX_FAIL(ATX_ERR_LAUNCH, "%s: %s", (what), hipGetErrorString(e_)); \
    } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Attention dropout (host and device).
// Element (b, h, i, j) of the [B, H, S_q, S_kv] attention weights is kept
// when drop_hash(((b * H + h) * S_q + i) * S_kv + j) >= thresh, thresh =
// floor(p * 2^32); kept weights are scaled by 1 / (1 - p).  The hash mixes
// the index's two 32-bit halves with a 64-bit key derived from the caller's
// (seed, offset) (splitmix64) and finishes with MurmurHash3's fmix32.  For a
// fixed key and upper half the map from the lower 32 index bits to hashes is
// a bijection.  The forward, the backward and atx_dropout_mask all call this
// one function, so they agree on every element.
// ---------------------------------------------------------------------------
__host__ __device__ inline uint32_t fmix32(uint32_t h) {
    h ^= h >> 16;
    h *= 0x85EBCA6Bu;
    h ^= h >> 13;
    h *= 0xC2B2AE35u;
    h ^= h >> 16;
    return h;
}
__host__ __device__ inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
struct DropKey {
    uint32_t k0, k1;  // the 64-bit key's halves
    uint32_t thresh;  // keep when hash >= thresh
    float scale;      // 1 / (1 - p)
};
__host__ __device__ inline uint32_t drop_hash(uint64_t idx, uint32_t k0, uint32_t k1) {
    uint32_t h = ((uint32_t)idx ^ k0) * 0x9E3779B1u;
    h ^= ((uint32_t)(idx >> 32) ^ k1) * 0x85EBCA77u;
    return fmix32(h);
}
inline DropKey make_drop_key(float p, uint64_t seed, uint64_t offset) {
    const uint64_t key = splitmix64(seed ^ splitmix64(offset));
    DropKey d;
    d.k0 = (uint32_t)key;
    d.k1 = (uint32_t)(key >> 32);
    const double t = (double)p * 4294967296.0;
    d.thresh = t >= 4294967295.0 ? 0xFFFFFFFFu : (uint32_t)t;
    d.scale = p > 0.f ? 1.f / (1.f - p) : 1.f;
    return d;
}

// ---------------------------------------------------------------------------
// Device: vector types.
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Streaming variants (nontemporal hint) for data touched exactly once.  On
// MI355X a streaming store pays off only when each store instruction writes
// whole 128-byte lines (measured: whole lines 214 us vs 229 us plain for the
// attention traffic of C3; half lines per instruction 235 us), which is how
// the attention kernel stages its output rows.
#ifndef ATX_STREAM_LOADS
#define ATX_STREAM_LOADS 1
#endif
#ifndef ATX_STREAM_STORES
#define ATX_STREAM_STORES 1
#endif

constexpr float kLog2e = 1.4426950408889634f;

// 16-bit element types that run on the 16x16x32 MFMA.
template <typename T>
struct Mfma16;

template <>
struct Mfma16<__bf16> {
    static constexpr int kDtype = ATX_DTYPE_BF16;
    static constexpr uint32_t kOnes2 = 0x3F803F80u;  // two packed 1.0
    __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    // Two floats -> packed pair, round to nearest even (v_cvt_pk_bf16_f32).
    __device__ static inline uint32_t pack2(float lo, float hi) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        bf16x2 r;
        r[0] = static_cast<__bf16>(lo);
        r[1] = static_cast<__bf16>(hi);
        return __builtin_bit_cast(uint32_t, r);
    }
    __device__ static inline float to_float(uint16_t bits) {
        return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
    }
    // c + a.lo * b.lo + a.hi * b.hi over packed pairs (v_dot2_f32_bf16).
    __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
    }
};

template <>
struct Mfma16<_Float16> {
    static constexpr int kDtype = ATX_DTYPE_FP16;
    static constexpr uint32_t kOnes2 = 0x3C003C00u;  // two packed 1.0
    __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                     __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    __device__ static inline uint32_t pack2(float lo, float hi) {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        f16x2 r;
        r[0] = static_cast<_Float16>(lo);
        r[1] = static_cast<_Float16>(hi);
        return __builtin_bit_cast(uint32_t, r);
    }
    __device__ static inline float to_float(uint16_t bits) {
        return static_cast<float>(__builtin_bit_cast(_Float16, bits));
    }
    // c + a.lo * b.lo + a.hi * b.hi over packed pairs (v_dot2_f32_f16).
    __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
    }
};

// Reinterpret a 16-byte chunk as four floats.  The whole vector is cast and
// then indexed: hipcc's __builtin_bit_cast applied to one element of an
// ext_vector_type (bit_cast<float>(v[i])) yields element 0 for every i.
__device__ inline f32x4 as_f32x4(u32x4 v) { return __builtin_bit_cast(f32x4, v); }

__device__ inline f32x4 mma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Lane-level helpers (wave64).
__device__ inline int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

__device__ inline float shfl_xor(float v, int mask) {
    int l = lane_id();
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((l ^ mask) << 2, __builtin_bit_cast(int, v)));
}

// Max / sum over the four lanes {l, l^16, l^32, l^48} that share an MFMA
// output column, with gfx950's lane-swap instructions (no LDS round trip).
// v_permlane16_swap a, b swaps the odd 16-lane rows of a with the even rows of
// b; applied to two copies of v it leaves v[l] in one register and v[l ^ 16]
// in the other (which one depends on l; max and the commutative add do not
// see the order).  v_permlane32_swap pairs l and l ^ 32 the same way.  The
// sum is (v[l] + v[l^16]) + (v[l^32] + v[l^48]) in every lane.  (Inline asm:
// this compiler's builtins for these instructions return the first register
// for both results.  The s_nops cover the VALU-write-to-permlane hazard on
// each side, which the compiler does not track through asm.)
__device__ inline void lane_swap16(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ inline void lane_swap32(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
// Sum over the 16 lanes of a row (lanes 16r .. 16r + 15), every lane getting
// the row's total: DPP butterflies (xor 1, xor 2 within quads, then the
// half-row and row mirrors), VALU only.
template <int CTRL>
__device__ inline float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ inline float row16_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    return v + dpp_mov<0x140>(v);  // row_mirror
}

__device__ inline float colgroup_max(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    lane_swap16(a, b);
    v = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    a = b = __builtin_bit_cast(uint32_t, v);
    lane_swap32(a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ inline float colgroup_sum(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    lane_swap16(a, b);
    v = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
    a = b = __builtin_bit_cast(uint32_t, v);
    lane_swap32(a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Raw buffer access through a per-tensor descriptor (gfx9 dword 3 =
// 0x00020000).  A load whose offset lies past `bytes` returns zero and such a
// store is dropped, so tile edges need neither clamps nor predicates.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ inline rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
constexpr int kAuxNt = 2;   // cache-policy bit of the streaming (nontemporal) hint
constexpr int kAuxGlc = 1;  // globally coherent: the load bypasses the CU's L1
__device__ inline u32x4 buf_ld16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, ATX_STREAM_LOADS ? kAuxNt : 0);
}
// Load without the streaming hint, for data many workgroups re-read (weights).
__device__ inline u32x4 buf_ld16_keep(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0); }
__device__ inline void buf_st16(rsrc_t r, uint32_t off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, ATX_STREAM_STORES ? kAuxNt : 0);
}
// Stores without the streaming hint (L2 keeps the line and merges the
// pieces of partly written lines before writing back).
__device__ inline void buf_st16_cached(rsrc_t r, uint32_t off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, 0);
}
__device__ inline void buf_st8_cached(rsrc_t r, uint32_t off, u32x2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)off, 0, 0);
}
__device__ inline void buf_st4_cached(rsrc_t r, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, (int)off, 0, 0);
}

// LDS byte pointer.  Kernels address their shared memory through this type so
// that every access stays a ds_* instruction.
typedef __attribute__((address_space(3))) char lds_t;

__device__ inline lds_t* lds_base() {
    extern __shared__ __attribute__((aligned(16))) char smem_dyn[];
    return (lds_t*)smem_dyn;  // generic -> LDS address-space cast
}

// Returns `p` through an empty asm so the compiler cannot treat LDS reads that
// use it as loop-invariant: without this, a loop over query tiles gets every
// K and V^T operand read hoisted out of it and the kernel runs out of VGPRs.
__device__ inline lds_t* lds_opaque(lds_t* p) {
    asm volatile("" : "+v"(p));
    return p;
}

// A value the compiler cannot see through (for values it would otherwise
// hoist out of a loop and keep live across it): per-lane (VGPR) and
// wave-uniform (SGPR) forms.
__device__ inline int opaque_v(int x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ inline int opaque_s(int x) {
    asm volatile("" : "+s"(x));
    return x;
}

// Hand-off of LDS data between the lanes of one wave.  The hardware runs a
// wave's LDS instructions in order, so no instruction is needed; but for the
// compiler, one lane reading what another lane wrote without synchronisation
// is a data race, and it may keep a value a lane loaded earlier from the same
// address (or move the read into the writers' branch).  A wavefront-scope
// fence makes the writes visible to the reads that follow it.
__device__ inline void wave_lds_handoff() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline u32x4 lds_ld16(const lds_t* p) { return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(p); }
__device__ inline void lds_st16(lds_t* p, u32x4 v) { *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(p) = v; }
// ds_read_b64_tr_b16: within each 16-lane group, lane j receives element j%4
// of the 8-byte rows addressed by lanes j/4, j/4+4, j/4+8, j/4+12.
__device__ inline u32x2 lds_ld8_tr16(const lds_t* p) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(p));
    return __builtin_bit_cast(u32x2, v);
}
__device__ inline u32x2 lds_ld8(const lds_t* p) { return *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>(p); }
__device__ inline void lds_st8(lds_t* p, u32x2 v) { *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(p) = v; }
__device__ inline uint32_t lds_ld4(const lds_t* p) { return *reinterpret_cast<const __attribute__((address_space(3))) uint32_t*>(p); }
__device__ inline void lds_st4(lds_t* p, uint32_t v) { *reinterpret_cast<__attribute__((address_space(3))) uint32_t*>(p) = v; }
__device__ inline uint32_t lds_ld1(const lds_t* p) { return *reinterpret_cast<const __attribute__((address_space(3))) uint8_t*>(p); }
__device__ inline void lds_st1(lds_t* p, uint32_t v) { *reinterpret_cast<__attribute__((address_space(3))) uint8_t*>(p) = (uint8_t)v; }
__device__ inline void lds_st2(lds_t* p, uint32_t v) { *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(p) = (uint16_t)v; }

// 16-byte global load / store through the vector memory path.
__device__ inline u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ inline void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ inline void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }


__device__ inline u32x4 ld16_stream(const void* p) {
    if constexpr (ATX_STREAM_LOADS) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return ld16(p);
}
__device__ inline void st16_stream(void* p, u32x4 v) {
    if constexpr (ATX_STREAM_STORES) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
    else st16(p, v);
}
__device__ inline void st8_stream(void* p, u32x2 v) {
    if constexpr (ATX_STREAM_STORES) __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p));
    else st8(p, v);
}

}  // namespace atx
