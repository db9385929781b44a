// slideformer_amd: the element types and the wave-level memory access of the
// update kernels (gfx950, wave64), shared by the library and by the stream
// probe kernels that measure its memory ceiling.
//
// A lane owns 4 consecutive elements of every stream: fp32 streams move 16
// bytes per lane, 16-bit streams 8, so one wave instruction covers 256
// consecutive elements.  The update kernel addresses each stream through a
// raw buffer descriptor per wave (base = the wave's first element, size =
// its valid elements), so the lanes of a partial last wave need no branch.
#ifndef SLIDEFORMER_AMD_WAVE_IO_H
#define SLIDEFORMER_AMD_WAVE_IO_H

#include <hip/hip_runtime.h>

#include <cstdint>

// Nontemporal hints on the streaming loads / stores.
#ifndef LA_NT_LOAD
#define LA_NT_LOAD 1
#endif
#ifndef LA_NT_STORE
#define LA_NT_STORE 1
#endif
// Wave priority in the update kernel: raise it (s_setprio 3) while a wave
// issues its loads, so a freshly started wave gets its requests out ahead of
// the arithmetic and stores of older waves.  Measured on MI355X, C2 layer:
// off -> 6.30 TB/s, on -> 6.45 TB/s.  Raising it for the stores as well, or
// for the grad-norm kernel's loads, measured no gain.
#ifndef LA_SETPRIO
#define LA_SETPRIO 1
#endif

namespace {

constexpr int kVec = 4;  // elements per lane per group

// ---------------------------------------------------------------------------
// element types
// ---------------------------------------------------------------------------
struct bf16_t { uint16_t x; };
struct f16_t { uint16_t x; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// RNE with NaN -> 0x7FC0, the reference's bf16 store (simd.h:56-86) and c10's
// round_to_nearest_even used by the fp32->bf16 copy_ (transformer_layer.py:304).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f)
{
    const uint32_t u = __float_as_uint(f);
    const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    return ((u & 0x7fffffffu) > 0x7f800000u) ? 0x7fc0u : r;
}

// Two adjacent elements of a 16-bit store at once, low half first.  With
// LA_HW_BF16 the bf16 pair is rounded by one v_cvt_pk_bf16_f32 (IEEE
// round-to-nearest-even in the default mode, fp32 denormals kept).  Every NaN
// is first replaced by 0x7FC00000, whose rounding is the reference's 0x7FC0;
// the empty asm keeps that replaced value opaque, so the backend cannot treat
// the replacement as a no-op (NaN payloads through a conversion are not
// defined by the IR).
#ifndef LA_HW_BF16
#define LA_HW_BF16 1
#endif
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi)
{
#if LA_HW_BF16
    float c0 = (lo != lo) ? __uint_as_float(0x7fc00000u) : lo;
    float c1 = (hi != hi) ? __uint_as_float(0x7fc00000u) : hi;
    asm("" : "+v"(c0), "+v"(c1));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{c0, c1}, bf16x2_t));
#else
    return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
#endif
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// IEEE binary16 round-to-nearest-even by the hardware conversion
// (v_cvt_f16_f32 in the default round-to-nearest-even mode, fp16 denormals
// kept).  The empty asm makes the value opaque, so the backend cannot fold the
// preceding fmaf into one v_fma_mixlo_f16: that would round once to f16 where
// the reference rounds to f32 and then to f16 (cpu_adam.h:190 /
// c10::Half(float) in cpu_adam_impl.cpp:64).  A NaN stays a NaN (its payload
// bits are the hardware's).  Measured on MI355X, C2 shape, (f16, f16, f16):
// 0.711 ms with the former integer rounding in software, see the triples profile.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f)
{
    asm("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename V, bool NT = (LA_NT_LOAD != 0)> __device__ __forceinline__ V vload(const void* p)
{
    if constexpr (NT) return __builtin_nontemporal_load(static_cast<const V*>(p));
    else return *static_cast<const V*>(p);
}

template <typename V> __device__ __forceinline__ void vstore(void* p, V v)
{
#if LA_NT_STORE
    __builtin_nontemporal_store(v, static_cast<V*>(p));
#else
    *static_cast<V*>(p) = v;
#endif
}

// 4 consecutive elements <-> 4 floats; `e` is a multiple of 4 past an aligned head.
template <typename T> struct Io;

template <> struct Io<float> {
    static constexpr int kBytes = 4;
    template <bool NT = (LA_NT_LOAD != 0)>
    __device__ __forceinline__ static void load4(const void* base, uint64_t e, float (&x)[kVec])
    {
        const f32x4 a = vload<f32x4, NT>(static_cast<const float*>(base) + e);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    }
    __device__ __forceinline__ static void store4(void* base, uint64_t e, const float (&x)[kVec])
    {
        vstore<f32x4>(static_cast<float*>(base) + e, f32x4{x[0], x[1], x[2], x[3]});
    }
    __device__ __forceinline__ static float load1(const void* base, uint64_t e)
    {
        return static_cast<const float*>(base)[e];
    }
    __device__ __forceinline__ static void store1(void* base, uint64_t e, float x)
    {
        static_cast<float*>(base)[e] = x;
    }
};

template <typename Conv> struct Io16 {
    static constexpr int kBytes = 2;
    template <bool NT = (LA_NT_LOAD != 0)>
    __device__ __forceinline__ static void load4(const void* base, uint64_t e, float (&x)[kVec])
    {
        const u32x2 u = vload<u32x2, NT>(static_cast<const uint16_t*>(base) + e);
        x[0] = Conv::to_f32(u.x & 0xffffu);
        x[1] = Conv::to_f32(u.x >> 16);
        x[2] = Conv::to_f32(u.y & 0xffffu);
        x[3] = Conv::to_f32(u.y >> 16);
    }
    __device__ __forceinline__ static void store4(void* base, uint64_t e, const float (&x)[kVec])
    {
        const uint32_t lo = Conv::from_f32x2(x[0], x[1]);
        const uint32_t hi = Conv::from_f32x2(x[2], x[3]);
        vstore<u32x2>(static_cast<uint16_t*>(base) + e, u32x2{lo, hi});
    }
    __device__ __forceinline__ static float load1(const void* base, uint64_t e)
    {
        return Conv::to_f32(static_cast<const uint16_t*>(base)[e]);
    }
    __device__ __forceinline__ static void store1(void* base, uint64_t e, float x)
    {
        static_cast<uint16_t*>(base)[e] = static_cast<uint16_t>(Conv::from_f32(x));
    }
};

struct ConvBf16 {
    __device__ __forceinline__ static float to_f32(uint32_t h) { return bf16_bits_to_f32(h); }
    __device__ __forceinline__ static uint32_t from_f32(float f) { return f32_to_bf16_bits(f); }
    __device__ __forceinline__ static uint32_t from_f32x2(float lo, float hi) { return f32x2_to_bf16x2_bits(lo, hi); }
};
struct ConvF16 {
    __device__ __forceinline__ static float to_f32(uint32_t h) { return f16_bits_to_f32(h); }
    __device__ __forceinline__ static uint32_t from_f32(float f) { return f32_to_f16_bits(f); }
    __device__ __forceinline__ static uint32_t from_f32x2(float lo, float hi)
    {
        return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
    }
};
template <> struct Io<bf16_t> : Io16<ConvBf16> {};
template <> struct Io<f16_t> : Io16<ConvF16> {};

// Raw buffer access for the update kernel: 4 consecutive elements per lane at
// byte offset lane * 4 * sizeof(T) from a per-wave descriptor.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kRsrcFlags = 0x00020000;          // word 3 of a gfx9 raw buffer descriptor
// Cache-policy bits of the update kernel's buffer loads / stores (bit 0 sc0,
// bit 1 nt, bit 4 sc1).  Loads: nt.  Stores: nt + sc1 (device scope), so the
// results are written through instead of waiting in the L2 as dirty lines.
// Measured on MI355X, C2 layer, same box: stores nt 0.971 ms, nt+sc1 0.960 ms,
// nt+sc0+sc1 0.959 ms, sc1 alone 0.987 ms; the load bits made no difference.
#ifndef LA_AUX_LOAD
#define LA_AUX_LOAD (LA_NT_LOAD ? 2 : 0)
#endif
#ifndef LA_AUX_STORE
#define LA_AUX_STORE (LA_NT_STORE ? 18 : 0)
#endif
constexpr int kAux = LA_AUX_LOAD;
constexpr int kAuxSt = LA_AUX_STORE;

template <typename T> struct WaveIo;

template <> struct WaveIo<float> {
    __device__ __forceinline__ static rsrc_t rsrc(const void* base, uint64_t e0, uint32_t nel)
    {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(static_cast<const float*>(base) + e0), 0,
                                                 static_cast<int>(nel * 4), kRsrcFlags);
    }
    __device__ __forceinline__ static void load4(rsrc_t r, uint32_t lane, float (&x)[kVec])
    {
        const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(lane * 16), 0, kAux);
        x[0] = __uint_as_float(u.x); x[1] = __uint_as_float(u.y);
        x[2] = __uint_as_float(u.z); x[3] = __uint_as_float(u.w);
    }
    __device__ __forceinline__ static void store4(rsrc_t r, uint32_t lane, const float (&x)[kVec])
    {
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(x[0]), __float_as_uint(x[1]),
                                                     __float_as_uint(x[2]), __float_as_uint(x[3])},
                                               r, static_cast<int>(lane * 16), 0, kAuxSt);
    }
};

template <typename Conv> struct WaveIo16 {
    __device__ __forceinline__ static rsrc_t rsrc(const void* base, uint64_t e0, uint32_t nel)
    {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(static_cast<const uint16_t*>(base) + e0), 0,
                                                 static_cast<int>(nel * 2), kRsrcFlags);
    }
    __device__ __forceinline__ static void load4(rsrc_t r, uint32_t lane, float (&x)[kVec])
    {
        const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(lane * 8), 0, kAux);
        x[0] = Conv::to_f32(u.x & 0xffffu);
        x[1] = Conv::to_f32(u.x >> 16);
        x[2] = Conv::to_f32(u.y & 0xffffu);
        x[3] = Conv::to_f32(u.y >> 16);
    }
    __device__ __forceinline__ static void store4(rsrc_t r, uint32_t lane, const float (&x)[kVec])
    {
        const uint32_t lo = Conv::from_f32x2(x[0], x[1]);
        const uint32_t hi = Conv::from_f32x2(x[2], x[3]);
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{lo, hi}, r, static_cast<int>(lane * 8), 0, kAuxSt);
    }
};
template <> struct WaveIo<bf16_t> : WaveIo16<ConvBf16> {};
template <> struct WaveIo<f16_t> : WaveIo16<ConvF16> {};

// The value of lane 0 of the wave, as a wave-uniform value.  The wave index is
// the same in every lane, but the compiler cannot prove it from threadIdx.x;
// without this it keeps the index in vector registers, builds the buffer
// descriptors there, wraps every buffer access in a readfirstlane loop and
// fetches the multi kernel's segment arguments with per-lane vector loads.
__device__ __forceinline__ uint64_t wave_uniform(uint64_t x)
{
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x >> 32)));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

}  // namespace

#endif  // SLIDEFORMER_AMD_WAVE_IO_H
