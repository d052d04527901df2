// Device helpers shared by the embedding-bag kernels (gfx950, wave64).
#pragma once

#include <type_traits>
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace cti {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------------
// Element types. Tables and outputs are raw 16-bit / 32-bit words; conversions are explicit.
// ---------------------------------------------------------------------------------------------
struct bf16_t {
  uint16_t bits;
};
struct f16_t {
  uint16_t bits;
};
// int8 row-quantised table element; a row's value is q * row_scale[row] (fp32 scale per row).
struct i8_t {
  int8_t q;
};

// bf16 -> fp32 is exact: the bf16 word is the high half of the fp32 word.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(h)));
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static constexpr int kBytes = 4;
  static constexpr int kVecBytes = 16;  // bytes of one lane's row vector
  __device__ static __forceinline__ float load(const void* p) { return *static_cast<const float*>(p); }
};
template <>
struct Elem<bf16_t> {
  static constexpr int kBytes = 2;
  static constexpr int kVecBytes = 16;  // bytes of one lane's row vector
  __device__ static __forceinline__ float load(const void* p) {
    return bf16_bits_to_f32(*static_cast<const uint16_t*>(p));
  }
};
template <>
struct Elem<f16_t> {
  static constexpr int kBytes = 2;
  static constexpr int kVecBytes = 16;  // bytes of one lane's row vector
  __device__ static __forceinline__ float load(const void* p) {
    return f16_bits_to_f32(*static_cast<const uint16_t*>(p));
  }
};
template <>
struct Elem<i8_t> {
  static constexpr int kBytes = 1;
  static constexpr int kVecBytes = 8;  // 8 elements per lane, as many as a 16-byte bf16 vector
  __device__ static __forceinline__ float load(const void* p) {  // unscaled q
    return static_cast<float>(*static_cast<const int8_t*>(p));
  }
};

// Whether rows of a table type carry a per-row scale.
template <typename T>
struct Quantized {
  static constexpr bool value = false;
};
template <>
struct Quantized<i8_t> {
  static constexpr bool value = true;
};

// Add the elements held in one 16-byte vector to fp32 accumulators, in element order.
__device__ __forceinline__ void acc16(float* a, const uint4& v, float) {
  a[0] += __uint_as_float(v.x);
  a[1] += __uint_as_float(v.y);
  a[2] += __uint_as_float(v.z);
  a[3] += __uint_as_float(v.w);
}
__device__ __forceinline__ void acc16(float* a, const uint4& v, bf16_t) {
  a[0] += __uint_as_float(v.x << 16);
  a[1] += __uint_as_float(v.x & 0xffff0000u);
  a[2] += __uint_as_float(v.y << 16);
  a[3] += __uint_as_float(v.y & 0xffff0000u);
  a[4] += __uint_as_float(v.z << 16);
  a[5] += __uint_as_float(v.z & 0xffff0000u);
  a[6] += __uint_as_float(v.w << 16);
  a[7] += __uint_as_float(v.w & 0xffff0000u);
}
__device__ __forceinline__ void acc16(float* a, const uint4& v, f16_t) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[2 * i] += f16_bits_to_f32(w[i] & 0xffffu);
    a[2 * i + 1] += f16_bits_to_f32(w[i] >> 16);
  }
}
// int8 rows: a[k] = fma(q_k, scale, a[k]) in element order (one rounding per element, as the
// reference's `acc += int8_row * scale_val` compiles to).
// int8 rows: the 8 elements in v.x, v.y, each a = fma(q, s, a) in element order.
__device__ __forceinline__ void acc8_scaled(float* a, const uint4& v, float s) {
  const uint32_t w[2] = {v.x, v.y};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      a[4 * i + k] = __builtin_fmaf(static_cast<float>(static_cast<int8_t>(w[i] >> (8 * k))), s, a[4 * i + k]);
  }
}

// One lane vector of a row (Elem<TT>::kVecBytes bytes) into the accumulators; `s` is the row's
// scale (quantized tables).
template <typename TT>
__device__ __forceinline__ void acc_row(float* a, const uint4& v, float s) {
  if constexpr (Quantized<TT>::value) acc8_scaled(a, v, s);
  else acc16(a, v, TT{});
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Output blocks of at least this many bytes are stored non-temporally (`stream`: through L2 with
// evict-first priority). A block that large would not stay in the caches until its consumer reads
// it, and streaming it keeps the table rows that later lookups hit in L2 (32,768 samples x 28
// fields of 128 bf16, a 235 MB block: pooling 280 -> 269 us, pooling then LayerNorm 441 -> 433.5
// us). A smaller block is stored plainly and stays in the 256 MB memory-side cache for its
// consumer (4,096 samples, a 29 MB block, streamed: pooling 0.8 us faster, the LayerNorm that
// reads it 2.7 us slower).
constexpr int64_t kStreamOutBytes = int64_t{128} << 20;

template <bool STREAM, typename V>
__device__ __forceinline__ void put_as(V* dst, V v) {
  if constexpr (STREAM) __builtin_nontemporal_store(v, dst);
  else *dst = v;
}
template <typename V>
__device__ __forceinline__ void put(V* dst, V v, bool stream) {
  if (stream) {
    // the barriers keep the two stores apart: hoisted or sunk into one, the store would lose its
    // non-temporal hint
    __builtin_amdgcn_sched_barrier(0);
    __builtin_nontemporal_store(v, dst);
    __builtin_amdgcn_sched_barrier(0);
  } else {
    *dst = v;
  }
}
// Runs f(std::true_type) when `stream` (uniform) is set, else f(std::false_type): a loop of stores
// written as f then holds no branch per store. The barriers keep the two copies apart (as in put).
template <typename F>
__device__ __forceinline__ void with_stream(bool stream, F&& f) {
  if (stream) {
    __builtin_amdgcn_sched_barrier(0);
    f(std::true_type{});
    __builtin_amdgcn_sched_barrier(0);
  } else {
    f(std::false_type{});
  }
}
__device__ __forceinline__ void put4(void* dst, uint32_t x, uint32_t y, uint32_t z, uint32_t w, bool stream) {
  const u32x4 v = {x, y, z, w};
  put(reinterpret_cast<u32x4*>(dst), v, stream);
}
__device__ __forceinline__ void put2(void* dst, uint32_t x, uint32_t y, bool stream) {
  const u32x2 v = {x, y};
  put(reinterpret_cast<u32x2*>(dst), v, stream);
}

// Store N fp32 values as output type OT (N * sizeof(OT) is a multiple of 8 bytes and the
// destination is aligned to that size by the host-side variant selection).
template <int N>
__device__ __forceinline__ void store_out(float* dst, const float* a, bool stream) {
  static_assert(N % 4 == 0, "fp32 stores are 16-byte vectors");
#pragma unroll
  for (int i = 0; i < N; i += 4)
    put4(dst + i, __float_as_uint(a[i]), __float_as_uint(a[i + 1]), __float_as_uint(a[i + 2]),
         __float_as_uint(a[i + 3]), stream);
}
// Two fp32 values to a packed bf16 pair, IEEE round to nearest even (one v_cvt_pk_bf16_f32 on
// gfx950): +-Inf and values that round past the largest finite bf16 become +-Inf, NaN stays NaN.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

template <int N>
__device__ __forceinline__ void store_out(bf16_t* dst, const float* a, bool stream) {
  static_assert(N % 4 == 0, "16-bit stores are 8- or 16-byte vectors");
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 8)
      put4(dst + i, pack_bf16x2(a[i], a[i + 1]), pack_bf16x2(a[i + 2], a[i + 3]), pack_bf16x2(a[i + 4], a[i + 5]),
           pack_bf16x2(a[i + 6], a[i + 7]), stream);
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4)
      put2(dst + i, pack_bf16x2(a[i], a[i + 1]), pack_bf16x2(a[i + 2], a[i + 3]), stream);
  }
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
}
template <int N>
__device__ __forceinline__ void store_out(f16_t* dst, const float* a, bool stream) {
  static_assert(N % 4 == 0, "16-bit stores are 8- or 16-byte vectors");
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 8)
      put4(dst + i, pack_f16x2(a[i], a[i + 1]), pack_f16x2(a[i + 2], a[i + 3]), pack_f16x2(a[i + 4], a[i + 5]),
           pack_f16x2(a[i + 6], a[i + 7]), stream);
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) put2(dst + i, pack_f16x2(a[i], a[i + 1]), pack_f16x2(a[i + 2], a[i + 3]), stream);
  }
}

__device__ __forceinline__ void store_one(float* dst, float a, bool stream) { put(dst, a, stream); }
__device__ __forceinline__ void store_one(bf16_t* dst, float a, bool stream) {
  put(reinterpret_cast<uint16_t*>(dst), static_cast<uint16_t>(pack_bf16x2(a, 0.f)), stream);
}
__device__ __forceinline__ void store_one(f16_t* dst, float a, bool stream) {
  put(reinterpret_cast<uint16_t*>(dst), static_cast<uint16_t>(f32_to_f16_bits(a)), stream);
}

// a[i] / L for a bag of L >= 1 rows, each rounded once to fp32, given inv = 1/L rounded to fp64.
// For quotients in the normal range RN32(RN64(a * inv)) = RN32(a / L): the fp64 product is
// within 2^-52 (relative) of a / L, and a / L (a has a 24-bit significand, L <= 2^24) is at
// least 2^-49 (relative) away from every fp32 rounding midpoint it is not equal to, while it
// is never equal to one there (its odd part has at most 24 bits). Quotients below the normal
// range, where a midpoint can be hit exactly, and zero sums are recomputed by IEEE division (a
// branch that is rarely taken for real data).
template <int N>
__device__ __forceinline__ void div_by_count(float* a, double inv, float fl) {
  // |a| < 2^-126 * L (exact: L <= 2^24) <=> the quotient is below the normal range (or zero)
  const float tiny = 1.17549435e-38f * fl;
  float q[N];
  bool fix = false;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q[i] = static_cast<float>(static_cast<double>(a[i]) * inv);
    fix |= __builtin_fabsf(a[i]) < tiny;
  }
  if (__builtin_expect(fix, 0)) {
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = __builtin_fabsf(a[i]) < tiny ? a[i] / fl : q[i];
  }
#pragma unroll
  for (int i = 0; i < N; ++i) a[i] = q[i];
}

// ---------------------------------------------------------------------------------------------
// Cross-lane moves inside one wavefront (ds_bpermute: any-to-any, all 64 lanes must be active).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

__device__ __forceinline__ int shfl_i32(int v, int src_lane) {
  return __builtin_amdgcn_ds_bpermute(src_lane << 2, v);
}
__device__ __forceinline__ int64_t shfl_i64(int64_t v, int src_lane) {
  const int lo = shfl_i32(static_cast<int>(static_cast<uint64_t>(v)), src_lane);
  const int hi = shfl_i32(static_cast<int>(static_cast<uint64_t>(v) >> 32), src_lane);
  return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                              static_cast<uint32_t>(lo));
}
__device__ __forceinline__ float shfl_xor_f32(float v, int mask) {
  return __int_as_float(shfl_i32(__float_as_int(v), lane_id() ^ mask));
}
__device__ __forceinline__ uint4 load16(const char* p) {
  return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ int64_t clamp_i64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}


// Sum over the workgroup (WAVES wavefronts) in a fixed order: xor butterfly inside each
// wavefront, then the wavefront sums in wavefront order. Every thread gets the total.
template <int WAVES>
__device__ __forceinline__ float block_sum(float v, float* s_red) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) v += shfl_xor_f32(v, m);
  if constexpr (WAVES == 1) {
    return v;
  } else {
    const int w = static_cast<int>(threadIdx.x) / kWave;
    __syncthreads();  // earlier readers of s_red are done
    if (lane_id() == 0) s_red[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < WAVES; ++i) t += s_red[i];
    return t;
  }
}

// N sums over the workgroup at once (each as block_sum would take it: the same butterfly and
// wavefront order, so each result is bitwise what block_sum<WAVES> gives), two barriers in all.
// s_red holds WAVES * N floats.
template <int WAVES, int N>
__device__ __forceinline__ void block_sum_n(float* v, float* s_red) {
#pragma unroll
  for (int k = 0; k < N; ++k) {
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) v[k] += shfl_xor_f32(v[k], m);
  }
  if constexpr (WAVES > 1) {
    const int w = static_cast<int>(threadIdx.x) / kWave;
    __syncthreads();  // earlier readers of s_red are done
    if (lane_id() == 0) {
#pragma unroll
      for (int k = 0; k < N; ++k) s_red[k * WAVES + w] = v[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < N; ++k) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < WAVES; ++i) t += s_red[k * WAVES + i];
      v[k] = t;
    }
  }
}

__device__ __forceinline__ void unpack16(const uint4& v, float* a, float) {
  a[0] = __uint_as_float(v.x);
  a[1] = __uint_as_float(v.y);
  a[2] = __uint_as_float(v.z);
  a[3] = __uint_as_float(v.w);
}
__device__ __forceinline__ void unpack16(const uint4& v, float* a, bf16_t) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[2 * i] = __uint_as_float(w[i] << 16);
    a[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack16(const uint4& v, float* a, f16_t) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
    a[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
  }
}

// VEC parameters starting at element c0 (16-byte aligned): 16-byte loads, or one 8-byte load.
template <typename PT, int VEC>
__device__ __forceinline__ void load_params(const void* p, int64_t c0, float* out) {
  const char* base = static_cast<const char*>(p) + c0 * Elem<PT>::kBytes;
  constexpr int BYTES = VEC * Elem<PT>::kBytes;
  if constexpr (BYTES == 8) {  // four 16-bit parameters
    const uint2 u = *reinterpret_cast<const uint2*>(base);
    float t[8];
    unpack16(make_uint4(u.x, u.y, 0u, 0u), t, PT{});
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[e] = t[e];
  } else {
#pragma unroll
    for (int h = 0; h < BYTES / 16; ++h) unpack16(load16(base + h * 16), out + h * (16 / Elem<PT>::kBytes), PT{});
  }
}

}  // namespace cti
