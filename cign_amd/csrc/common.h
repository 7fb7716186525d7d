// Shared device helpers and C-ABI error plumbing for libcign_amd.
//
// Every kernel in this library is written for gfx950 (CDNA4): 64-lane
// wavefronts, 256-thread workgroups (4 waves), fp32 accumulation. Feature
// tensors are row-major; bf16 storage is supported through the load/store
// helpers below (accumulation always stays fp32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace cign {

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

// dtype codes used on the C-ABI. kBF16F32: bf16 features (values a bf16
// projection produced, so exact in bf16) with fp32 outputs and gradients.
enum DType : int { kF32 = 0, kBF16 = 1, kBF16F32 = 2 };

// Return codes used on the C-ABI.
enum Status : int { kOk = 0, kInvalid = 1, kHipError = 2 };

// Thread-local "last error" text, readable through cign_last_error().
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---------------------------------------------------------------------------
// bf16 <-> fp32 (round to nearest even, NaN kept quiet).
// ---------------------------------------------------------------------------
struct bf16 {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float f);
template <>
__device__ __forceinline__ float from_f32<float>(float f) { return f; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float f) {
  uint32_t u = __float_as_uint(f);
  bf16 r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.bits = static_cast<uint16_t>((u >> 16) | 0x40u);
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    r.bits = static_cast<uint16_t>(u >> 16);
  }
  return r;
}

// bf16 storage that a kernel reads and writes four values (8 bytes) per lane
// instead of eight: the feature-layout GAT kernels of small graphs take bf16
// features this way, so a row spreads over as many lanes as an fp32 row and
// each lane of a latency-bound launch has half the work.
struct bf16h {
  uint16_t bits;
};
__device__ __forceinline__ float to_f32(bf16h v) { return __uint_as_float(static_cast<uint32_t>(v.bits) << 16); }
template <>
__device__ __forceinline__ bf16h from_f32<bf16h>(float f) {
  bf16h r;
  r.bits = from_f32<bf16>(f).bits;
  return r;
}

// Features stored as bf16 whose results and gradients are fp32 (the
// collapsed GAT on a bf16 projection under selective AMP, whose fp32 input
// holds bf16 values exactly): loads are those of bf16, every output type is
// float (GatOut).
struct bf16x {
  uint16_t bits;
};
__device__ __forceinline__ float to_f32(bf16x v) { return __uint_as_float(static_cast<uint32_t>(v.bits) << 16); }

// Type of the outputs and incoming gradients of kernels whose inputs are T.
template <typename T>
struct GatOutOf {
  using type = T;
};
template <>
struct GatOutOf<bf16x> {
  using type = float;
};
template <typename T>
using GatOut = typename GatOutOf<T>::type;

// A 16-byte (or 1-element) vector chunk of T, unpacked to fp32 registers.
// W = elements per chunk: 4 (fp32 x4), 8 (bf16 x8) or 1 (scalar fallback).
template <typename T, int W>
struct Chunk;

template <>
struct Chunk<float, 4> {
  // The 16 raw bytes (kept in flight by gather batches, unpacked on use).
  using Raw = float4;
  static __device__ __forceinline__ Raw load_raw(const float* p) { return *reinterpret_cast<const float4*>(p); }
  static __device__ __forceinline__ Raw zero_raw() { return make_float4(0.0f, 0.0f, 0.0f, 0.0f); }
  static __device__ __forceinline__ void unpack(const Raw& q, float (&v)[4]) {
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  }
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    const float4 q = *reinterpret_cast<const float4*>(p);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

template <>
struct Chunk<bf16, 8> {
  using Raw = uint4;
  static __device__ __forceinline__ Raw load_raw(const bf16* p) { return *reinterpret_cast<const uint4*>(p); }
  static __device__ __forceinline__ Raw zero_raw() { return make_uint4(0u, 0u, 0u, 0u); }
  static __device__ __forceinline__ void unpack(const Raw& q, float (&v)[8]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void load(const bf16* p, float (&v)[8]) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void store(bf16* p, const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = from_f32<bf16>(v[2 * i]).bits;
      const uint32_t hi = from_f32<bf16>(v[2 * i + 1]).bits;
      w[i] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};

template <>
struct Chunk<bf16h, 4> {
  using Raw = uint2;
  static __device__ __forceinline__ Raw load_raw(const bf16h* p) { return *reinterpret_cast<const uint2*>(p); }
  static __device__ __forceinline__ Raw zero_raw() { return make_uint2(0u, 0u); }
  static __device__ __forceinline__ void unpack(const Raw& q, float (&v)[4]) {
    v[0] = __uint_as_float(q.x << 16);
    v[1] = __uint_as_float(q.x & 0xffff0000u);
    v[2] = __uint_as_float(q.y << 16);
    v[3] = __uint_as_float(q.y & 0xffff0000u);
  }
  static __device__ __forceinline__ void load(const bf16h* p, float (&v)[4]) { unpack(load_raw(p), v); }
  static __device__ __forceinline__ void store(bf16h* p, const float (&v)[4]) {
    const uint32_t w0 = from_f32<bf16>(v[0]).bits | (static_cast<uint32_t>(from_f32<bf16>(v[1]).bits) << 16);
    const uint32_t w1 = from_f32<bf16>(v[2]).bits | (static_cast<uint32_t>(from_f32<bf16>(v[3]).bits) << 16);
    *reinterpret_cast<uint2*>(p) = make_uint2(w0, w1);
  }
};

template <>
struct Chunk<bf16x, 8> {
  using Raw = uint4;
  static __device__ __forceinline__ Raw load_raw(const bf16x* p) { return *reinterpret_cast<const uint4*>(p); }
  static __device__ __forceinline__ Raw zero_raw() { return make_uint4(0u, 0u, 0u, 0u); }
  static __device__ __forceinline__ void unpack(const Raw& q, float (&v)[8]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void load(const bf16x* p, float (&v)[8]) { unpack(load_raw(p), v); }
};

// Eight fp32 values (the outputs of a bf16x chunk): two 16-byte accesses.
template <>
struct Chunk<float, 8> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[8]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
};

template <typename T>
struct Chunk<T, 1> {
  using Raw = T;
  static __device__ __forceinline__ Raw load_raw(const T* p) { return *p; }
  static __device__ __forceinline__ Raw zero_raw() { return from_f32<T>(0.0f); }
  static __device__ __forceinline__ void unpack(const Raw& q, float (&v)[1]) { v[0] = to_f32(q); }
  static __device__ __forceinline__ void load(const T* p, float (&v)[1]) { v[0] = to_f32(*p); }
  static __device__ __forceinline__ void store(T* p, const float (&v)[1]) { *p = from_f32<T>(v[0]); }
};

// ---------------------------------------------------------------------------
// Wavefront primitives (64 lanes).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ float shfl(float v, int src) { return __shfl(v, src, kWave); }
__device__ __forceinline__ int shfl(int v, int src) { return __shfl(v, src, kWave); }

__device__ __forceinline__ int shfl_xor_i(int v, int m) { return __shfl_xor(v, m, kWave); }

// DPP move with control CTRL, all rows and banks. bound_ctrl: a lane reading a
// disabled lane gets 0 (as from an old value of 0) and the destination needs
// no initialisation.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// v of lane (lane ^ O), O a compile-time power of two below 64, the value
// shfl_xor(v, O) returns: DPP inside a 16-lane row for O <= 8 (quad permutes
// for 1 and 2; a row half-mirror then a quad reverse for 4, as 7 - (3 - i) =
// i ^ 4 within 8 lanes; a row rotation by 8 for 8), a swizzle inside 32 lanes
// for 16 and a backward permute for 32. Butterflies over low lane bits then
// run on the VALU instead of waiting on LDS-pipe permutes. The partner lane
// must be active.
template <int O>
__device__ __forceinline__ float xor_shfl(float v) {
  static_assert(O > 0 && O < kWave && (O & (O - 1)) == 0, "lane offset");
  if constexpr (O == 1) return dpp<0xB1>(v);               // quad_perm [1,0,3,2]
  else if constexpr (O == 2) return dpp<0x4E>(v);          // quad_perm [2,3,0,1]
  else if constexpr (O == 4) return dpp<0x1B>(dpp<0x141>(v));  // row_half_mirror, quad_perm [3,2,1,0]
  else if constexpr (O == 8) return dpp<0x128>(v);         // row_ror:8
  else if constexpr (O == 16) return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  else return shfl_xor(v, O);
}

// f(integral_constant<int, O>) for O = 1, 2, 4, ..., 32 with FROM <= O < TO
// (compile-time lane offsets of a butterfly).
template <int FROM, int TO, typename F>
__device__ __forceinline__ void for_offsets(F&& f) {
  if constexpr (FROM < TO) {
    f(std::integral_constant<int, FROM>{});
    for_offsets<FROM * 2, TO>(f);
  }
}

// Edge-batch driver of the gather kernels: runs fn.template run<U>(k0) for
// k0 = 0, U, 2U, ... < need, with U the smallest power of two >= need, capped
// at UMAX. `need` must be wave-uniform: a batch issues all of its U gathers
// before consuming any, so U is the number of loads a lane keeps in flight.
template <int UMAX, typename Fn>
__device__ __forceinline__ void for_batches(int need, Fn& fn) {
  static_assert(UMAX == 1 || UMAX == 2 || UMAX == 4 || UMAX == 8 || UMAX == 16, "UMAX is a power of two <= 16");
  if (need <= 0) return;
  if (need <= 1 || UMAX == 1) {
    for (int k0 = 0; k0 < need; ++k0) fn.template run<1>(k0);
  } else if (need <= 2 || UMAX == 2) {
    for (int k0 = 0; k0 < need; k0 += 2) fn.template run<2>(k0);
  } else if (need <= 4 || UMAX == 4) {
    for (int k0 = 0; k0 < need; k0 += 4) fn.template run<4>(k0);
  } else if (need <= 8 || UMAX == 8) {
    for (int k0 = 0; k0 < need; k0 += 8) fn.template run<8>(k0);
  } else {
    for (int k0 = 0; k0 < need; k0 += 16) fn.template run<16>(k0);
  }
}

// Sum over lanes whose ids differ only in bits >= `from` (all lanes sharing
// lane % from); every such lane receives the total.
__device__ __forceinline__ float sum_across(float v, int from) {
  for_offsets<1, kWave>([&](auto OC) {
    constexpr int o = decltype(OC)::value;
    if (o >= from) v += xor_shfl<o>(v);
  });
  return v;
}

// sum_across of every element of v, the butterflies interleaved step by step
// so that their shuffles overlap instead of each waiting on the previous one.
template <int N, int M>
__device__ __forceinline__ void sum_across_n(float (&v)[N][M], int from) {
  for_offsets<1, kWave>([&](auto OC) {
    constexpr int o = decltype(OC)::value;
    if (o >= from)
#pragma unroll
      for (int i = 0; i < N; ++i)
#pragma unroll
        for (int j = 0; j < M; ++j) v[i][j] += xor_shfl<o>(v[i][j]);
  });
}

// ---------------------------------------------------------------------------
// Math helpers shared by the GAT, pack and block kernels.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float leaky(float x, float slope) { return x > 0.0f ? x : x * slope; }

// e^x of a softmax weight (x = score - running max <= 0): the hardware base-2
// exponential (v_exp_f32, 1 ulp) of x * log2(e). Rounding the product adds a
// relative error of at most |x| * 2^-24, so about 5e-6 at x = -88 where the
// result leaves the normal range; results below 2^-126 flush to zero. Three
// instructions instead of the dozen of the correctly rounded expf.
__device__ __forceinline__ float softmax_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
// 1 / (1 + e^-x) from the hardware exponential and reciprocal (v_exp_f32,
// v_rcp_f32, 1 ulp each; the product -x * log2(e) adds a relative error of
// at most |x| * 2^-24 to e^-x): a few ulp against the correctly rounded
// expf and IEEE division, in four instructions instead of about twenty.
// Saturates to 0 (e^-x overflows to inf) and 1 (e^-x underflows) as those do.
__device__ __forceinline__ float sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}
__device__ __forceinline__ float silu(float x) { return x * sigmoid(x); }
__device__ __forceinline__ float silu_grad(float x) {
  const float s = sigmoid(x);
  return s * (1.0f + x * (1.0f - s));
}

// splitmix64 finaliser (Steele, Lea, Flood 2014; public-domain constants as
// published by S. Vigna). Used by the dropout masks so they match the
// reference bit for bit.
__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
constexpr uint64_t kIdxMul = 0xD2B74407B1CE6E93ull;

// Edge-dropout keep bit of the collapsed GAT: 32-bit uniform, keep = u > p.
__device__ __forceinline__ bool gat_keep(uint64_t seed, uint64_t idx, float p) {
  const uint64_t r = splitmix64(seed ^ (idx * kIdxMul));
  const uint32_t hi = static_cast<uint32_t>(r >> 32);
  const float u = (static_cast<float>(hi) + 0.5f) * 2.3283064365386963e-10f;
  return u > p;
}

// Block-op dropout keep bit: 53-bit uniform in double, keep = u >= p.
__device__ __forceinline__ bool block_keep(uint64_t seed, uint64_t idx, float p) {
  if (p <= 0.0f) return true;
  const uint64_t r = splitmix64(seed ^ (idx * kIdxMul));
  const double u = static_cast<double>(r >> 11) * (1.0 / 9007199254740992.0);
  return u >= static_cast<double>(p);
}

// ---------------------------------------------------------------------------
// Cross-workgroup "last arrival" for segmented rows. Each participating block
// publishes its partial result with st_agent (below), then calls this with
// thread 0's view of the per-row counter. Exactly one block (the last to
// arrive) sees `true`; it resets the counter so the next launch starts from
// zero again, and reads the partials with ld_agent. No block ever waits on
// another, so this cannot hang.
//
// The handoff needs no L2 write-back or invalidate: the partials are stored
// with agent-scope atomic stores (written through to the level coherent
// across the XCDs' L2 caches) and loaded with agent-scope atomic loads (read
// from it), so the only order to keep is each store's completion before the
// counter's increment (s_waitcnt vmcnt(0) in every wavefront, then the
// barrier). An agent-scope release/acquire pair instead writes back and
// invalidates the whole L2 of the XCD twice per call (buffer_wbl2 sc1,
// buffer_inv sc1): at the c2 layer that was 4 us of the GAT backward's 23.
// Every datum one block hands to another in the same launch must go through
// st_agent / ld_agent.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int N>
__device__ __forceinline__ void st_agent_n(float* p, const float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) st_agent(p + i, v[i]);
}

template <int N>
__device__ __forceinline__ void ld_agent_n(const float* p, float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = ld_agent(p + i);
}

__device__ __forceinline__ bool arrive_last(int* counter, int expected, int* lds_flag) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = (prev == expected - 1);
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = last ? 1 : 0;
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return *lds_flag != 0;
}

}  // namespace cign
