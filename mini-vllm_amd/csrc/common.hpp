// Wave64 building blocks shared by every kernel in this library.
//
// CDNA4 (gfx950) executes 64-lane wavefronts. Everything here is written for that
// width: a 16-byte load per lane is the unit of global traffic, and cross-lane
// reductions inside a 16-lane DPP row are single VALU instructions with a DPP
// modifier (quad_perm / row_half_mirror / row_mirror), so a 16-lane all-reduce costs
// four instructions and touches no LDS.
//
// Replaces the warp32 helpers of the reference's csrc/kernel_utils.cuh:14-133
// (warp_reduce_sum/max, block_reduce_*, Vector<T>); the reduction structure is
// different by design, not translated.

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

constexpr int kWave = 64;

// Storage type codes shared with the C ABI (include/minivllm_hip.h).
enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2, kFP8E4M3 = 3 };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------ conversions

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };
struct fp8_t { uint8_t bits; };

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950), the rounding
// torch's `.to(torch.bfloat16)` performs, which parity with the oracle requires.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v;
  const uint16_t b = static_cast<uint16_t>(h);
  __builtin_memcpy(&v, &b, 2);
  return static_cast<float>(v);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  // f is an fp32 value that must be rounded to fp16 as it stands. Without the empty asm
  // the compiler may fold the multiply that produced f into the conversion
  // (v_fma_mixlo_f16: one rounding of the exact product), which differs from PyTorch's
  // fp32 multiply then .to(float16) whenever the fp32 result lands on an fp16 tie.
  asm volatile("" : "+v"(f));
  const _Float16 v = static_cast<_Float16>(f);  // v_cvt_f16_f32, round to nearest even
  uint16_t b;
  __builtin_memcpy(&b, &v, 2);
  return b;
}

// OCP fp8 e4m3fn (max 448, no infinities) -> fp32, exactly, with gfx950's packed
// conversion (v_cvt_pk_f32_fp8 decodes OCP e4m3fn on this architecture: checked
// code by code against the format's definition, all 256 codes).
__device__ __forceinline__ float fp8e4m3_to_f32(uint32_t byte) {
  return __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(byte), false)[0];
}

// Element access for the generic templates: load one element as float.
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kBytes = 4;
  __device__ static float load(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
  __device__ static void store(void* p, int64_t i, float v) { static_cast<float*>(p)[i] = v; }
  __device__ static float round(float v) { return v; }
};
template <> struct Elem<bf16_t> {
  static constexpr int kBytes = 2;
  __device__ static float load(const void* p, int64_t i) {
    return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
  }
  __device__ static void store(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_bf16_bits(v));
  }
  __device__ static float round(float v) { return __uint_as_float(f32_to_bf16_bits(v) << 16); }
};
template <> struct Elem<f16_t> {
  static constexpr int kBytes = 2;
  __device__ static float load(const void* p, int64_t i) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ static void store(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_f16_bits(v));
  }
  __device__ static float round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
};
template <> struct Elem<fp8_t> {
  static constexpr int kBytes = 1;
  __device__ static float load(const void* p, int64_t i) {
    return fp8e4m3_to_f32(static_cast<const uint8_t*>(p)[i]);
  }
};

// Unpack a 16-byte chunk (four dwords) into N = 16 / sizeof(T) floats.
template <typename T> struct Chunk;
template <> struct Chunk<float> {
  static constexpr int kN = 4;
  __device__ static void unpack(const u32x4& w, float* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(w[i]);
  }
};
template <> struct Chunk<bf16_t> {
  static constexpr int kN = 8;
  __device__ static void unpack(const u32x4& w, float* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = bf16_lo(w[i]);
      out[2 * i + 1] = bf16_hi(w[i]);
    }
  }
};
template <> struct Chunk<f16_t> {
  static constexpr int kN = 8;
  __device__ static void unpack(const u32x4& w, float* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
      out[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  }
};
template <> struct Chunk<fp8_t> {
  static constexpr int kN = 16;
  __device__ static void unpack(const u32x4& w, float* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), true);
      out[4 * i] = lo[0];
      out[4 * i + 1] = lo[1];
      out[4 * i + 2] = hi[0];
      out[4 * i + 3] = hi[1];
    }
  }
};

// SwiGLU of one element with the reference's rounding points (basics.py:39-41,
// csrc/swiglu.cu:48-51): T(T(g * T(sigmoid(g))) * u), sigmoid = 1 / (1 + expf(-g)); the
// caller rounds the returned product to T. Shared by the elementwise kernel and the
// fused gate/up projection so both give the same bits.
template <typename T>
__device__ __forceinline__ float swiglu_one(float g, float u) {
  const float sig = Elem<T>::round(1.0f / (1.0f + expf(-g)));
  const float act = Elem<T>::round(__fmul_rn(g, sig));
  return __fmul_rn(act, u);
}

// swiglu_one for |g| < 32, the same bits in fewer instructions (the elementwise SwiGLU
// at 8 elements per lane is bound by its vector ALU, not by memory, with swiglu_one's
// ~33 instructions per element). The two library routines inside it are written out
// with the steps they take for such arguments, their range handling left out:
//   expf(-g): the product -g log2(e) as a rounded head ph and an fma tail plus the
//     constant's low part, 2^(ph - rint(ph) + tail) by v_exp_f32, scaled by
//     2^rint(ph) (v_ldexp); the device library's under/overflow clamps (|g| > 88) never
//     apply here;
//   1 / d for d = 1 + expf(-g) in [1, 2^47): the IEEE division's reciprocal and three
//     Newton/remainder fma steps; its operand pre-scaling, scaled final fma and
//     special-case fixup are identities for a numerator of 1 and such denominators.
// Callers take this path only when every lane's arguments are inside the range; the
// 16-bit types are checked against swiglu_one (through torch) over all 65536 inputs.
// Returns the unrounded quotient 1 / (1 + expf(-g)).
__device__ __forceinline__ float sigmoid_small(float g) {
  const float c_hi = __uint_as_float(0xbfb8aa3bu);  // -log2(e), rounded
  const float c_lo = __uint_as_float(0xb2a5705fu);  // -(log2(e) - c_hi)
  const float ph = __fmul_rn(g, c_hi);
  const float k = __builtin_rintf(ph);
  const float tail = fmaf(g, c_lo, fmaf(g, c_hi, -ph));
  const float frac = __fadd_rn(__fsub_rn(ph, k), tail);
  const float e = __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(frac), static_cast<int>(k));
  const float d = __fadd_rn(1.0f, e);
  const float r0 = __builtin_amdgcn_rcpf(d);
  const float r = fmaf(fmaf(-d, r0, 1.0f), r0, r0);
  const float q1 = fmaf(fmaf(-d, r, 1.0f), r, r);
  return fmaf(fmaf(-d, q1, 1.0f), r, q1);
}

// Two values rounded to T (one packed conversion for bf16).
template <typename T>
__device__ __forceinline__ void round_pair(float& a, float& b) {
  if constexpr (__is_same(T, bf16_t)) {
    uint32_t w = pack_bf16x2(a, b);
    asm("" : "+v"(w));  // keeps the one packed conversion (not split back into two)
    a = bf16_lo(w);
    b = bf16_hi(w);
  } else {
    a = Elem<T>::round(a);
    b = Elem<T>::round(b);
  }
}

// swiglu_one of two elements with |g0|, |g1| < 32 (products returned unrounded).
template <typename T>
__device__ __forceinline__ void swiglu_two_small(float g0, float g1, float u0, float u1,
                                                 float& r0, float& r1) {
  float s0 = sigmoid_small(g0), s1 = sigmoid_small(g1);
  round_pair<T>(s0, s1);
  float a0 = __fmul_rn(g0, s0), a1 = __fmul_rn(g1, s1);
  round_pair<T>(a0, a1);
  r0 = __fmul_rn(a0, u0);
  r1 = __fmul_rn(a1, u1);
}

// 16-byte global load / store through the vector memory path.
__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void store16(void* p, const u32x4& v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

// Streaming variants: data touched once per call is loaded and stored nontemporally,
// so it does not displace lines that other waves reuse (page tables, weights, tables).
__device__ __forceinline__ u32x4 nt_load16(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void nt_store16(void* p, const u32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

// 16 bytes per lane from global memory (base + voff, base wave-uniform) straight into
// LDS: lane i's bytes land at LDS address lds + 16 i. Written as asm so that the
// compiler's wait-count pass neither tracks it nor drains it: the callers wait for it
// explicitly (vmcnt) before the data is read. M0 carries the LDS address; nothing else
// in the kernels that use this sets M0.
__device__ __forceinline__ void copy_to_lds(const char* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base),
               "s"(lds)
               : "memory");
}

// A workgroup-uniform load of read-only metadata through the scalar cache (s_load): it
// is waited for on its own counter, so it does not drain outstanding vector loads.
typedef __attribute__((address_space(4))) const int32_t constant_i32;
__device__ __forceinline__ int32_t sload(const int32_t* p) {
  return *reinterpret_cast<constant_i32*>(reinterpret_cast<uintptr_t>(p));
}

// ------------------------------------------------------------------- reductions

// DPP control codes (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, false));
}

// All-reduce over aligned groups of `kWidth` lanes (kWidth in {1,2,4,8,16,32,64}).
// Widths up to 16 stay inside a DPP row: quad xor-1, quad xor-2, half-row mirror and
// row mirror each pair every lane with a distinct partner of the same group, so
// after log2(kWidth) steps every lane of the group holds the group's total. Wider
// groups finish with ds_swizzle-free xor shuffles across rows.
template <int kWidth>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (kWidth >= 2) v += dpp<kDppQuadXor1>(v);
  if constexpr (kWidth >= 4) v += dpp<kDppQuadXor2>(v);
  if constexpr (kWidth >= 8) v += dpp<kDppRowHalfMirror>(v);
  if constexpr (kWidth >= 16) v += dpp<kDppRowMirror>(v);
  if constexpr (kWidth >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (kWidth >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

template <int kWidth>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (kWidth >= 2) v = fmaxf(v, dpp<kDppQuadXor1>(v));
  if constexpr (kWidth >= 4) v = fmaxf(v, dpp<kDppQuadXor2>(v));
  if constexpr (kWidth >= 8) v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
  if constexpr (kWidth >= 16) v = fmaxf(v, dpp<kDppRowMirror>(v));
  if constexpr (kWidth >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
  if constexpr (kWidth >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }

// Pack N floats (N = 16 / sizeof(T)) back into one 16-byte chunk of T.
template <typename T>
__device__ __forceinline__ u32x4 pack_chunk(const float* v) {
  u32x4 r;
  if constexpr (__is_same(T, float)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = __float_as_uint(v[e]);
  } else if constexpr (__is_same(T, bf16_t)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = f32_to_f16_bits(v[2 * e]) | (f32_to_f16_bits(v[2 * e + 1]) << 16);
  }
  return r;
}

// Qwen3's per-head QK-norm followed by RoPE on one head row of D = kR N elements held
// as one 16-byte chunk per lane of a kR-lane group (lane r: elements r N .. r N + N - 1):
// rmsnorm -> rope with the unfused kernels' rounding points (the sum of squares in
// rmsnorm_vec_kernel's order, the norm output rounded to T, then the rotation of those
// rounded values). `wf` are the lane's norm weights, `c` and `sn` its cosines and sines
// at the row's position, the sign of the low half already folded into `sn`
// (x_lo cos - x_hi sin = x_lo cos + x_hi (-sin), exactly). The rotation partner holds
// dims +-D/2, i.e. lane r ^ (kR / 2): for kR = 16 a rotation by 8 inside a 16-lane DPP
// row. Every lane of the group must call it (cross-lane operations). Returns the
// rotated chunk rounded to T. Shared by the QK-norm + RoPE kernel and the decode
// attention that normalises the step's new token itself, so both give the same bits;
// every file that calls it is compiled with -ffp-contract=off (each product and sum
// rounded on its own, as the unfused kernels and torch round them).
template <typename T, int kR>
__device__ __forceinline__ u32x4 norm_rope_chunk(const u32x4& held, const float* wf,
                                                 const float* c, const float* sn, float eps) {
  constexpr int N = Chunk<T>::kN;
  constexpr int D = kR * N;
  float f[N];
  Chunk<T>::unpack(held, f);
  float sumsq = 0.0f;
#pragma unroll
  for (int e = 0; e < N; ++e) sumsq = fmaf(f[e], f[e], sumsq);
  sumsq = group_sum<kR>(sumsq);
  const float inv = rsqrtf(sumsq / static_cast<float>(D) + eps);
  float y[N];
#pragma unroll
  for (int e = 0; e < N; e += 2) {
    if constexpr (N == 4) {
      y[e] = __fmul_rn(__fmul_rn(f[e], inv), wf[e]);
      y[e + 1] = __fmul_rn(__fmul_rn(f[e + 1], inv), wf[e + 1]);
    } else {
      float n0 = __fmul_rn(f[e], inv), n1 = __fmul_rn(f[e + 1], inv);
      round_pair<T>(n0, n1);
      y[e] = __fmul_rn(n0, wf[e]);
      y[e + 1] = __fmul_rn(n1, wf[e + 1]);
      round_pair<T>(y[e], y[e + 1]);
    }
  }
  float out[N];
#pragma unroll
  for (int e = 0; e < N; ++e) {
    float py;
    if constexpr (kR == 16) {
      py = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(y[e]), 0x128, 0xF, 0xF, false));
    } else {
      py = __shfl_xor(y[e], kR / 2, kWave);
    }
    out[e] = __fadd_rn(__fmul_rn(y[e], c[e]), __fmul_rn(py, sn[e]));
  }
  return pack_chunk<T>(out);
}

// Sum over a workgroup of `kWaves` waves, through `kWaves` floats of LDS. Every
// thread of the workgroup must call it.
template <int kWaves>
__device__ __forceinline__ float block_sum(float v, float* lds) {
  v = wave_sum(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) lds[wave] = v;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) total += lds[w];
  return total;
}

}  // namespace mvllm
