// Shared device helpers for the gfx950 (CDNA4) kernels of libqutai_amd.
//
// Element codes follow the storage dtype table of the reference CUDA backend
// (src/qutai/backends/cuda.py:17, `_TYPES` order: float32=0, float64=1,
// complex64=2, complex128=3, int64=4, bfloat16=5), so a host that already
// speaks those codes can pass them straight through the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qa {

enum Dtype : int { F32 = 0, F64 = 1, I64 = 4, BF16 = 5 };

typedef uint16_t bf16_t;  // raw bfloat16 bits in HBM
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(short)))) short i16x8;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

// bfloat16 -> float is exact: the 16 bits become the high half of an fp32.
__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}

// float -> bfloat16 with gfx950's v_cvt_pk_bf16_f32: round to nearest even,
// denormals kept, and a NaN becomes (bits >> 16) | 0x40 (quiet, sign and top
// payload bits kept).  That is bit for bit the reference host encoder's rule
// (src/qutai/backends/cuda.py:98-101), checked on the GPU over the special
// values and 4M random bit patterns.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {  // low half = a
  f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return (bf16_t)(pack_bf16x2(f, 0.0f) & 0xffffu); }

// silu(v) = v * sigmoid(v) = v / (1 + e^-v), the function of lm_silu
// (src/qutai/backends/cuda/lm.cu:54), from the hardware exp2 (v_exp_f32) and
// reciprocal (v_rcp_f32): a few fp32 ulps, far inside one bf16 ulp, and
// branch-free for every v (e^-v = inf gives v * 0).  One definition for the
// elementwise SwiGLU kernels and the fused GEMM epilogue, so both round the
// same values.
__device__ __forceinline__ float sigmoid_f(float v) { return __builtin_amdgcn_rcpf(1.f + __expf(-v)); }
__device__ __forceinline__ float silu_f(float v) { return v * sigmoid_f(v); }

// Store through a global (address space 1) pointer: a generic pointer makes
// the compiler emit flat stores, which also count against lgkmcnt, so every
// later wait for an LDS read would wait for the stores as well.
template <class V, class P>
__device__ __forceinline__ void global_store(P* p, const V& v) {
  *(__attribute__((address_space(1))) V*)(p) = v;
}
// Streaming store (the nontemporal hint): for outputs written once and not
// read back by the same kernel, e.g. GEMM results.  Config 3's write-bound
// score product S = Q K^T: 294 -> 224 us (3.9 -> 5.1 TB/s).
template <class V, class P>
__device__ __forceinline__ void global_store_nt(P* p, const V& v) {
  __builtin_nontemporal_store(v, (__attribute__((address_space(1))) V*)(p));
}
template <class V, class P>
__device__ __forceinline__ V global_load(const P* p) {
  return *(const __attribute__((address_space(1))) V*)(p);
}
// Streaming load (the nontemporal hint) of data read once by the launch, in
// whole 128-byte lines per instruction (see lds_load16_nt).
template <class V, class P>
__device__ __forceinline__ V global_load_nt(const P* p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) V*)(p));
}

// Values that are the same for the whole wavefront but that the compiler
// cannot prove uniform (e.g. derived from a runtime division of blockIdx)
// are pinned to scalar registers; a buffer descriptor built from them then
// stays in SGPRs instead of needing a per-lane waterfall loop.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)v);
  uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int uniform32(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <class P>
__device__ __forceinline__ P* uniform_ptr(P* p) {
  return reinterpret_cast<P*>(uniform64(reinterpret_cast<int64_t>(p)));
}

// MI355X has 8 XCDs, each with its own L2.  Consecutive workgroup ids are
// dispatched round-robin over the XCDs, so id i runs on XCD i % 8.  This maps
// the hardware id to a "logical" id such that each XCD receives one
// contiguous range of logical ids (sizes differ by at most one); tiles that
// are adjacent in logical order then share one L2.
__device__ __forceinline__ int xcd_remap(int pid, int n) {
  const int xcds = 8;
  int xcd = pid % xcds, q = pid / xcds;
  int per = n / xcds, rem = n % xcds;
  return xcd < rem ? xcd * (per + 1) + q : rem * (per + 1) + (xcd - rem) * per + q;
}

// ---- direct-to-LDS buffer loads ---------------------------------------------
// Buffer descriptor words (base, stride 0, num_records, dword3) held in
// SGPRs; an offset at or beyond num_records reads as zeros.
__device__ __forceinline__ u32x4 lds_rsrc(const void* base, int64_t bytes) {
  const uint32_t n = bytes > 0x7ffffff0 ? 0x7ffffff0u : (uint32_t)(bytes < 0 ? 0 : bytes);
  const uint64_t a = (uint64_t)(uintptr_t)base;
  u32x4 d = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
             (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu),
             (uint32_t)__builtin_amdgcn_readfirstlane(n), 0x00020000u};
  return d;
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// buffer_load_dwordx4 ... lds: lane l's 16 bytes at `voffset` land at
// lds + 16 l.  Issued from inline assembly so that the compiler does not
// treat it as a pending LDS write that every later LDS read has to wait for
// (it cannot tell the destination apart from the buffers being read and
// would insert s_waitcnt vmcnt(0) before them).  Callers order copies and
// reads themselves: s_waitcnt vmcnt, then s_barrier, before reading a
// buffer; no copy into a buffer before every wave has finished reading it.
__device__ __forceinline__ void lds_load16(u32x4 rsrc, void* lds, uint32_t voffset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}
// The same copy with the nontemporal (streaming) hint, for an operand that
// the launch reads exactly once, in whole 128-byte lines (each 16-byte
// chunk's line is consumed by the same instruction): such lines are not
// kept for reuse.  Streamed reads of 1 GiB measured 6.7-6.8 TB/s with the
// hint against 5.9-6.0 TB/s without it; reading half lines with it lets the
// other half miss and be fetched a second time (a 64-byte-per-row walk of
// the config-3 P.V operand ran 40% slower), hence the whole-line condition.
__device__ __forceinline__ void lds_load16_nt(u32x4 rsrc, void* lds, uint32_t voffset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(m0), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}
// s_waitcnt vmcnt(N) through the builtin (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima), so that the
// compiler's own wait placement knows that the loads it issued are done.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// Same with 4 bytes per lane (lane l's dword lands at lds + 4 l).
__device__ __forceinline__ void lds_load4(u32x4 rsrc, void* lds, uint32_t voffset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

}  // namespace qa
