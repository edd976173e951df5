// Shared device/host helpers for the gfx950 kernels of the pre-LN transformer forward.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <string>

#include "tttj_amd.h"

namespace tt {

using half = _Float16;
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
// 16-byte staging register.  A native vector (not the uint4 struct): LLVM turns a struct
// load + store pair into a memcpy placed at the store, which would delay a prefetch load.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// ---- error reporting across the C ABI (no exceptions cross it) ----
void set_error(const std::string& msg);
int fail(int code, const char* fmt, ...);

#define TT_HIP(call)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (call);                                                            \
    if (e_ != hipSuccess)                                                              \
      return ::tt::fail(TT_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_));   \
  } while (0)

#define TT_REQUIRE(cond, ...)                                                          \
  do {                                                                                 \
    if (!(cond)) return ::tt::fail(TT_ERR_INVALID, __VA_ARGS__);                       \
  } while (0)

inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TT_ERR_HIP, "launch of %s failed: %s", what, hipGetErrorString(e));
  return TT_OK;
}

// ---- device helpers ----
__device__ __forceinline__ floatx16 mfma32x32x16(half8 a, half8 b, floatx16 c) {
  // v_mfma_f32_32x32x16_f16.  Lane l supplies A[row = l%32][k = 8*(l/32) + i] and
  // B[k = 8*(l/32) + i][col = l%32]; it receives C[row = 8*(j/4) + 4*(l/32) + j%4][col = l%32].
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx4 mfma16x16x32(half8 a, half8 b, floatx4 c) {
  // v_mfma_f32_16x16x32_f16.  Lane l supplies A[row = l%16][k = 8*(l/16) + i] and
  // B[k = 8*(l/16) + i][col = l%16]; it receives C[row = 4*(l/16) + j][col = l%16].
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// s_waitcnt on the vector-memory counter only: wait until at most N of this wave's vector memory
// operations are still in flight (loads, including global -> LDS copies, complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Workgroup barrier without the memory fence that __syncthreads() implies (that fence waits for
// every in-flight global load, vmcnt(0), which would drain a multi-stage copy pipeline).  Callers
// wait for exactly the copies they need with wait_vmcnt first.  The empty asm statements keep the
// compiler from moving memory operations across the barrier.
__device__ __forceinline__ void raw_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Barrier after this wave's LDS operations have completed (s_waitcnt lgkmcnt(0), vector-memory
// loads left in flight): for pipelines whose global loads run several stages ahead in registers.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt 63, expcnt 7, lgkmcnt 0
  raw_barrier();
}

// Cache policy of a load (the instruction's cache-control bits): kLoadDefault may hit in the CU's
// L1; kLoadDevice (sc1, device scope) misses the L1 and is served by the L2 of the XCD the CU
// belongs to.  Data written earlier in the same launch by a workgroup on another CU of the same
// XCD is in that shared L2 once the writer's stores have completed, while the reader's L1 may
// still hold older copies of those lines, so such data is read with kLoadDevice.
constexpr int kLoadDefault = 0;
constexpr int kLoadDevice = 16;

// Global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4): lane l writes LDS bytes
// [16 l, 16 l + 16) after the wave-uniform destination `lds_dst`.
template <int POLICY = kLoadDefault>
__device__ __forceinline__ void lds_copy16(const half* src, half* lds_dst) {
  __builtin_amdgcn_global_load_lds((const void*)src,
                                   (__attribute__((address_space(3))) void*)lds_dst, 16, 0, POLICY);
}

// 16 bytes per lane from byte offset `off` of the buffer `r` straight into LDS at lds_dst +
// 16 * lane (lds_dst wave-uniform); lanes whose 16 bytes lie outside the buffer read nothing
// from memory.
template <int POLICY = kLoadDefault>
__device__ __forceinline__ void lds_copy16_buf(__amdgpu_buffer_rsrc_t r, uint32_t off, half* lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_dst, 16,
                                           off, 0, 0, POLICY);
}

// Raw buffer resource over [base, base + bytes): stride 0; 0x00020000 is the data-format word
// for untyped 32-bit accesses.  `base` must be wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// 16-byte load at byte offset `off` of the buffer `r` with cache policy POLICY.
template <int POLICY>
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POLICY);
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of G lanes (G in {8, 16, 32, 64}), returned in every lane of the group.
// VALU-only: DPP within 16-lane rows (xor 1, xor 2, half-mirror, mirror), then the gfx950 row
// swaps v_permlane16_swap / v_permlane32_swap across rows (no LDS round trips).
template <int G>
__device__ __forceinline__ float seg_sum(float v) {
  static_assert(G == 8 || G == 16 || G == 32 || G == 64, "group size");
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror: lanes i <-> 7 - i within 8
  if constexpr (G >= 16) v += dpp_mov<0x140>(v);  // row_mirror: i <-> 15 - i within 16
  if constexpr (G >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (G >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return seg_sum<64>(v); }

// Sum over aligned groups of G lanes for G in {4, 8, 16, 32, 64} (quad_perm for 4).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G == 1) {
    return v;
  } else if constexpr (G == 4) {
    v += dpp_mov<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);  // quad_perm [2,3,0,1]
    return v;
  } else {
    return seg_sum<G>(v);
  }
}

// Partial row statistics for a LayerNorm folded into the next projection: a slot holds
// (mean, M2) -- the mean and the centred sum of squares -- of N consecutive values of a row.
// `v` are this lane's NV values; the slot spans the G aligned lanes of the group (NV G values).
template <int G, int NV>
__device__ __forceinline__ float2 slot_stats(const float (&v)[NV]) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < NV; ++e) s += v[e];
  const float mean = group_sum<G>(s) * (1.0f / (NV * G));
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < NV; ++e) {
    const float t = v[e] - mean;
    q = fmaf(t, t, q);
  }
  return make_float2(mean, group_sum<G>(q));
}

// combine_row_stats for a row shared by G aligned lanes: lane j takes slots j, j + G, ... (one load
// each when slots <= G), and the G partial results are merged with group sums.
template <int G>
__device__ __forceinline__ float2 combine_row_stats_group(const float2* part, int slots, int K) {
  const int j = threadIdx.x & (G - 1);
  const float n = (float)(K / slots);
  float mean = 0.f, m2 = 0.f, cnt = 0.f;
  for (int s = j; s < slots; s += G) {
    const float2 v = part[s];
    const float tot = cnt + n, d = v.x - mean;
    m2 += v.y + d * d * (cnt * n / tot);
    mean += d * (n / tot);
    cnt = tot;
  }
  const float mu = group_sum<G>(cnt * mean) / (float)K;
  const float d = mean - mu;
  const float M2 = group_sum<G>(fmaf(cnt * d, d, m2));
  return make_float2(mu, rsqrtf(M2 / (float)K + 1e-5f));
}

// (mean, rstd) of a row of K values from its `slots` partial (mean, M2) slots of K / slots values
// each, biased variance and eps 1e-5 (the statistics nn.LayerNorm uses).  Slots are loaded 16 at a
// time with one wait (indices clamped, so every load is unconditional), each chunk combined as
// M2 = sum M2_s + n sum (mean_s - mean)^2, and chunks merged pairwise (Chan et al.).
__device__ __forceinline__ float2 combine_row_stats(const float2* part, int slots, int K) {
  constexpr int C = 16;
  const float n = (float)(K / slots);
  float mean = 0.f, m2 = 0.f, cnt = 0.f;
  for (int s0 = 0; s0 < slots; s0 += C) {
    float2 v[C];
#pragma unroll
    for (int i = 0; i < C; ++i) v[i] = part[min(s0 + i, slots - 1)];
    const int c = min(C, slots - s0);
    float cm = 0.f;
#pragma unroll
    for (int i = 0; i < C; ++i) cm += i < c ? v[i].x : 0.f;
    cm *= __builtin_amdgcn_rcpf((float)c);
    float cq = 0.f;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const float d = v[i].x - cm;
      cq += i < c ? fmaf(n * d, d, v[i].y) : 0.f;
    }
    const float cn = n * (float)c, tot = cnt + cn;
    const float d = cm - mean;
    m2 += cq + d * d * (cnt * cn / tot);
    mean += d * (cn / tot);
    cnt = tot;
  }
  return make_float2(mean, rsqrtf(m2 / (float)K + 1e-5f));
}

__device__ __forceinline__ float gelu_erf(float v) {
  // Exact-erf GELU, F.gelu(approximate="none"): v * Phi(v), Phi(v) = erfc(-v / sqrt 2) / 2.
  // With z = |v| / sqrt 2, erfc(z) = t * exp(-z^2 + P(t)), t = 1 / (1 + z/2) and P a degree-6
  // polynomial fitted at Chebyshev nodes on t in [0.4, 1] (z <= 3; the form of Numerical Recipes
  // 6.2; fit_erfc.py derives the coefficients), relative error < 3.4e-7 there; for larger z the
  // polynomial extrapolates smoothly and exp(-z^2) makes |v| q negligible against v (v > 0) or the
  // result an fp16 subnormal (v < 0).  Evaluated in the exp2 domain: w = |v| sqrt(log2(e) / 2),
  // q = erfc(z) / 2 = t * exp2(Q(t) - w^2) with Q = log2(e) P - 1, and since Phi(v) = 1 - q for
  // v >= 0 and q for v < 0, GELU(v) = max(v, 0) - |v| q for either sign: branch-free, 14 VALU
  // operations.  The fp16 result is the correctly rounded GELU on all but ~3e-4 of the fp16 inputs
  // in [-12, 12], which are one ulp off next to a rounding tie.
  const float a = fabsf(v);
  const float w = a * 8.493218003e-01f;
  const float t = __builtin_amdgcn_rcpf(fmaf(w, 4.162773056e-01f, 1.0f));
  float p = -2.175998778e-01f;
  p = fmaf(p, t, 1.191431602e+00f);
  p = fmaf(p, t, -2.406964312e+00f);
  p = fmaf(p, t, 1.837399633e+00f);
  p = fmaf(p, t, -1.574934214e-01f);
  p = fmaf(p, t, 1.592239249e+00f);
  p = fmaf(p, t, -2.839012633e+00f);
  const float q = t * __builtin_amdgcn_exp2f(fmaf(-w, w, p));
  return fmaf(-a, q, fmaxf(v, 0.f));
}

}  // namespace tt
