// Shared device helpers for the gfx950 self-spec kernels: bf16 bit conversions, wavefront reductions, vector types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gss.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define GSS_DEV __device__ __forceinline__

GSS_DEV float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// Round-to-nearest-even fp32 -> bf16, the rounding of torch's .to(torch.bfloat16), in gfx950's conversion
// instruction (v_cvt_pk_bf16_f32, one instruction per pair; NaN stays a quiet NaN).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

GSS_DEV uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

GSS_DEV uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

GSS_DEV float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// The value lane (lane ^ o) holds, for o in {1, 2, 4, 8, 16, 32}: what __shfl_xor(v, o, 64) returns, without its
// LDS-crossbar round trip (~100 clocks each, six of them chained in a wave reduction): the gfx950 lane swaps across
// 32 and across 16 lanes, and DPP within a row of 16 (rotating a row by 8 is xor 8; xor 4 takes the row shifted by
// 4 one way or the other; xor 2 and 1 are quad permutations). Every lane of the wave must be active. With o a
// constant after unrolling, the switch folds to one case.
GSS_DEV uint32_t lane_xor(uint32_t u, int o) {
  const int lane = threadIdx.x & 63;
  switch (o) {
    case 32: {
      const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      return lane < 32 ? p[1] : p[0];
    }
    case 16: {
      const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
      return (lane & 16) ? p[0] : p[1];
    }
    case 8:
      return __builtin_amdgcn_update_dpp(0u, u, 0x128, 0xf, 0xf, false);  // row_ror:8
    case 4: {
      const uint32_t r = __builtin_amdgcn_update_dpp(0u, u, 0x114, 0xf, 0xf, false);  // row_shr:4
      const uint32_t l = __builtin_amdgcn_update_dpp(0u, u, 0x104, 0xf, 0xf, false);  // row_shl:4
      return (lane & 4) ? r : l;
    }
    case 2:
      return __builtin_amdgcn_update_dpp(0u, u, 0x4e, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    case 1:
      return __builtin_amdgcn_update_dpp(0u, u, 0xb1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    default:
      return static_cast<uint32_t>(__shfl_xor(static_cast<int>(u), o, 64));
  }
}
GSS_DEV float lane_xor(float v, int o) { return __uint_as_float(lane_xor(__float_as_uint(v), o)); }
GSS_DEV int lane_xor(int v, int o) { return static_cast<int>(lane_xor(static_cast<uint32_t>(v), o)); }

GSS_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += lane_xor(v, o);
  return v;
}

GSS_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, lane_xor(v, o));
  return v;
}

// Block-wide sum for blockDim.x threads (multiple of 64, <= 1024); `red` needs blockDim.x / 64 floats of LDS.
GSS_DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nw; ++i) s += red[i];
  return s;
}

// Handoffs between workgroups of one kernel (a last-arriving workgroup finishing the work of the others). The data
// handed over is written and read with agent-scope relaxed atomics, which on gfx950 are plain vector stores / loads
// with the sc1 bit: written through to, and read from, the coherence point shared by all XCDs. No L2 write-back or
// invalidate is needed for it. A writer issues wait_stores() in every wave (its stores are complete), then a
// workgroup barrier, then a relaxed counter increment; the workgroup that sees the final count reads with ld_agent.
GSS_DEV void st_agent(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
GSS_DEV void st_agent(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
GSS_DEV uint32_t ld_agent(const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
GSS_DEV uint64_t ld_agent(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
GSS_DEV void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
GSS_DEV uint32_t count_arrival(uint32_t* ctr) {
  return __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
GSS_DEV void reset_counter(uint32_t* ctr) { __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Coherent 16-byte store (st_agent's sc1 form of global_store_dwordx4); 16-byte aligned.
GSS_DEV void st_agent_x4(void* p, u32x4_t v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

// Batched coherent 4-byte loads (ld_agent's instruction), n (1..3) issued back to back and waited for once.
GSS_DEV void ld_agent_u32(int n, const uint32_t* p0, const uint32_t* p1, const uint32_t* p2, uint32_t& r0,
                          uint32_t& r1, uint32_t& r2) {
  switch (n) {
    case 1:
      asm volatile("global_load_dword %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=&v"(r0) : "v"(p0) : "memory");
      break;
    case 2:
      asm volatile("global_load_dword %0, %2, off sc1\n\tglobal_load_dword %1, %3, off sc1\n\ts_waitcnt vmcnt(0)"
                   : "=&v"(r0), "=&v"(r1)
                   : "v"(p0), "v"(p1)
                   : "memory");
      break;
    default:
      asm volatile(
          "global_load_dword %0, %3, off sc1\n\tglobal_load_dword %1, %4, off sc1\n\t"
          "global_load_dword %2, %5, off sc1\n\ts_waitcnt vmcnt(0)"
          : "=&v"(r0), "=&v"(r1), "=&v"(r2)
          : "v"(p0), "v"(p1), "v"(p2)
          : "memory");
      break;
  }
}

// Batched coherent 16-byte loads for handed-over data: ld_agent's sc1 form of global_load_dwordx4, n (1..4) of them
// issued back to back and waited for once inside the same asm statement (the compiler waits after every atomic load,
// which serializes a series of ld_agent calls into one memory round trip each). Pointers must be 16-byte aligned.
GSS_DEV void ld_agent_x4(int n, const void* p0, const void* p1, const void* p2, const void* p3, u32x4_t& r0,
                         u32x4_t& r1, u32x4_t& r2, u32x4_t& r3) {
  switch (n) {
    case 1:
      asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=&v"(r0) : "v"(p0) : "memory");
      break;
    case 2:
      asm volatile(
          "global_load_dwordx4 %0, %2, off sc1\n\tglobal_load_dwordx4 %1, %3, off sc1\n\ts_waitcnt vmcnt(0)"
          : "=&v"(r0), "=&v"(r1)
          : "v"(p0), "v"(p1)
          : "memory");
      break;
    case 3:
      asm volatile(
          "global_load_dwordx4 %0, %3, off sc1\n\tglobal_load_dwordx4 %1, %4, off sc1\n\t"
          "global_load_dwordx4 %2, %5, off sc1\n\ts_waitcnt vmcnt(0)"
          : "=&v"(r0), "=&v"(r1), "=&v"(r2)
          : "v"(p0), "v"(p1), "v"(p2)
          : "memory");
      break;
    default:
      asm volatile(
          "global_load_dwordx4 %0, %4, off sc1\n\tglobal_load_dwordx4 %1, %5, off sc1\n\t"
          "global_load_dwordx4 %2, %6, off sc1\n\tglobal_load_dwordx4 %3, %7, off sc1\n\ts_waitcnt vmcnt(0)"
          : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
          : "v"(p0), "v"(p1), "v"(p2), "v"(p3)
          : "memory");
      break;
  }
}

inline int gss_launch_status() { return hipGetLastError() == hipSuccess ? GSS_OK : GSS_ERR_LAUNCH; }
