// mcpm_device.h -- device-side building blocks shared by the kernels.
#pragma once

#include "mcpm_internal.h"

namespace mcpm {


typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));  // native vectors: copies stay in registers

__device__ __forceinline__ u32x4 ld_stream4(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld_stream2(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
__device__ __forceinline__ uint16_t ld_stream_u16(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
}

// Loads and stores of data that other work groups of the same launch write
// or read (the fused kernels): the sc1 bit makes them coherent across the
// XCDs' L2s (written through, read from the coherence point).  The vector
// load goes through a raw buffer resource on a wave-uniform base so that its
// cache policy can be set; `byte_off` is the lane's offset from it.
__device__ __forceinline__ f32x4 ld_coh4(const float* base, uint32_t byte_off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0), 0x7fffffff, 0x00020000);
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16));
}
__device__ __forceinline__ float ld_coh(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this wave's stores are acknowledged (written through, for
// sc1 stores): before it tells other work groups that its outputs are there.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Lane moves within rows of 16 lanes (DPP): quad_perm [1,0,3,2] (lane ^ 1),
// quad_perm [2,3,0,1] (lane ^ 2), row rotate by 4 and by 8.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_ROR4 = 0x124, DPP_ROR8 = 0x128;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

// LDS stores of the wave before this point are seen by its loads after it
// (other lanes' stores included).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Maximum over the 16 lanes of the row, on every lane of the row.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<DPP_XOR1>(v));
  v = fmaxf(v, dpp_f<DPP_XOR2>(v));
  v = fmaxf(v, dpp_f<DPP_ROR4>(v));
  v = fmaxf(v, dpp_f<DPP_ROR8>(v));
  return v;
}

// v of lane ^ 16 and of lane ^ 32 by gfx950's row swaps (v_permlane16_swap /
// v_permlane32_swap on two copies of v), in VALU instead of an LDS-routed
// permute.  permlane16_swap(v, v) gives rows (0, 0, 2, 2) and (1, 1, 3, 3) of
// v; permlane32_swap(v, v) gives rows (0, 1, 0, 1) and (2, 3, 2, 3).
__device__ __forceinline__ float lane_xor16(float v) {
  const unsigned u = __float_as_uint(v);
  const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float((threadIdx.x & 16) ? p[0] : p[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
  const unsigned u = __float_as_uint(v);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float((threadIdx.x & 32) ? p[0] : p[1]);
}

// Maximum over the wave on every lane (order-free): within rows, then across.
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  v = fmaxf(v, lane_xor16(v));
  return fmaxf(v, lane_xor32(v));
}

// Pairwise tree over the 64 lanes: lane t += lane t+s for s = 32..1; lane 0
// holds the total (the oracle's tree_sum over 64 slots).  s = 32, 16 across
// rows (lane t < s reads lane t + s = t ^ s; the other lanes' values are not
// read again by lane 0's chain), s <= 8 by DPP row shifts (only lanes < s
// read, and those stay inside their row).  Only lane 0's value is defined.
__device__ __forceinline__ float wave_tree_sum(float v) {
  v = v + lane_xor32(v);
  v = v + lane_xor16(v);
  v = v + dpp_f<0x108>(v);  // row_shl:8
  v = v + dpp_f<0x104>(v);  // row_shl:4
  v = v + dpp_f<0x102>(v);  // row_shl:2
  v = v + dpp_f<0x101>(v);  // row_shl:1
  return v;
}

// Quantizes one 256-value block held by a wave (lane l owns values 4l..4l+3):
// packed bytes of the lane, the block scale d, and (on lanes l%4 == 0) the sum
// of the 16 values of group l/4.  amax == 0 gives an all-zero block
// (src/ops/ops.cpp:704-709, src/ops/ops_avx2.cpp:106-111).
__device__ __forceinline__ void quant_block_wave(const float v[4], bool away, uint32_t& packed, float& d,
                                                 int& gsum) {
  float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  const float amax = wave_max(a);
  if (amax == 0.0f) {
    packed = 0;
    d = 0.0f;
    gsum = 0;
    return;
  }
  d = amax * (1.0f / 127.0f);
  const float mul = 127.0f / amax;
  int s = 0;
  uint32_t p = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float t = v[k] * mul;
    float r = away ? roundf(t) : rintf(t);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    const int q = static_cast<int>(r);
    s += q;
    p |= (static_cast<uint32_t>(q) & 0xffu) << (8 * k);
  }
  s += dpp_i<DPP_XOR1>(s);
  s += dpp_i<DPP_XOR2>(s);
  packed = p;
  gsum = s;
}

// Quantizes one 256-value block held by a row of 16 lanes (lane j owns values
// 16j..16j+15, i.e. Q8_K group j): the lane's 16 codes packed four to a dword,
// the block scale d, and the sum of the lane's codes (bsums[j]).  The same
// operations as quant_block_wave; amax == 0 gives an all-zero block.
__device__ __forceinline__ void quant_block_row16(const float (&v)[16], bool away, u32x4& packed, float& d,
                                                  int& gsum) {
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) a = fmaxf(a, fabsf(v[i]));
  const float amax = row16_max(a);
  const bool zero = (amax == 0.0f);
  d = zero ? 0.0f : amax * (1.0f / 127.0f);
  const float mul = zero ? 0.0f : 127.0f / amax;
  int q[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float t = v[i] * mul;
    // ties away: t + copysign(0.5 - 2^-25, t) truncates to roundf(t) for every
    // |t| < 128 (|t| <= 127 here), so the clamp and the truncating conversion
    // finish both roundings
    float r = away ? t + __builtin_copysignf(0.49999997f, t) : rintf(t);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    q[i] = static_cast<int>(r);
  }
  // low bytes of four codes into a dword (three byte permutes), and the code
  // sum as byte dots against 1s
  uint32_t w[4];
  int s = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo = __builtin_amdgcn_perm(static_cast<uint32_t>(q[4 * k + 1]), static_cast<uint32_t>(q[4 * k]), 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(static_cast<uint32_t>(q[4 * k + 3]), static_cast<uint32_t>(q[4 * k + 2]), 0x0c0c0400u);
    w[k] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    s = __builtin_amdgcn_sdot4(static_cast<int>(w[k]), 0x01010101, s, false);
  }
  packed = u32x4{w[0], w[1], w[2], w[3]};
  gsum = s;
}

// The same tree (kept under the name its callers use).
__device__ __forceinline__ float wave_tree_sum_fast(float v) { return wave_tree_sum(v); }

// block_rms_from_partials with one barrier: every wave runs the tree over the
// 256 slots itself (slots l, l+64, l+128, l+192 on lane l, then the wave tree),
// so no second barrier hands the result out.  Same sums in the same order.
__device__ __forceinline__ float block_rms_1sync(float p, int dim, float eps, float* s_red) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 256) s_red[tid] = p;
  __syncthreads();
  float v = (s_red[lane] + s_red[lane + 128]) + (s_red[lane + 64] + s_red[lane + 192]);
  v = wave_tree_sum_fast(v);
  v = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
  return 1.0f / sqrtf(v / static_cast<float>(dim) + eps);
}

// 1/sqrt(sum/dim + eps) where sum is the 256-slot pairwise tree (slot t +=
// slot t+s for s = 128..1) over the partials p of threads 0..255; every
// thread of the work group (at least 256) gets it.
// Threads 256 and up (in larger work groups) take no slot.
__device__ __forceinline__ float block_rms_from_partials(float p, int dim, float eps, float* s_red) {
  const int tid = threadIdx.x;
  if (tid < 256) s_red[tid] = p;
  __syncthreads();
  if (tid < 128) s_red[tid] = s_red[tid] + s_red[tid + 128];
  __syncthreads();
  if (tid < 64) {
    float v = s_red[tid] + s_red[tid + 64];
    v = wave_tree_sum(v);
    if (tid == 0) s_red[256] = 1.0f / sqrtf(v / static_cast<float>(dim) + eps);
  }
  __syncthreads();
  const float r = s_red[256];
  __syncthreads();
  return r;
}

// Sum of squares over dim values with 256 threads: thread t sums x[t],
// x[t+256], ... (multiply then add), then the 256-slot pairwise tree.  All
// threads receive 1/sqrt(sum/dim + eps).  The loads are issued 8 at a time.
__device__ float block_rms_scale(const float* __restrict__ x, int dim, float eps, float* s_red) {
  const int tid = threadIdx.x;
  float p = 0.0f;
  for (int i0 = tid; i0 < dim; i0 += 8 * 256) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = x[min(i0 + 256 * k, dim - 1)];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (i0 + 256 * k < dim) p = p + v[k] * v[k];
  }
  return block_rms_from_partials(p, dim, eps, s_red);
}

// --------------------------------------------------------- weight planes ---
// Chunked planes hold 16-byte chunk c of block (b, r) at ((b*nc + c)*rows + r)*16
// (nc chunks per block), so consecutive rows' chunk c are adjacent.
__device__ __forceinline__ size_t chunk_off(int nc, size_t rows, int b, int c, size_t r) {
  return ((static_cast<size_t>(b) * nc + c) * rows + r) * 16;
}

// ------------------------------------------------------------- dequant -----
// Value e (0..255) of block (b, r).  Q4_K: (d*sc)*q - dmin*mn; Q6_K:
// (d*sc)*(q-32); Q8_0 handled separately.  Same expressions as
// src/ops/ops.cpp:655-664 and :194-228.
__device__ __forceinline__ float dequant_value(const WView& w, int r, int b, int e) {
  const size_t rows = static_cast<size_t>(w.rows);
  const size_t blk = static_cast<size_t>(b) * rows + r;
  if (w.type == MCPM_TYPE_Q4_K) {
    const uint8_t* meta = w.p1 + blk * 16;
    const uint16_t dh = meta[0] | (meta[1] << 8), mh = meta[2] | (meta[3] << 8);
    const uint8_t* sc = meta + 4;
    const int c = e / 64, l = e % 32, hi = (e % 64) >= 32;
    const int j = 2 * c + hi;
    int scv, mnv;
    if (j < 4) {
      scv = sc[j] & 63;
      mnv = sc[j + 4] & 63;
    } else {
      scv = (sc[j + 4] & 0x0f) | ((sc[j - 4] >> 6) << 4);
      mnv = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
    const int qbyte = 32 * c + l;  // native quant byte
    const uint8_t qb = w.p0[chunk_off(8, rows, b, qbyte >> 4, r) + (qbyte & 15)];
    const int qv = hi ? (qb >> 4) : (qb & 0x0f);
    const float d1 = fp16_to_fp32(dh) * static_cast<float>(scv);
    const float m1 = fp16_to_fp32(mh) * static_cast<float>(mnv);
    return d1 * static_cast<float>(qv) - m1;
  } else {
    const int h = e / 128, rr = e % 128, g = rr / 32, l = rr % 32;
    const int qlbyte = 64 * h + 32 * (g & 1) + l;  // native ql byte
    const uint8_t qlb = w.p0[chunk_off(8, rows, b, qlbyte >> 4, r) + (qlbyte & 15)];
    const int qhbyte = 32 * h + l;  // native qh byte
    const uint8_t qhb = w.p1[chunk_off(4, rows, b, qhbyte >> 4, r) + (qhbyte & 15)];
    const int lo = (g < 2) ? (qlb & 0x0f) : (qlb >> 4);
    const int qv = lo | (((qhb >> (2 * g)) & 3) << 4);
    const int8_t scv = static_cast<int8_t>(w.p2[blk * 16 + e / 16]);
    const uint16_t dh = w.p3[blk * 2] | (w.p3[blk * 2 + 1] << 8);
    return (fp16_to_fp32(dh) * static_cast<float>(scv)) * static_cast<float>(qv - 32);
  }
}

}  // namespace mcpm
