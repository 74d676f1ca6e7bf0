// mcpm_kernels.hip -- gfx950 kernels of the decode path.
//
// Numerics contract (the CPU oracle follows the same sequences):
//  * Q4_K/Q6_K x Q8_K dots form, per 256-block, the eight int32 lane sums of
//    the reference's AVX2 kernels (src/ops/ops_avx2.cpp:161-181, 224-270):
//    lane m folds bytes 4m..4m+3 of every 32-byte group.  Per row, lane m then
//    runs acc_m = fma(d_x*d_w, float(isum_m), acc_m) over blocks in order,
//    Q4_K adds acc_min = fma(-(d_x*dmin_w), float(minsum), acc_min), and the
//    lanes are summed ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) (ops_avx2.cpp:43-48).
//    The result is bit-identical to the reference's compiled AVX2 GEMV.
//  * Q8_K quantization: d = amax*(1/127), v = x*(127/amax), rint or round.
//  * Sums of squares: 256 strided partials, then a pairwise tree.
//  * Everything is compiled with -ffp-contract=off; fused multiply-adds are
//    explicit.
#include "mcpm_internal.h"

namespace mcpm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x4 ld_stream4(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld_stream2(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
__device__ __forceinline__ uint16_t ld_stream_u16(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Pairwise tree over the 64 lanes: lane t += lane t+s for s = 32..1; lane 0
// holds the total (the oracle's tree_sum over 64 slots).
__device__ __forceinline__ float wave_tree_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = v + __shfl_down(v, o);
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
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  packed = p;
  gsum = s;
}

// Sum of squares over dim values with 256 threads: thread t sums x[t],
// x[t+256], ... (multiply then add), then the 256-slot pairwise tree.  All
// threads receive 1/sqrt(sum/dim + eps).
__device__ float block_rms_scale(const float* __restrict__ x, int dim, float eps, float* s_red) {
  const int tid = threadIdx.x;
  float p = 0.0f;
  for (int i = tid; i < dim; i += 256) {
    const float v = x[i];
    p = p + v * v;
  }
  s_red[tid] = p;
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

// Position of the activation dword holding elements 4l..4l+3 of a block in
// the GEMV's LDS image: lane m of 8 reads dwords x[32k+4m] (k = 0..7) as 32
// contiguous bytes at m*32.
__device__ __forceinline__ int xq_slot(int l) { return (l & 7) * 8 + (l >> 3); }

// --------------------------------------------------------------- Q4_K -------
// One block of one row for lane m: isum over the lane's bytes and the lane's
// share of the min correction, mn[m] * (bsums[2m] + bsums[2m+1]).
__device__ __forceinline__ void q4k_lane(const u32x4 q, const u32x4 meta, const uint32_t* __restrict__ xl,
                                         const int* __restrict__ bs, int m, int& isum, int& minp) {
  const uint32_t s0 = meta.y, s1 = meta.z, s2 = meta.w;
  int sc[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sc[j] = (s0 >> (8 * j)) & 63;
    sc[j + 4] = ((s2 >> (8 * j)) & 0x0f) | (((s0 >> (8 * j + 6)) & 3) << 4);
  }
  int mn;
  if (m < 4) mn = (s1 >> (8 * m)) & 63;
  else mn = ((s2 >> (8 * (m - 4) + 4)) & 0x0f) | (((s1 >> (8 * (m - 4) + 6)) & 3) << 4);
  int acc = 0;
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int lo = static_cast<int>(qw[j] & 0x0f0f0f0fu);
    const int hi = static_cast<int>((qw[j] >> 4) & 0x0f0f0f0fu);
    const int dlo = __builtin_amdgcn_sdot4(lo, static_cast<int>(xl[2 * j]), 0, false);
    const int dhi = __builtin_amdgcn_sdot4(hi, static_cast<int>(xl[2 * j + 1]), 0, false);
    acc += sc[2 * j] * dlo + sc[2 * j + 1] * dhi;
  }
  isum = acc;
  minp = mn * (bs[2 * m] + bs[2 * m + 1]);
}

// --------------------------------------------------------------- Q6_K -------
__device__ __forceinline__ int sbyte(const u32x4 w, int i) {
  const uint32_t word = (i < 4) ? w.x : (i < 8) ? w.y : (i < 12) ? w.z : w.w;
  return static_cast<int>(static_cast<int8_t>((word >> (8 * (i & 3))) & 0xffu));
}

__device__ __forceinline__ int q6k_lane(const u32x4 ql, const u32x2 qh, const u32x4 scw,
                                        const uint32_t* __restrict__ xl, const int* __restrict__ bs, int m) {
  const int hi = (m >= 4) ? 1 : 0;
  int acc = 0;
  const uint32_t A[4] = {ql.x, ql.y, ql.z, ql.w};
  const uint32_t H[2] = {qh.x, qh.y};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t a0 = A[2 * h], a1 = A[2 * h + 1], hb = H[h];
    const uint32_t q0 = (a0 & 0x0f0f0f0fu) | ((hb & 0x03030303u) << 4);
    const uint32_t q1 = (a1 & 0x0f0f0f0fu) | ((hb & 0x0c0c0c0cu) << 2);
    const uint32_t q2 = ((a0 >> 4) & 0x0f0f0f0fu) | (hb & 0x30303030u);
    const uint32_t q3 = ((a1 >> 4) & 0x0f0f0f0fu) | ((hb & 0xc0c0c0c0u) >> 2);
    const int d0 = __builtin_amdgcn_sdot4(static_cast<int>(q0), static_cast<int>(xl[4 * h + 0]), 0, false);
    const int d1 = __builtin_amdgcn_sdot4(static_cast<int>(q1), static_cast<int>(xl[4 * h + 1]), 0, false);
    const int d2 = __builtin_amdgcn_sdot4(static_cast<int>(q2), static_cast<int>(xl[4 * h + 2]), 0, false);
    const int d3 = __builtin_amdgcn_sdot4(static_cast<int>(q3), static_cast<int>(xl[4 * h + 3]), 0, false);
    acc += sbyte(scw, 8 * h + 0 + hi) * d0 + sbyte(scw, 8 * h + 2 + hi) * d1 + sbyte(scw, 8 * h + 4 + hi) * d2 +
           sbyte(scw, 8 * h + 6 + hi) * d3;
  }
  const int off = bs[2 * m] * sbyte(scw, 2 * m) + bs[2 * m + 1] * sbyte(scw, 2 * m + 1);
  return acc - 32 * off;
}

// ------------------------------------------------------------ the GEMV ------
struct GemvSmem {
  uint32_t xq[MAX_NB * 64];
  float xd[MAX_NB];
  int bsum[MAX_NB * 16];
  int isum[MAX_NB * 64];
  int minsum[MAX_NB * 8];
  float ds[MAX_NB * 8];
  float dm[MAX_NB * 8];
  float red[260];
};

__device__ __forceinline__ void resolve_slot(const GemvArgs& a, int g, int s, int& reg, int& r, bool& valid) {
  if (a.pair) {
    reg = s >> 2;
    r = g * 4 + (s & 3);
    valid = r < a.total_rows;
  } else {
    const int vr = g * ROWS_PER_GROUP + s;
    valid = vr < a.total_rows;
    reg = 0;
    if (a.nreg > 1 && vr >= a.reg[1].row0) reg = 1;
    if (a.nreg > 2 && vr >= a.reg[2].row0) reg = 2;
    r = vr - a.reg[reg].row0;
  }
}

template <int PRO, int EPI>
__global__ void __launch_bounds__(GEMV_THREADS) k_gemv_q8k(const GemvArgs a) {
  __shared__ GemvSmem sm;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nb = a.nb;

  // ---- prologue: Q8_K activations into LDS
  if constexpr (PRO == PRO_Q8K) {
    for (int b = wave; b < nb; b += 4) {
      const BlockQ8K* blk = a.xq + b;
      sm.xq[b * 64 + xq_slot(lane)] = reinterpret_cast<const uint32_t*>(blk->qs)[lane];
      if (lane < 16) sm.bsum[b * 16 + lane] = blk->bsums[lane];
      if (lane == 0) sm.xd[b] = blk->d;
    }
  } else {
    constexpr bool norm = (PRO == PRO_NORM_AWAY || PRO == PRO_NORM_EVEN);
    constexpr bool away = (PRO == PRO_QUANT_AWAY || PRO == PRO_NORM_AWAY);
    float rms = 1.0f;
    if constexpr (norm) rms = block_rms_scale(a.x, nb * QK_K, a.eps, sm.red);
    for (int b = wave; b < nb; b += 4) {
      const float4 xv = reinterpret_cast<const float4*>(a.x + b * QK_K)[lane];
      float v[4] = {xv.x, xv.y, xv.z, xv.w};
      if constexpr (norm) {
        const float4 gv = reinterpret_cast<const float4*>(a.gamma + b * QK_K)[lane];
        v[0] = (v[0] * rms) * gv.x;
        v[1] = (v[1] * rms) * gv.y;
        v[2] = (v[2] * rms) * gv.z;
        v[3] = (v[3] * rms) * gv.w;
      }
      uint32_t packed;
      float d;
      int gsum;
      quant_block_wave(v, away, packed, d, gsum);
      sm.xq[b * 64 + xq_slot(lane)] = packed;
      if ((lane & 3) == 0) sm.bsum[b * 16 + (lane >> 2)] = gsum;
      if (lane == 0) sm.xd[b] = d;
    }
  }
  __syncthreads();

  const int s = lane >> 3, m = lane & 7;
  const int ngroups = a.pair ? (a.total_rows + 3) / 4 : (a.total_rows + ROWS_PER_GROUP - 1) / ROWS_PER_GROUP;
  float best_v = -__builtin_inff();
  int best_i = 0x7fffffff;

  for (int g = blockIdx.x; g < ngroups; g += gridDim.x) {
    int reg, r;
    bool valid;
    resolve_slot(a, g, s, reg, r, valid);
    const WView w = a.reg[reg].w;
    const bool is_q4 = (w.type == MCPM_TYPE_Q4_K);

    // ---- integer lanes: wave `wave` takes block columns wave, wave+4, ...
    for (int b = wave; b < nb; b += 4) {
      int isum = 0, minp = 0;
      float ds = 0.0f, dm = 0.0f;
      if (valid) {
        const size_t blk = static_cast<size_t>(b) * w.rows + r;
        const uint32_t* xl = &sm.xq[b * 64 + m * 8];
        const int* bs = &sm.bsum[b * 16];
        if (is_q4) {
          const u32x4 q = ld_stream4(w.p0 + blk * 128 + m * 16);
          const u32x4 meta = ld_stream4(w.p1 + blk * 16);
          q4k_lane(q, meta, xl, bs, m, isum, minp);
          ds = sm.xd[b] * fp16_to_fp32(static_cast<uint16_t>(meta.x & 0xffffu));
          dm = sm.xd[b] * fp16_to_fp32(static_cast<uint16_t>(meta.x >> 16));
        } else {
          const u32x4 ql = ld_stream4(w.p0 + blk * 128 + m * 16);
          const u32x2 qh = ld_stream2(w.p1 + blk * 64 + m * 8);
          const u32x4 scw = ld_stream4(w.p2 + blk * 16);
          const uint16_t dw = ld_stream_u16(w.p3 + blk * 2);
          isum = q6k_lane(ql, qh, scw, xl, bs, m);
          ds = sm.xd[b] * fp16_to_fp32(dw);
        }
      }
      sm.isum[b * 64 + lane] = isum;
      minp += __shfl_xor(minp, 1);
      minp += __shfl_xor(minp, 2);
      minp += __shfl_xor(minp, 4);
      if (m == 0) {
        sm.minsum[b * 8 + s] = minp;
        sm.ds[b * 8 + s] = ds;
        sm.dm[b * 8 + s] = dm;
      }
    }
    __syncthreads();

    // ---- float chain per (row, lane), blocks in order, then the lane tree
    if (wave == 0) {
      float acc = 0.0f, accm = 0.0f;
      for (int b = 0; b < nb; ++b) {
        acc = __builtin_fmaf(sm.ds[b * 8 + s], static_cast<float>(sm.isum[b * 64 + lane]), acc);
        accm = __builtin_fmaf(-sm.dm[b * 8 + s], static_cast<float>(sm.minsum[b * 8 + s]), accm);
      }
      float v = acc + __shfl_down(acc, 4);
      v = v + __shfl_down(v, 2);
      v = v + __shfl_down(v, 1);
      if (is_q4) v = v + accm;

      if constexpr (EPI == EPI_STORE) {
        if (m == 0 && valid) a.reg[reg].out[r] = v;
      } else if constexpr (EPI == EPI_RESID) {
        if (m == 0 && valid) a.resid[r] = a.resid[r] + v;
      } else if constexpr (EPI == EPI_SWIGLU) {
        const float u = __shfl(v, (s + 4) * 8);
        if (m == 0 && s < 4 && valid) {
          const float silu = v / (1.0f + exp_f32(-v));
          a.h_out[r] = silu * u;
        }
      } else if constexpr (EPI == EPI_QKV) {
        // adjacent-pair RoPE (src/ops/ops.cpp:502-516) for q (reg 0) and k
        // (reg 1); k and v rows go to the KV cache at pos.
        const float partner = __shfl(v, (s ^ 1) * 8);
        if (m == 0 && valid) {
          const int pos = a.state[1];
          if (reg < 2) {
            const int i = r % a.head_dim;
            const float2 cs = a.rope_cs[static_cast<size_t>(pos) * (a.head_dim / 2) + (i >> 1)];
            float o;
            if ((i & 1) == 0) o = v * cs.x - partner * cs.y;
            else o = partner * cs.y + v * cs.x;
            if (reg == 0) a.reg[0].out[r] = o;
            else a.k_cache[static_cast<size_t>(pos) * a.kvd + r] = o;
          } else {
            a.v_cache[static_cast<size_t>(pos) * a.kvd + r] = v;
          }
        }
      } else if constexpr (EPI == EPI_LOGITS) {
        if (m == 0 && valid) {
          a.reg[0].out[r] = v;
          if (v > best_v || (v == best_v && r < best_i)) {
            best_v = v;
            best_i = r;
          }
        }
      }
    }
    __syncthreads();
  }

  if constexpr (EPI == EPI_LOGITS) {
    if (wave == 0) {
      // first index of the maximum over the WG's rows
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best_v, o);
        const int oi = __shfl_xor(best_i, o);
        if (ov > best_v || (ov == best_v && oi < best_i)) {
          best_v = ov;
          best_i = oi;
        }
      }
      if (lane == 0) a.argmax_part[blockIdx.x] = make_float2(best_v, __int_as_float(best_i));
    }
  }
}

int gemv_grid(const GemvArgs& a, int n_cu) {
  const int ngroups = a.pair ? (a.total_rows + 3) / 4 : (a.total_rows + ROWS_PER_GROUP - 1) / ROWS_PER_GROUP;
  const int cap = n_cu * 4;
  return ngroups < cap ? ngroups : cap;
}

#define MCPM_GEMV_CASE(P, E)                                                     \
  if (prologue == P && epilogue == E) {                                          \
    hipLaunchKernelGGL((k_gemv_q8k<P, E>), dim3(grid), dim3(GEMV_THREADS), 0, s, a); \
    return hipGetLastError();                                                    \
  }

hipError_t launch_gemv(const GemvArgs& a, int prologue, int epilogue, int n_cu, hipStream_t s) {
  const int grid = gemv_grid(a, n_cu);
  if (grid <= 0) return hipSuccess;
  MCPM_GEMV_CASE(PRO_Q8K, EPI_STORE)
  MCPM_GEMV_CASE(PRO_QUANT_EVEN, EPI_STORE)
  MCPM_GEMV_CASE(PRO_QUANT_EVEN, EPI_RESID)
  MCPM_GEMV_CASE(PRO_QUANT_AWAY, EPI_RESID)
  MCPM_GEMV_CASE(PRO_NORM_AWAY, EPI_QKV)
  MCPM_GEMV_CASE(PRO_NORM_AWAY, EPI_SWIGLU)
  MCPM_GEMV_CASE(PRO_NORM_EVEN, EPI_LOGITS)
  MCPM_GEMV_CASE(PRO_NORM_EVEN, EPI_STORE)
  return hipErrorInvalidValue;
}

// ------------------------------------------------------- standalone ops ----

// Q8_K blocks of an fp32 vector (optionally RMS-normalised) in native layout.
// mode: PRO_QUANT_EVEN / PRO_QUANT_AWAY / PRO_NORM_AWAY / PRO_NORM_EVEN.
__global__ void __launch_bounds__(256) k_quantize_q8k(const float* __restrict__ x, const float* __restrict__ gamma,
                                                      float eps, int dim, int mode, BlockQ8K* __restrict__ out) {
  __shared__ float red[260];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool norm = (mode == PRO_NORM_AWAY || mode == PRO_NORM_EVEN);
  const bool away = (mode == PRO_QUANT_AWAY || mode == PRO_NORM_AWAY);
  float rms = 1.0f;
  if (norm) rms = block_rms_scale(x, dim, eps, red);
  const int nb = dim / QK_K;
  for (int b = wave; b < nb; b += 4) {
    const float4 xv = reinterpret_cast<const float4*>(x + b * QK_K)[lane];
    float v[4] = {xv.x, xv.y, xv.z, xv.w};
    if (norm) {
      const float4 gv = reinterpret_cast<const float4*>(gamma + b * QK_K)[lane];
      v[0] = (v[0] * rms) * gv.x;
      v[1] = (v[1] * rms) * gv.y;
      v[2] = (v[2] * rms) * gv.z;
      v[3] = (v[3] * rms) * gv.w;
    }
    uint32_t packed;
    float d;
    int gsum;
    quant_block_wave(v, away, packed, d, gsum);
    reinterpret_cast<uint32_t*>(out[b].qs)[lane] = packed;
    if ((lane & 3) == 0) out[b].bsums[lane >> 2] = static_cast<int16_t>(gsum);
    if (lane == 0) out[b].d = d;
  }
}

hipError_t launch_quantize_q8k(const float* x, const float* gamma, float eps, int dim, int mode, BlockQ8K* out,
                               hipStream_t s) {
  hipLaunchKernelGGL(k_quantize_q8k, dim3(1), dim3(256), 0, s, x, gamma, eps, dim, mode, out);
  return hipGetLastError();
}

// rmsnorm (src/ops/ops.cpp:468-481): out = (x*rms)*w.
__global__ void __launch_bounds__(256) k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w, float eps,
                                                 int dim, float* __restrict__ out) {
  __shared__ float red[260];
  const float rms = block_rms_scale(x, dim, eps, red);
  for (int i = threadIdx.x; i < dim; i += 256) out[i] = (x[i] * rms) * w[i];
}

hipError_t launch_rmsnorm(const float* x, const float* w, float eps, int dim, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(256), 0, s, x, w, eps, dim, out);
  return hipGetLastError();
}

// swiglu_and_quantize_q8k (src/ops/ops.cpp:725-765): dim/256 blocks, lround.
__global__ void __launch_bounds__(256) k_swiglu_quant(const float* __restrict__ g, const float* __restrict__ u, int dim,
                                                      BlockQ8K* __restrict__ out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nb = dim / QK_K;
  for (int b = wave; b < nb; b += 4) {
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = b * QK_K + 4 * lane + k;
      const float gg = g[i];
      const float silu = gg / (1.0f + exp_f32(-gg));
      v[k] = silu * u[i];
    }
    uint32_t packed;
    float d;
    int gsum;
    quant_block_wave(v, true, packed, d, gsum);
    reinterpret_cast<uint32_t*>(out[b].qs)[lane] = packed;
    if ((lane & 3) == 0) out[b].bsums[lane >> 2] = static_cast<int16_t>(gsum);
    if (lane == 0) out[b].d = d;
  }
}

hipError_t launch_swiglu_quant(const float* g, const float* u, int dim, BlockQ8K* out, hipStream_t s) {
  hipLaunchKernelGGL(k_swiglu_quant, dim3(1), dim3(256), 0, s, g, u, dim, out);
  return hipGetLastError();
}

// apply_rope for every head with a host-built (cos, sin) row for pos.
__global__ void k_rope(float* __restrict__ vec, const float2* __restrict__ cs, int n_pairs, int half_hd) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n_pairs) return;
  const float2 c = cs[p % half_hd];
  const float v0 = vec[2 * p], v1 = vec[2 * p + 1];
  vec[2 * p] = v0 * c.x - v1 * c.y;
  vec[2 * p + 1] = v0 * c.y + v1 * c.x;
}

hipError_t launch_rope(float* vec, const float2* cs, int n_heads, int head_dim, hipStream_t s) {
  const int n_pairs = n_heads * head_dim / 2;
  hipLaunchKernelGGL(k_rope, dim3((n_pairs + 255) / 256), dim3(256), 0, s, vec, cs, n_pairs, head_dim / 2);
  return hipGetLastError();
}

__global__ void k_kv_append(const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ kc,
                            float* __restrict__ vc, const int* __restrict__ state, int kvd) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= kvd) return;
  const size_t pos = static_cast<size_t>(state[1]);
  kc[pos * kvd + i] = k[i];
  vc[pos * kvd + i] = v[i];
}

hipError_t launch_kv_append(const float* k, const float* v, float* kc, float* vc, const int* state, int kvd,
                            hipStream_t s) {
  hipLaunchKernelGGL(k_kv_append, dim3((kvd + 255) / 256), dim3(256), 0, s, k, v, kc, vc, state, kvd);
  return hipGetLastError();
}

// ------------------------------------------------------------- attention ---
// One wave per (kv head, chunk of ATTN_CHUNK positions); the group's query
// heads (n_heads / n_kv_heads, at most 8) share each K and V row.  Per head:
//   s_t = (fma chain over i of q_i*k_ti) * scale          (lane j = position)
//   m_c = max(-1e9, s_t); e_t = exp(s_t - m_c); z_c = tree over lanes
//   o_c[i] = fma chain over t of e_t*v_ti                  (lane i = dim)
// The last wave to finish a kv head combines its chunks in order:
//   m = max m_c; f_c = exp(m_c - m); Z = fma(z_c, f_c, Z); O_i = fma(o_c[i], f_c, O_i)
//   out_i = O_i / Z
// part layout: [n_heads][max_chunks][2 + head_dim] floats (m, z, o[]).
constexpr int ATTN_MAX_GROUP = 8;
constexpr int ATTN_MAX_HD = 128;

__global__ void __launch_bounds__(64) k_attention(const float* __restrict__ q, const float* __restrict__ kc,
                                                  const float* __restrict__ vc, const int* __restrict__ state,
                                                  int n_heads, int n_kv_heads, int head_dim, int max_chunks,
                                                  float* __restrict__ part, unsigned* __restrict__ counters,
                                                  float* __restrict__ out) {
  __shared__ float s_q[ATTN_MAX_GROUP * ATTN_MAX_HD];
  __shared__ float s_e[ATTN_MAX_GROUP * ATTN_CHUNK];
  __shared__ int s_last;
  const int kvh = blockIdx.x, c = blockIdx.y, lane = threadIdx.x;
  const int pos = state[1];
  const int T = pos + 1;
  const int nch = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
  if (c >= nch) return;
  const int group = n_heads / n_kv_heads;
  const int kvd = n_kv_heads * head_dim;
  const int stride = 2 + head_dim;
  const float scale = 1.0f / sqrtf(static_cast<float>(head_dim));

  for (int i = lane; i < group * head_dim; i += 64) s_q[i] = q[kvh * group * head_dim + i];
  __syncthreads();

  // scores: lane j <-> position t0 + j
  const int t = c * ATTN_CHUNK + lane;
  const bool present = t < T;
  float sc[ATTN_MAX_GROUP];
#pragma unroll
  for (int hh = 0; hh < ATTN_MAX_GROUP; ++hh) sc[hh] = 0.0f;
  if (present) {
    const float* kt = kc + static_cast<size_t>(t) * kvd + static_cast<size_t>(kvh) * head_dim;
    for (int i0 = 0; i0 < head_dim; i0 += 4) {
      const float4 k4 = *reinterpret_cast<const float4*>(kt + i0);
      const float kk[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int hh = 0; hh < ATTN_MAX_GROUP; ++hh)
          if (hh < group) sc[hh] = __builtin_fmaf(s_q[hh * head_dim + i0 + u], kk[u], sc[hh]);
      }
    }
  }
#pragma unroll
  for (int hh = 0; hh < ATTN_MAX_GROUP; ++hh) {
    if (hh >= group) break;
    const float sv = present ? sc[hh] * scale : -1e9f;
    const float mc = fmaxf(wave_max(sv), -1e9f);
    const float e = present ? exp_f32(sv - mc) : 0.0f;
    const float z = wave_tree_sum(e);
    s_e[hh * ATTN_CHUNK + lane] = e;
    if (lane == 0) {
      float* pp = part + (static_cast<size_t>(kvh * group + hh) * max_chunks + c) * stride;
      pp[0] = mc;
      pp[1] = z;
    }
  }
  __syncthreads();

  // weighted V: lane i <-> dim i (two passes when head_dim = 128)
  const int nt = min(ATTN_CHUNK, T - c * ATTN_CHUNK);
  for (int i = lane; i < head_dim; i += 64) {
    float o[ATTN_MAX_GROUP];
#pragma unroll
    for (int hh = 0; hh < ATTN_MAX_GROUP; ++hh) o[hh] = 0.0f;
    for (int j = 0; j < nt; ++j) {
      const float vv =
          vc[static_cast<size_t>(c * ATTN_CHUNK + j) * kvd + static_cast<size_t>(kvh) * head_dim + i];
#pragma unroll
      for (int hh = 0; hh < ATTN_MAX_GROUP; ++hh)
        if (hh < group) o[hh] = __builtin_fmaf(s_e[hh * ATTN_CHUNK + j], vv, o[hh]);
    }
#pragma unroll
    for (int hh = 0; hh < ATTN_MAX_GROUP; ++hh)
      if (hh < group) part[(static_cast<size_t>(kvh * group + hh) * max_chunks + c) * stride + 2 + i] = o[hh];
  }

  // the last chunk-wave of this kv head combines
  __threadfence();
  __syncthreads();
  if (lane == 0) {
    const unsigned prev = atomicAdd(&counters[kvh], 1u);
    s_last = (prev == static_cast<unsigned>(nch - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int hh = 0; hh < group; ++hh) {
    const int h = kvh * group + hh;
    const float* ph = part + static_cast<size_t>(h) * max_chunks * stride;
    float mx = ph[0];
    for (int cc = 1; cc < nch; ++cc) mx = fmaxf(mx, ph[cc * stride]);
    for (int i = lane; i < head_dim; i += 64) {
      float Z = 0.0f, O = 0.0f;
      for (int cc = 0; cc < nch; ++cc) {
        const float f = exp_f32(ph[cc * stride] - mx);
        Z = __builtin_fmaf(ph[cc * stride + 1], f, Z);
        O = __builtin_fmaf(ph[cc * stride + 2 + i], f, O);
      }
      out[h * head_dim + i] = O / Z;
    }
  }
  if (lane == 0) counters[kvh] = 0u;
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc, const int* state, int n_heads,
                            int n_kv_heads, int head_dim, int max_chunks, float* part, unsigned* counters,
                            float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_attention, dim3(n_kv_heads, max_chunks), dim3(64), 0, s, q, kc, vc, state, n_heads,
                     n_kv_heads, head_dim, max_chunks, part, counters, out);
  return hipGetLastError();
}

// ------------------------------------------------------------- dequant -----
// Value e (0..255) of block (b, r).  Q4_K: (d*sc)*q - dmin*mn; Q6_K:
// (d*sc)*(q-32); Q8_0 handled separately.  Same expressions as
// src/ops/ops.cpp:655-664 and :194-228.
__device__ __forceinline__ float dequant_value(const WView& w, int r, int b, int e) {
  const size_t blk = static_cast<size_t>(b) * w.rows + r;
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
    // native byte 32c + l sits in dword (c*8 + l/4) -> permuted (l/4)*4 + c
    const int dword = ((l >> 2) << 2) + c;
    const uint8_t qb = w.p0[blk * 128 + dword * 4 + (l & 3)];
    const int qv = hi ? (qb >> 4) : (qb & 0x0f);
    const float d1 = fp16_to_fp32(dh) * static_cast<float>(scv);
    const float m1 = fp16_to_fp32(mh) * static_cast<float>(mnv);
    return d1 * static_cast<float>(qv) - m1;
  } else {
    const int h = e / 128, rr = e % 128, g = rr / 32, l = rr % 32;
    const int qlbyte = 64 * h + 32 * (g & 1) + l;  // native ql index
    const int qld = qlbyte >> 2;                    // native dword j*8+m
    const int qlp = ((qld & 7) << 2) + (qld >> 3);  // permuted dword
    const uint8_t qlb = w.p0[blk * 128 + qlp * 4 + (qlbyte & 3)];
    const int qhbyte = 32 * h + l;
    const int qhd = qhbyte >> 2;
    const int qhp = ((qhd & 7) << 1) + (qhd >> 3);
    const uint8_t qhb = w.p1[blk * 64 + qhp * 4 + (qhbyte & 3)];
    const int lo = (g < 2) ? (qlb & 0x0f) : (qlb >> 4);
    const int qv = lo | (((qhb >> (2 * g)) & 3) << 4);
    const int8_t scv = static_cast<int8_t>(w.p2[blk * 16 + e / 16]);
    const uint16_t dh = w.p3[blk * 2] | (w.p3[blk * 2 + 1] << 8);
    return (fp16_to_fp32(dh) * static_cast<float>(scv)) * static_cast<float>(qv - 32);
  }
}

__global__ void k_dequant_rows(const WView w, int row0, int n_rows, int cols, float* __restrict__ out) {
  const int r = row0 + blockIdx.y;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < cols; i += gridDim.x * blockDim.x) {
    float v;
    if (w.type == MCPM_TYPE_Q8_0) {
      const size_t blk = static_cast<size_t>(i / QK8_0) * w.rows + r;
      const int8_t q = static_cast<int8_t>(w.p0[blk * 32 + i % QK8_0]);
      const uint16_t dh = w.p1[blk * 2] | (w.p1[blk * 2 + 1] << 8);
      v = fp16_to_fp32(dh) * static_cast<float>(q);
    } else if (w.type == MCPM_TYPE_F32) {
      v = reinterpret_cast<const float*>(w.p0)[static_cast<size_t>(r) * cols + i];
    } else {
      v = dequant_value(w, r, i / QK_K, i % QK_K);
    }
    out[static_cast<size_t>(blockIdx.y) * cols + i] = v;
  }
}

hipError_t launch_dequant_rows(const WView& w, int row0, int n_rows, int cols, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_dequant_rows, dim3((cols + 255) / 256, n_rows), dim3(256), 0, s, w, row0, n_rows, cols, out);
  return hipGetLastError();
}

// get_embedding: row `token` (from the step state) dequantized to x.
__global__ void k_embedding(const WView w, const int* __restrict__ state, int dim, float* __restrict__ out) {
  const int token = state[0];
  for (int i = threadIdx.x; i < dim; i += blockDim.x) out[i] = dequant_value(w, token, i / QK_K, i % QK_K);
}

hipError_t launch_embedding(const WView& w, const int* state, int dim, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_embedding, dim3(1), dim3(256), 0, s, w, state, dim, out);
  return hipGetLastError();
}

// ------------------------------------------------- fp32-activation GEMVs ----
// gemv_f32 (src/ops/ops.cpp:32-43): lane t sums w*x over c = t, t+64, ...
// (multiply then add), then the 64-lane pairwise tree.  One wave per row.
__global__ void __launch_bounds__(256) k_gemv_f32(const float* __restrict__ w, const float* __restrict__ x,
                                                  float* __restrict__ out, int rows, int cols) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float* wr = w + static_cast<size_t>(r) * cols;
  float p = 0.0f;
  for (int c = lane; c < cols; c += 64) p = p + wr[c] * x[c];
  p = wave_tree_sum(p);
  if (lane == 0) out[r] = p;
}

hipError_t launch_gemv_f32(const float* w, const float* x, float* out, int rows, int cols, hipStream_t s) {
  hipLaunchKernelGGL(k_gemv_f32, dim3((rows + 3) / 4), dim3(256), 0, s, w, x, out, rows, cols);
  return hipGetLastError();
}

// gemv_q8_0 (src/ops/ops.cpp:58-79): per block s = sum over i of float(q_i)*x_i
// (i ascending, multiply then add); row = row + s*d over blocks in order.
// One lane per row.
__global__ void __launch_bounds__(256) k_gemv_q8_0(const WView w, const float* __restrict__ x,
                                                   float* __restrict__ out, int rows, int cols) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int nb = cols / QK8_0;
  float row = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const size_t blk = static_cast<size_t>(b) * w.rows + r;
    const int8_t* q = reinterpret_cast<const int8_t*>(w.p0 + blk * 32);
    float s = 0.0f;
    for (int i = 0; i < QK8_0; ++i) s = s + static_cast<float>(q[i]) * x[b * QK8_0 + i];
    const uint16_t dh = w.p1[blk * 2] | (w.p1[blk * 2 + 1] << 8);
    row = row + s * fp16_to_fp32(dh);
  }
  out[r] = row;
}

hipError_t launch_gemv_q8_0(const WView& w, const float* x, float* out, int rows, int cols, hipStream_t s) {
  hipLaunchKernelGGL(k_gemv_q8_0, dim3((rows + 255) / 256), dim3(256), 0, s, w, x, out, rows, cols);
  return hipGetLastError();
}

// ------------------------------------------------------------- argmax ------
__global__ void __launch_bounds__(256) k_argmax_partial(const float* __restrict__ x, int n, float2* __restrict__ part) {
  __shared__ float sv[4];
  __shared__ int si[4];
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const float v = x[i];
    if (v > bv || (v == bv && i < bi)) {
      bv = v;
      bi = i;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; ++k)
      if (sv[k] > bv || (sv[k] == bv && si[k] < bi)) {
        bv = sv[k];
        bi = si[k];
      }
    part[blockIdx.x] = make_float2(bv, __int_as_float(bi));
  }
}

hipError_t launch_argmax_partial(const float* x, int n, float2* part, int nparts, hipStream_t s) {
  hipLaunchKernelGGL(k_argmax_partial, dim3(nparts), dim3(256), 0, s, x, n, part);
  return hipGetLastError();
}

// Reduces (value, index) partials to the first index of the maximum; writes
// it to out_token, and when a step state is given, feeds it back as the next
// input token, appends it to out_tokens and advances pos.
__global__ void __launch_bounds__(64) k_argmax_final(const float2* __restrict__ part, int nparts,
                                                     int* __restrict__ out_token, StepState* st,
                                                     int* __restrict__ out_tokens) {
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < nparts; i += 64) {
    const float v = part[i].x;
    const int idx = __float_as_int(part[i].y);
    if (v > bv || (v == bv && idx < bi)) {
      bv = v;
      bi = idx;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (threadIdx.x == 0) {
    if (out_token) *out_token = bi;
    if (st) {
      st->token = bi;
      st->pos = st->pos + 1;
      if (out_tokens && st->step < st->n_out) out_tokens[st->step] = bi;
      st->step = st->step + 1;
    }
  }
}

hipError_t launch_argmax_final(const float2* part, int nparts, int* out_token, StepState* st, int* out_tokens,
                               hipStream_t s) {
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(64), 0, s, part, nparts, out_token, st, out_tokens);
  return hipGetLastError();
}

__global__ void k_fill_f32(float* p, float v, size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

hipError_t launch_fill_f32(float* p, float v, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_f32, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, p, v, n);
  return hipGetLastError();
}

}  // namespace mcpm
