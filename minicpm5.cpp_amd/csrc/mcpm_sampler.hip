// mcpm_sampler.hip -- the temperature / top-p sampler on the device.
//
// Sampler::sample (src/sampler.cpp:8-73) step for step: temperature, softmax
// with the max subtracted, the (p desc, id asc) order when 0 < top_p < 1, the
// top-p cut, the walk over the running sum.  The reference's running sums are
// sequential in float; here every running sum is taken in double over blocks
// of SMP_B positions of its order -- in order within a block, the blocks in
// order, a position's running sum being the sum of the blocks before it plus
// its in-block running sum -- so the blocks are summed in parallel and only
// the block sums run in sequence.  The walk compares r*C (C = the running sum
// at the cut) with the running sum of p, the reference's comparison of r with
// the running sum of p/cum without the per-term division.  The difference
// from the reference is rounding only.
//
// Passes (n = vocab, nblk = ceil(n / SMP_B) work groups of SMP_B threads):
//   k_smp_max   scaled logits, the block's max
//   k_smp_exp   e = exp(v - max) (max over the block maxima), the block's
//               double sum of e in order
//   k_smp_prob  s = float(sum of the block sums in order), p = e / s; with a
//               top-p cut the sort keys ~bits(p) (ascending = p descending)
//   (radix sort of (key, id) pairs, stable: equal p keep ascending ids)
//   k_smp_bsum  the block's double sum of p in the walk's order
//   k_smp_pick  one work group: block search, then the in-block running sum,
//               for the cut and for the walk; writes the token and advances
//               the step state like the greedy argmax
#include <cstring>

#include <rocprim/device/device_radix_sort.hpp>

#include "mcpm_device.h"

namespace mcpm {

namespace {

constexpr int SMP_B = 256;


__device__ __forceinline__ float smp_logit(const float* __restrict__ logits, int i, float inv_temp, int apply) {
  const float l = logits[i];
  return apply ? l * inv_temp : l;
}

// the value at position k of the walk's order
__device__ __forceinline__ float smp_val(const uint32_t* __restrict__ key, const float* __restrict__ p, int topp,
                                         int k) {
  return topp ? __uint_as_float(~key[k]) : p[k];
}

__device__ __forceinline__ float block_max256(float v, float* red) {
  v = wave_max(v);
  const int tid = threadIdx.x;
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return v;
}

__global__ void __launch_bounds__(SMP_B) k_smp_max(const float* __restrict__ logits, int n, float inv_temp,
                                                   int apply, float* __restrict__ pmax) {
  __shared__ float red[4];
  const int i = blockIdx.x * SMP_B + threadIdx.x;
  const float v = i < n ? smp_logit(logits, i, inv_temp, apply) : -__builtin_inff();
  const float m = block_max256(v, red);
  if (threadIdx.x == 0) pmax[blockIdx.x] = m;
}

__global__ void __launch_bounds__(SMP_B) k_smp_exp(const float* __restrict__ logits, int n, float inv_temp, int apply,
                                                   const float* __restrict__ pmax, int nblk, float* __restrict__ e,
                                                   double* __restrict__ bs) {
  __shared__ float red[4];
  __shared__ float se[SMP_B];
  const int tid = threadIdx.x;
  float m = -1e9f;  // the reference's initial max
  for (int j = tid; j < nblk; j += SMP_B) m = fmaxf(m, pmax[j]);
  m = block_max256(m, red);
  const int i = blockIdx.x * SMP_B + tid;
  const float ev = i < n ? exp_f32(smp_logit(logits, i, inv_temp, apply) - m) : 0.0f;
  if (i < n) e[i] = ev;
  se[tid] = ev;
  __syncthreads();
  if (tid == 0) {
    const int cnt = min(SMP_B, n - static_cast<int>(blockIdx.x) * SMP_B);
    double s = 0.0;
    for (int k = 0; k < cnt; ++k) s = s + static_cast<double>(se[k]);
    bs[blockIdx.x] = s;
  }
}

// the sum of the block sums, in order, by thread 0 (block sums staged in LDS)
__device__ __forceinline__ double smp_total(const double* __restrict__ bs, int nblk, double* sb) {
  double t = 0.0;
  for (int b0 = 0; b0 < nblk; b0 += SMP_B) {
    const int m = min(SMP_B, nblk - b0);
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < m) sb[threadIdx.x] = bs[b0 + threadIdx.x];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int k = 0; k < m; ++k) t = t + sb[k];
  }
  return t;  // thread 0's value
}

__global__ void __launch_bounds__(SMP_B) k_smp_prob(const float* __restrict__ e, int n, const double* __restrict__ bs,
                                                    int nblk, int topp, uint32_t* __restrict__ key,
                                                    int* __restrict__ id, float* __restrict__ p) {
  __shared__ double sb[SMP_B];
  __shared__ float s_sum;
  const double t = smp_total(bs, nblk, sb);
  if (threadIdx.x == 0) s_sum = static_cast<float>(t);
  __syncthreads();
  const int i = blockIdx.x * SMP_B + threadIdx.x;
  if (i >= n) return;
  const float pv = e[i] / s_sum;
  if (topp) {
    key[i] = ~__float_as_uint(pv);
    id[i] = i;
  } else {
    p[i] = pv;
  }
}

__global__ void __launch_bounds__(SMP_B) k_smp_bsum(const uint32_t* __restrict__ key, const float* __restrict__ p,
                                                    int n, int topp, double* __restrict__ bs) {
  __shared__ float sv[SMP_B];
  const int tid = threadIdx.x;
  const int k = blockIdx.x * SMP_B + tid;
  sv[tid] = k < n ? smp_val(key, p, topp, k) : 0.0f;
  __syncthreads();
  if (tid == 0) {
    const int cnt = min(SMP_B, n - static_cast<int>(blockIdx.x) * SMP_B);
    double s = 0.0;
    for (int j = 0; j < cnt; ++j) s = s + static_cast<double>(sv[j]);
    bs[blockIdx.x] = s;
  }
}

// One work group: the cut and the walk.  Position k's running sum is the
// sum of the block sums before its block, added in order (P[j] = P[j-1] +
// bs[j], double, from 0), plus its in-block running sum (double, in order,
// from 0).  The sequential chains run on thread 0 into LDS; every search over
// them is parallel (first index whose sum reaches the threshold).
//   cut:  the first block j with float(P[j]) >= top_p, then the first
//         position of it whose float(P[j-1] + in-block sum) >= top_p; the
//         cut keeps positions up to that one, C = its running sum (no cut: C =
//         the total).
//   walk: t = r * C; the first block j at or before the cut's with t <= P[j],
//         then its first position before the cut with t <= P[j-1] + in-block
//         sum; none: the cut's last position.
constexpr int SMP_REC = 2048;  // blocks: vocabularies up to 524,288

// the first i < count with pred(i), or -1 (every thread; a barrier at entry
// and exit)
template <class Pred>
__device__ __forceinline__ int smp_first(int count, Pred pred, int* s_hit) {
  const int tid = threadIdx.x;
  __syncthreads();
  if (tid == 0) *s_hit = 0x7fffffff;
  __syncthreads();
  for (int i = tid; i < count; i += SMP_B) {
    if (pred(i)) {
      atomicMin(s_hit, i);
      break;
    }
  }
  __syncthreads();
  const int h = *s_hit;
  return h == 0x7fffffff ? -1 : h;
}

// in-block running sums of the block at k0 (cnt values, zeros past them)
// into pr[0..SMP_B), thread 0 in order, the values staged in sv (all threads
// call).  The chain is straight-line: 16 values read ahead, then 16
// dependent adds and their stores.
__device__ __forceinline__ void smp_block_prefix(const uint32_t* __restrict__ key, const float* __restrict__ p,
                                                 int topp, int k0, int cnt, float* sv, double* pr) {
  const int tid = threadIdx.x;
  __syncthreads();
  sv[tid] = tid < cnt ? smp_val(key, p, topp, k0 + tid) : 0.0f;
  __syncthreads();
  if (tid == 0) {
    double acc = 0.0;
#pragma unroll 1
    for (int j0 = 0; j0 < SMP_B; j0 += 16) {
      f32x4 v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const f32x4*>(sv + j0 + 4 * q);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const double a0 = acc + static_cast<double>(v[q].x);
        const double a1 = a0 + static_cast<double>(v[q].y);
        const double a2 = a1 + static_cast<double>(v[q].z);
        const double a3 = a2 + static_cast<double>(v[q].w);
        *reinterpret_cast<double2*>(pr + j0 + 4 * q) = double2{a0, a1};
        *reinterpret_cast<double2*>(pr + j0 + 4 * q + 2) = double2{a2, a3};
        acc = a3;
      }
    }
  }
  __syncthreads();
}

__global__ void __launch_bounds__(SMP_B) k_smp_pick(const uint32_t* __restrict__ key, const int* __restrict__ id,
                                                    const float* __restrict__ p, int n, const double* __restrict__ bs,
                                                    int nblk, int topp, float top_p, float r, int* __restrict__ out_token,
                                                    StepState* st, int* __restrict__ out_tokens) {
  __shared__ __attribute__((aligned(16))) double P[SMP_REC];  // inclusive block prefix sums (zero-padded)
  __shared__ __attribute__((aligned(16))) double pr[SMP_B];   // in-block running sums of one block
  __shared__ __attribute__((aligned(16))) float sv[SMP_B];
  __shared__ int s_hit;
  const int tid = threadIdx.x;
  const int nb16 = (nblk + 15) & ~15;  // <= SMP_REC (a multiple of 16)
  for (int j = tid; j < nb16; j += SMP_B) P[j] = j < nblk ? bs[j] : 0.0;
  __syncthreads();
  if (tid == 0) {
    // straight-line: 16 sums read ahead, then 16 dependent adds and stores
    double acc = 0.0;
#pragma unroll 1
    for (int j0 = 0; j0 < nb16; j0 += 16) {
      double2 v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = *reinterpret_cast<const double2*>(P + j0 + 2 * q);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const double a0 = acc + v[q].x;
        const double a1 = a0 + v[q].y;
        *reinterpret_cast<double2*>(P + j0 + 2 * q) = double2{a0, a1};
        acc = a1;
      }
    }
  }
  __syncthreads();
  int cnt = n;                // positions the walk may take
  double C = P[nblk - 1];     // the cut's running sum (no cut: the total)
  int pr_block = -1;          // the block whose running sums pr[] holds
  if (topp) {
    const int jc = smp_first(nblk, [&](int j) { return static_cast<float>(P[j]) >= top_p; }, &s_hit);
    if (jc >= 0) {
      const int k0 = jc * SMP_B, nb = min(SMP_B, n - k0);
      const double off = jc > 0 ? P[jc - 1] : 0.0;
      smp_block_prefix(key, p, topp, k0, nb, sv, pr);
      pr_block = jc;
      // the block's end sum reached top_p, and off + pr[nb-1] is that sum:
      // a position is found
      const int q = smp_first(nb, [&](int i) { return static_cast<float>(off + pr[i]) >= top_p; }, &s_hit);
      const int qq = q >= 0 ? q : nb - 1;
      cnt = k0 + qq + 1;
      C = off + pr[qq];
    }
  }
  const double t = static_cast<double>(r) * C;
  const int nrec = (cnt - 1) / SMP_B + 1;  // blocks through the cut's
  const int jw = smp_first(nrec, [&](int j) { return t <= P[j]; }, &s_hit);
  int k = -1;
  if (jw >= 0) {
    const int k0 = jw * SMP_B, nb = min(SMP_B, cnt - k0);
    const double off = jw > 0 ? P[jw - 1] : 0.0;
    if (jw != pr_block) smp_block_prefix(key, p, topp, k0, min(SMP_B, n - k0), sv, pr);
    const int q = smp_first(nb, [&](int i) { return t <= off + pr[i]; }, &s_hit);
    if (q >= 0) k = k0 + q;
  }
  if (tid == 0) {
    if (k < 0) k = cnt - 1;
    const int tok = topp ? id[k] : k;
    if (out_token) *out_token = tok;
    if (st) {
      st->token = tok;
      st->pos = st->pos + 1;
      if (out_tokens && st->step < st->n_out) out_tokens[st->step] = tok;
      st->step = st->step + 1;
    }
  }
}

// Scratch layout: e, p, key, key2, id, id2 (n each), pmax (nblk floats), bs
// (nblk doubles), the sort's scratch; every piece on a 256-byte boundary.
struct SmpLayout {
  size_t e, p, key, key2, id, id2, pmax, bs, sort, end, sort_bytes;
};

SmpLayout smp_layout(int n) {
  const size_t nblk = static_cast<size_t>((n + SMP_B - 1) / SMP_B);
  SmpLayout L{};
  size_t cur = 0;
  auto take = [&cur](size_t bytes) {
    const size_t at = cur;
    cur += (bytes + 255) & ~static_cast<size_t>(255);
    return at;
  };
  const size_t n4 = static_cast<size_t>(n) * 4;
  L.e = take(n4);
  L.p = take(n4);
  L.key = take(n4);
  L.key2 = take(n4);
  L.id = take(n4);
  L.id2 = take(n4);
  L.pmax = take(nblk * 4);
  L.bs = take(nblk * 8);
  (void)rocprim::radix_sort_pairs(nullptr, L.sort_bytes, static_cast<uint32_t*>(nullptr),
                                  static_cast<uint32_t*>(nullptr), static_cast<int*>(nullptr),
                                  static_cast<int*>(nullptr), n);
  L.sort = take(L.sort_bytes);
  L.end = cur;
  return L;
}

}  // namespace

size_t sampler_bytes(int n) { return n > 0 ? smp_layout(n).end : 0; }
int sampler_max_n() { return SMP_REC * SMP_B; }

hipError_t launch_sample(void* scratch, size_t scratch_bytes, const float* logits, int n, float temperature,
                         float top_p, float r, int* out_token, StepState* st, int* out_tokens, hipStream_t s) {
  if (n <= 0 || n > SMP_REC * SMP_B || !logits || !scratch) return hipErrorInvalidValue;
  const SmpLayout L = smp_layout(n);
  if (L.end > scratch_bytes) return hipErrorInvalidValue;
  const int nblk = (n + SMP_B - 1) / SMP_B;
  char* base = static_cast<char*>(scratch);
  float* e = reinterpret_cast<float*>(base + L.e);
  float* p = reinterpret_cast<float*>(base + L.p);
  uint32_t* key = reinterpret_cast<uint32_t*>(base + L.key);
  uint32_t* key2 = reinterpret_cast<uint32_t*>(base + L.key2);
  int* id = reinterpret_cast<int*>(base + L.id);
  int* id2 = reinterpret_cast<int*>(base + L.id2);
  float* pmax = reinterpret_cast<float*>(base + L.pmax);
  double* bs = reinterpret_cast<double*>(base + L.bs);
  void* sort_tmp = base + L.sort;
  size_t sort_bytes = L.sort_bytes;

  const float inv_temp = (temperature > 0.0f) ? (1.0f / temperature) : 1.0f;
  const int apply = (temperature != 1.0f && temperature > 0.0f) ? 1 : 0;
  const int topp = (top_p > 0.0f && top_p < 1.0f) ? 1 : 0;
  hipLaunchKernelGGL(k_smp_max, dim3(nblk), dim3(SMP_B), 0, s, logits, n, inv_temp, apply, pmax);
  hipLaunchKernelGGL(k_smp_exp, dim3(nblk), dim3(SMP_B), 0, s, logits, n, inv_temp, apply, pmax, nblk, e, bs);
  hipLaunchKernelGGL(k_smp_prob, dim3(nblk), dim3(SMP_B), 0, s, e, n, bs, nblk, topp, key, id, p);
  if (topp) {
    const hipError_t se = rocprim::radix_sort_pairs(sort_tmp, sort_bytes, key, key2, id, id2, n, 0, 32, s);
    if (se != hipSuccess) return se;
  }
  const uint32_t* kk = topp ? key2 : key;
  hipLaunchKernelGGL(k_smp_bsum, dim3(nblk), dim3(SMP_B), 0, s, kk, p, n, topp, bs);
  hipLaunchKernelGGL(k_smp_pick, dim3(1), dim3(SMP_B), 0, s, kk, id2, p, n, bs, nblk, topp, top_p, r, out_token, st,
                     out_tokens);
  return hipGetLastError();
}

}  // namespace mcpm
