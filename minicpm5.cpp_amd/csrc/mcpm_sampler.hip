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

// One work group.  For a threshold (the cut's top_p, or the walk's r*C) the
// first block whose end sum reaches it, then the first position of that
// block whose running sum does; positions at or past `limit` do not count.
// Returns (thread 0) the position, or -1 when no position below limit does;
// `run` gets that position's running sum.  The block phase either scans the
// block sums in order (recording each block's end sum in rec[] when rec is
// given and the blocks fit) or, with nrec >= 0, looks the block up among the
// end sums a previous scan recorded: the same sums, so the same block.
constexpr int SMP_REC = 2048;  // block end sums k_smp_pick keeps (vocabularies up to 524,288)

template <bool FLOAT_CMP>
__device__ int smp_search(const uint32_t* __restrict__ key, const float* __restrict__ p, int n, int topp,
                          const double* __restrict__ bs, int nblk, double thr_d, float thr_f, int limit, double* sb,
                          float* sv, int* s_int, double* s_dbl, double& run, double* rec, int nrec) {
  const int tid = threadIdx.x;
  double off = 0.0;
  int found = -1;
  if (nrec >= 0) {
    // first recorded block whose end sum reaches the threshold
    int best = 0x7fffffff;
    for (int j = tid; j < nrec; j += SMP_B) {
      const double e = rec[j];
      const bool hit = FLOAT_CMP ? (static_cast<float>(e) >= thr_f) : (thr_d <= e);
      if (hit) {
        best = j;
        break;
      }
    }
    if (tid == 0) s_int[0] = 0x7fffffff;
    __syncthreads();
    if (best != 0x7fffffff) atomicMin(s_int, best);
    __syncthreads();
    found = s_int[0] == 0x7fffffff ? -1 : s_int[0];
    off = found > 0 ? rec[found - 1] : found == 0 ? 0.0 : rec[nrec - 1];
    __syncthreads();
  } else {
    // block search over the block sums (staged through LDS), thread 0
    const bool keep = rec && nblk <= SMP_REC;
    for (int b0 = 0; b0 < nblk && found < 0; b0 += SMP_B) {
      const int m = min(SMP_B, nblk - b0);
      __syncthreads();
      if (tid < m) sb[tid] = bs[b0 + tid];
      __syncthreads();
      if (tid == 0) {
        // the sums in order, read 8 at a time ahead of their adds (the adds
        // stay one chain: this position's sum is the previous one's plus it)
        // (the eight adds of a batch run unconditionally, then the first hit
        // among them is picked: past it nothing is used)
        for (int j0 = 0; j0 < m && found < 0; j0 += 8) {
          double c[8];
          double acc = off;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            acc = acc + sb[min(j0 + q, m - 1)];
            c[q] = acc;
          }
          const int nv = min(8, m - j0);
          int hq = 8;
#pragma unroll
          for (int q = 7; q >= 0; --q) {
            const bool hit = FLOAT_CMP ? (static_cast<float>(c[q]) >= thr_f) : (thr_d <= c[q]);
            if (q < nv && hit) hq = q;
          }
          if (keep) {
#pragma unroll
            for (int q = 0; q < 8; ++q)
              if (q < nv && q <= hq) rec[b0 + j0 + q] = c[q];
          }
          // the sum before the hit, or after the batch (selects: no indexed array)
          const int lim = min(hq, nv);
#pragma unroll
          for (int q = 0; q < 8; ++q)
            if (q < lim) off = c[q];
          if (hq < 8) found = b0 + j0 + hq;
        }
        s_int[0] = found;
      }
      __syncthreads();
      found = s_int[0];
    }
    if (tid == 0) s_dbl[0] = off;
    __syncthreads();
    off = s_dbl[0];
  }
  if (found < 0) {
    run = off;  // the total
    return -1;
  }
  // in-block running sum of block `found`
  const int k0 = found * SMP_B;
  const int cnt = min(SMP_B, min(n, limit) - k0);
  if (tid < cnt) sv[tid] = smp_val(key, p, topp, k0 + tid);
  __syncthreads();
  int pos = -1;
  double pre = 0.0;
  if (tid == 0) {
    for (int j0 = 0; j0 < cnt && pos < 0; j0 += 8) {
      double pr[8];
      double acc = pre;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        acc = acc + static_cast<double>(sv[min(j0 + q, cnt - 1)]);
        pr[q] = acc;
      }
      const int nv = min(8, cnt - j0);
      int hq = 8;
#pragma unroll
      for (int q = 7; q >= 0; --q) {
        const double c = off + pr[q];
        const bool hit = FLOAT_CMP ? (static_cast<float>(c) >= thr_f) : (thr_d <= c);
        if (q < nv && hit) hq = q;
      }
      if (hq < 8) pos = k0 + j0 + hq;
      const int last = hq < 8 ? hq : nv - 1;  // the hit's running sum, or the batch's last
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (q <= last) pre = pr[q];
    }
  }
  run = off + pre;
  return pos;
}

__global__ void __launch_bounds__(SMP_B) k_smp_pick(const uint32_t* __restrict__ key, const int* __restrict__ id,
                                                    const float* __restrict__ p, int n, const double* __restrict__ bs,
                                                    int nblk, int topp, float top_p, float r, int* __restrict__ out_token,
                                                    StepState* st, int* __restrict__ out_tokens) {
  __shared__ double sb[SMP_B];
  __shared__ float sv[SMP_B];
  __shared__ int s_int[2];
  __shared__ double s_dbl[1];
  __shared__ double rec[SMP_REC];  // block end sums of the cut's scan, for the walk's lookup
  // the cut: first position whose running sum, rounded to float, reaches top_p
  // (the scan records the end sums of the blocks it passes, up to the cut's)
  int cnt = n;
  double C = 0.0;
  if (topp) {
    const int k = smp_search<true>(key, p, n, topp, bs, nblk, 0.0, top_p, n, sb, sv, s_int, s_dbl, C, rec, -1);
    if (k >= 0) cnt = k + 1;  // else: every position, C = the total
  } else {
    (void)smp_search<true>(key, p, n, topp, bs, nblk, 0.0, __builtin_inff(), n, sb, sv, s_int, s_dbl, C, rec, -1);
  }
  // thread 0 holds cnt and C; the walk's threshold to every thread (after
  // every thread's last read of the search's broadcast slots)
  __syncthreads();
  if (threadIdx.x == 0) {
    s_int[0] = cnt;
    s_int[1] = cnt > 0 ? (cnt - 1) / SMP_B + 1 : 0;  // blocks the cut's scan recorded: through the cut's block
    s_dbl[0] = static_cast<double>(r) * C;
  }
  __syncthreads();
  cnt = s_int[0];
  const int nrec = nblk <= SMP_REC ? min(s_int[1], nblk) : -1;
  const double t = s_dbl[0];
  __syncthreads();
  // the walk: t = r*C < C, so its block is at or before the cut's, whose end
  // sums the scan recorded
  double run = 0.0;
  int k = smp_search<false>(key, p, n, topp, bs, nblk, t, 0.0f, cnt, sb, sv, s_int, s_dbl, run, rec, nrec);
  if (threadIdx.x == 0) {
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

hipError_t launch_sample(void* scratch, size_t scratch_bytes, const float* logits, int n, float temperature,
                         float top_p, float r, int* out_token, StepState* st, int* out_tokens, hipStream_t s) {
  if (n <= 0 || !logits || !scratch) return hipErrorInvalidValue;
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
