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
// then, with a top-p cut up to 0.998 (every running sum up to the cut is
// exact, so no order of addition matters; see k_smp_prob_hist):
//   k_smp_prob_hist  p, sort keys ~bits(p) and each key bucket's mass
//   k_smp_seg        bucket masses as prefix sums per segment of 256
//   k_smp_gather<0>, k_smp_resolve<0>  the cut's bucket, then the cut within it
//   k_smp_gather<1>, k_smp_resolve<1>  the draw's bucket, then the draw;
//                    writes the token and advances the step state
// otherwise:
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

// The uniform draw: draws[st->step] when the draws are in device memory (a
// captured token graph, one draw per generated token), else the argument.
__device__ __forceinline__ float smp_draw(float r, const float* __restrict__ draws, const StepState* st) {
  return draws ? draws[min(max(st->step, 0), st->n_out - 1)] : r;
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

// the sum of the block sums, in order, by thread 0 (block sums staged in LDS,
// zero-padded to a multiple of 16: adding +0.0 to a sum of non-negative
// terms leaves it unchanged).  The chain reads 16 sums ahead, then runs 16
// dependent adds.
__device__ __forceinline__ double smp_total(const double* __restrict__ bs, int nblk, double* sb) {
  double t = 0.0;
  for (int b0 = 0; b0 < nblk; b0 += SMP_B) {
    const int m = min(SMP_B, nblk - b0);
    __syncthreads();
    sb[threadIdx.x] = static_cast<int>(threadIdx.x) < m ? bs[b0 + threadIdx.x] : 0.0;
    __syncthreads();
    if (threadIdx.x == 0) {
      const int m16 = (m + 15) & ~15;
#pragma unroll 1
      for (int k = 0; k < m16; k += 16) {
        double2 v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = *reinterpret_cast<const double2*>(sb + k + 2 * q);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          t = t + v[q].x;
          t = t + v[q].y;
        }
      }
    }
  }
  return t;  // thread 0's value
}

__global__ void __launch_bounds__(SMP_B) k_smp_prob(const float* __restrict__ e, int n, const double* __restrict__ bs,
                                                    int nblk, int topp, uint32_t* __restrict__ key,
                                                    int* __restrict__ id, float* __restrict__ p) {
  __shared__ __attribute__((aligned(16))) double sb[SMP_B];
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
                                                    StepState* st, int* __restrict__ out_tokens,
                                                    const float* __restrict__ draws) {
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
  const double t = static_cast<double>(smp_draw(r, draws, st)) * C;
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

// ---------------------------------------------- top-p without the sort ----
// When every p up to the cut is a multiple of 2^-52 (p >= 2^-29 or 0), every
// running sum of the sampler is exact in double (all partial sums are below
// 2 and multiples of 2^-52), so the blocked sums equal the exact sums of the
// largest p in (p desc, id asc) order, whatever order they are added in.
// Elements below 2^-29 hold at most n * 2^-29 <= 2^-10 of the mass for n <=
// 524,288, so with top_p <= 0.998 (sum of p within 2^-23 of 1) the cut is
// reached before any of them.  Then the cut and the draw's position need no
// sort: masses as integers in units of 2^-52 (exact), summed per bucket of
// the sort key's top 16 bits, locate the buckets of the cut and the draw; a
// descent over the 8-bit digits of (key, id) within the gathered buckets
// finds the element at which the exact running sum first passes each test.
constexpr float SMP_HIST_TOPP = 0.998f;
constexpr int SMP_NBKT = 65536;  // buckets: key >> 16
constexpr int SMP_HCOPY = 8;     // copies of the bucket masses (one per XCD of the adding work group)
constexpr int SMP_HWG = 1024;    // elements per work group of the histogram pass (256 per wave)
constexpr int SMP_WTAB = 512;    // LDS hash slots per wave (> 256: never full)
constexpr uint32_t SMP_EMPTY = 0xffffffffu;

struct SmpMeta {
  unsigned int count;          // gathered elements
  unsigned int pad;
  unsigned long long base;     // mass of the buckets before the gathered one
  unsigned long long c_mass;   // the cut's running sum (units of 2^-52)
  uint2 cut;                   // the cut's element (key, id)
};

// p in units of 2^-52 (exact for p >= 2^-29; smaller ones truncated, they
// come after the cut)
__device__ __forceinline__ unsigned long long smp_fixed(float p) {
  const uint32_t b = __float_as_uint(p);
  const int ex = static_cast<int>((b >> 23) & 0xffu);
  if (ex == 0) return 0ull;
  const unsigned long long m = (b & 0x7fffffu) | 0x800000u;
  const int sh = min(ex - 98, 40);  // p * 2^52 = m * 2^(ex - 150 + 52)
  return sh >= 0 ? (m << sh) : (sh > -32 ? (m >> -sh) : 0ull);
}
__device__ __forceinline__ double smp_mass(unsigned long long m) { return static_cast<double>(m) * 0x1p-52; }

// p = e / s and its sort key (as k_smp_prob), and the masses summed per
// bucket: first in an LDS hash per wave, then one global atomic per bucket
// and wave, into the copy of the work group's XCD.
__global__ void __launch_bounds__(SMP_B) k_smp_prob_hist(const float* __restrict__ e, int n,
                                                         const double* __restrict__ bs, int nblk,
                                                         uint32_t* __restrict__ key, unsigned long long* __restrict__ hm) {
  __shared__ __attribute__((aligned(16))) double sb[SMP_B];
  __shared__ float s_sum;
  __shared__ uint32_t tk[4][SMP_WTAB];
  __shared__ unsigned long long tm[4][SMP_WTAB];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const double t = smp_total(bs, nblk, sb);
  if (tid == 0) s_sum = static_cast<float>(t);
  for (int i = lane; i < SMP_WTAB; i += 64) {
    tk[wave][i] = SMP_EMPTY;
    tm[wave][i] = 0ull;
  }
  __syncthreads();
  const float sv = s_sum;
  uint32_t* wk = tk[wave];
  unsigned long long* wm = tm[wave];
#pragma unroll
  for (int k = 0; k < SMP_HWG / SMP_B; ++k) {
    // the wave takes 64 consecutive elements per round
    const int i = static_cast<int>(blockIdx.x) * SMP_HWG + wave * (SMP_HWG / 4) + k * 64 + lane;
    if (i < n) {
      const float pv = e[i] / sv;
      const uint32_t kv = ~__float_as_uint(pv);
      key[i] = kv;
      const uint32_t bk = kv >> 16;
      uint32_t h = (bk * 2654435761u) >> 23;  // 9 bits
      for (;;) {
        const uint32_t prev = atomicCAS(&wk[h], SMP_EMPTY, bk);
        if (prev == SMP_EMPTY || prev == bk) break;
        h = (h + 1) & (SMP_WTAB - 1);
      }
      atomicAdd(&wm[h], smp_fixed(pv));
    }
  }
  __syncthreads();
  unsigned long long* hc = hm + static_cast<size_t>(blockIdx.x & (SMP_HCOPY - 1)) * SMP_NBKT;
  for (int i = lane; i < SMP_WTAB; i += 64)
    if (wk[i] != SMP_EMPTY && wm[i] != 0ull) atomicAdd(&hc[wk[i]], wm[i]);
}

// Block inclusive scan of one value per thread (256 threads), in LDS.
__device__ __forceinline__ unsigned long long smp_scan256(unsigned long long v, unsigned long long* sc) {
  const int tid = threadIdx.x;
  sc[tid] = v;
  __syncthreads();
#pragma unroll
  for (int d = 1; d < SMP_B; d <<= 1) {
    const unsigned long long a = tid >= d ? sc[tid - d] : 0ull;
    __syncthreads();
    sc[tid] += a;
    __syncthreads();
  }
  return sc[tid];
}

// Work group g of 256: the masses of buckets 256g .. 256g+255 (summed over
// the copies) as prefix sums within the segment (pfx) and the segment's
// total (seg); the copies are cleared for the next call.
__global__ void __launch_bounds__(SMP_B) k_smp_seg(unsigned long long* __restrict__ hm,
                                                   unsigned long long* __restrict__ pfx,
                                                   unsigned long long* __restrict__ seg) {
  __shared__ unsigned long long sc[SMP_B];
  const int b = static_cast<int>(blockIdx.x) * SMP_B + threadIdx.x;
  unsigned long long v = 0ull;
#pragma unroll
  for (int c = 0; c < SMP_HCOPY; ++c) {
    unsigned long long* p = hm + static_cast<size_t>(c) * SMP_NBKT + b;
    v += *p;
    *p = 0ull;
  }
  const unsigned long long cs = smp_scan256(v, sc);
  pfx[b] = cs;
  if (threadIdx.x == SMP_B - 1) seg[blockIdx.x] = cs;
}

// The first bucket whose cumulative mass M passes test(M) (every thread;
// barriers inside); *before gets the mass of the buckets before it.  -1 when
// none does.
template <class Test>
__device__ __forceinline__ int smp_bucket(const unsigned long long* __restrict__ pfx,
                                          const unsigned long long* segc, Test test, unsigned long long* before,
                                          int* s_hit) {
  const int tid = threadIdx.x;
  __syncthreads();
  if (tid == 0) *s_hit = 0x7fffffff;
  __syncthreads();
  if (test(segc[tid])) atomicMin(s_hit, tid);
  __syncthreads();
  const int sg = *s_hit;
  if (sg == 0x7fffffff) return -1;
  const unsigned long long off = sg > 0 ? segc[sg - 1] : 0ull;
  const unsigned long long v = pfx[sg * SMP_B + tid];
  __syncthreads();
  if (tid == 0) *s_hit = 0x7fffffff;
  __syncthreads();
  if (test(off + v)) atomicMin(s_hit, tid);
  __syncthreads();
  const int j = *s_hit;
  const int b = sg * SMP_B + (j == 0x7fffffff ? SMP_B - 1 : j);
  // mass before bucket b: the segment's offset plus the prefix of the bucket before it
  *before = off + (j > 0 && j != 0x7fffffff ? pfx[sg * SMP_B + j - 1] : 0ull);
  return b;
}

// Segment totals as a prefix, in LDS (every thread calls).
__device__ __forceinline__ void smp_seg_prefix(const unsigned long long* __restrict__ seg, unsigned long long* segc,
                                               unsigned long long* sc) {
  const unsigned long long c = smp_scan256(seg[threadIdx.x], sc);
  segc[threadIdx.x] = c;
  __syncthreads();
}

// Every work group alike finds one bucket -- WALK 0: the cut's (the first
// whose cumulative mass, rounded to float, reaches top_p); WALK 1: the
// draw's (the first whose cumulative mass reaches t = r * C, C the cut's
// running sum from the first resolve) -- and appends its elements to the
// list; work group 0 records the mass before it.
template <int WALK>
__global__ void __launch_bounds__(SMP_B) k_smp_gather(const uint32_t* __restrict__ key, int n,
                                                      const unsigned long long* __restrict__ pfx,
                                                      const unsigned long long* __restrict__ seg, float top_p, float r,
                                                      uint2* __restrict__ list, SmpMeta* __restrict__ meta,
                                                      const float* __restrict__ draws, const StepState* st) {
  __shared__ unsigned long long segc[SMP_B], sc[SMP_B];
  __shared__ int s_hit;
  __shared__ unsigned int s_cnt, s_base;
  smp_seg_prefix(seg, segc, sc);
  unsigned long long before = 0ull;
  int bk0;
  if constexpr (WALK) {
    // positions exist only in nonempty buckets: with t = 0 the draw is the
    // first element, in the first bucket of positive mass (the largest p is
    // at least 1/n)
    const double t = static_cast<double>(smp_draw(r, draws, st)) * smp_mass(meta->c_mass);
    bk0 = smp_bucket(pfx, segc, [&](unsigned long long m) { return m > 0ull && t <= smp_mass(m); }, &before, &s_hit);
  } else {
    bk0 = smp_bucket(pfx, segc, [&](unsigned long long m) { return static_cast<float>(smp_mass(m)) >= top_p; },
                     &before, &s_hit);
  }
  if (bk0 < 0) bk0 = SMP_NBKT;  // nothing passes (non-finite input): gather nothing
  if (blockIdx.x == 0 && threadIdx.x == 0) meta->base = before;
  const int i = static_cast<int>(blockIdx.x) * SMP_B + threadIdx.x;
  const uint32_t kv = i < n ? key[i] : 0xffffffffu;
  const bool in = i < n && static_cast<int>(kv >> 16) == bk0;
  if (threadIdx.x == 0) s_cnt = 0u;
  __syncthreads();
  unsigned int slot = 0u;
  if (in) slot = atomicAdd(&s_cnt, 1u);
  __syncthreads();
  if (threadIdx.x == 0 && s_cnt) s_base = atomicAdd(&meta->count, s_cnt);
  __syncthreads();
  // the count starts at zero and gathers at most n elements; the bound
  // keeps a corrupted count from writing past the list
  if (in && s_base + slot < static_cast<unsigned int>(n)) list[s_base + slot] = make_uint2(kv, static_cast<uint32_t>(i));
}

// Digit lvl (2..6) of the composite (key, id) within one bucket (the key's
// top 16 bits are the bucket), most significant first: key bits 15..8, 7..0,
// then id bits 23..16, 15..8, 7..0.
__device__ __forceinline__ uint32_t smp_digit(uint2 kv, int lvl) {
  return lvl < 4 ? (kv.x >> (24 - 8 * lvl)) & 0xffu : (kv.y >> (16 - 8 * (lvl - 4))) & 0xffu;
}
__device__ __forceinline__ bool smp_le(uint2 a, uint2 b) { return a.x < b.x || (a.x == b.x && a.y <= b.y); }
__device__ __forceinline__ unsigned long long smp_elem_mass(uint2 kv) { return smp_fixed(__uint_as_float(~kv.x)); }

struct SmpDescent {
  unsigned long long hm[SMP_B];  // mass per digit
  unsigned int hc[SMP_B];        // elements per digit
  unsigned long long sc[SMP_B];  // scan
  unsigned int cnt;              // compacted candidates
  int hit;
  uint2 found;
};

// Among the candidates src[0..n0) of one bucket (element order: (key, id)
// ascending; with `limit`, only those <= lim), the first element at which
// base + the running mass passes test; returns it and, in *total, the
// running mass through it.  One digit per level: the masses per digit value,
// the first digit whose cumulative mass passes, then only that digit's
// candidates (copied to the other buffer when they are fewer).  found.y ==
// 0xffffffff when none passes.
template <class Test>
__device__ uint2 smp_descend(const uint2* src, unsigned int n0, uint2* buf0, uint2* buf1, unsigned long long base,
                             Test test, bool limit, uint2 lim, unsigned long long* total, SmpDescent& D) {
  const int tid = threadIdx.x;
  const uint2* cur = src;
  unsigned int n = n0;
  bool first = true;  // the limit applies while reading src
  int which = 0;
  for (int lvl = 2; lvl < 7; ++lvl) {
    __syncthreads();
    D.hm[tid] = 0ull;
    D.hc[tid] = 0u;
    if (tid == 0) {
      D.cnt = 0u;
      D.hit = 0x7fffffff;
    }
    __syncthreads();
    for (unsigned int i = tid; i < n; i += SMP_B) {
      const uint2 kv = cur[i];
      if (first && limit && !smp_le(kv, lim)) continue;
      const uint32_t d = smp_digit(kv, lvl);
      atomicAdd(&D.hm[d], smp_elem_mass(kv));
      atomicAdd(&D.hc[d], 1u);
    }
    __syncthreads();
    const unsigned long long c = smp_scan256(D.hm[tid], D.sc);
    if (D.hc[tid] > 0u && test(base + c)) atomicMin(&D.hit, tid);
    __syncthreads();
    const int d = D.hit;
    if (d == 0x7fffffff) return make_uint2(0u, 0xffffffffu);
    base += d > 0 ? D.sc[d - 1] : 0ull;
    const unsigned int nd = D.hc[d];
    if (nd == 1u || lvl == 6) {
      // the one element of digit d: the answer
      for (unsigned int i = tid; i < n; i += SMP_B) {
        const uint2 kv = cur[i];
        if (first && limit && !smp_le(kv, lim)) continue;
        if (smp_digit(kv, lvl) == static_cast<uint32_t>(d)) D.found = kv;
      }
      __syncthreads();
      const uint2 f = D.found;
      *total = base + smp_elem_mass(f);
      return f;
    }
    if (nd < n || first) {
      // keep digit d's candidates only (order within the buffer is free)
      uint2* dst = which ? buf1 : buf0;
      for (unsigned int i = tid; i < n; i += SMP_B) {
        const uint2 kv = cur[i];
        if (first && limit && !smp_le(kv, lim)) continue;
        if (smp_digit(kv, lvl) == static_cast<uint32_t>(d)) dst[atomicAdd(&D.cnt, 1u)] = kv;
      }
      __threadfence();
      __syncthreads();
      cur = dst;
      n = D.cnt;
      which ^= 1;
      first = false;
    }
  }
  return make_uint2(0u, 0xffffffffu);  // not reached: level 6 returns
}

// One work group over the gathered bucket.  WALK 0: the cut (the first
// position whose running sum, rounded to float, reaches top_p), recorded with
// its running sum C.  WALK 1: the draw (the first position up to the cut whose
// running sum reaches r * C); writes the token and advances the step state
// like the greedy argmax.  Each leaves the list empty for the next gather.
template <int WALK>
__global__ void __launch_bounds__(SMP_B) k_smp_resolve(const uint2* __restrict__ list, uint2* __restrict__ buf0,
                                                       uint2* __restrict__ buf1, SmpMeta* __restrict__ meta, int n_vocab,
                                                       float top_p, float r, int* __restrict__ out_token,
                                                       StepState* st, int* __restrict__ out_tokens,
                                                       const float* __restrict__ draws) {
  __shared__ SmpDescent D;
  const unsigned int n = min(meta->count, static_cast<unsigned int>(n_vocab));
  const unsigned long long base = meta->base;
  unsigned long long cum = 0ull;
  if constexpr (!WALK) {
    const uint2 cut = smp_descend(list, n, buf0, buf1, base,
                                  [&](unsigned long long m) { return static_cast<float>(smp_mass(m)) >= top_p; },
                                  false, make_uint2(0u, 0u), &cum, D);
    __syncthreads();
    if (threadIdx.x == 0) {
      meta->count = 0u;
      meta->cut = cut;
      meta->c_mass = cut.y == 0xffffffffu ? 0ull : cum;
    }
  } else {
    const uint2 cut = meta->cut;
    const double t = static_cast<double>(smp_draw(r, draws, st)) * smp_mass(meta->c_mass);
    uint2 w = smp_descend(list, n, buf0, buf1, base, [&](unsigned long long m) { return t <= smp_mass(m); }, true,
                          cut, &cum, D);
    if (w.y == 0xffffffffu) w = cut;  // the walk's fallback: the cut's position
    __syncthreads();
    if (threadIdx.x == 0) {
      // non-finite inputs can leave no position found: a token in range still
      const int tok = w.y < static_cast<uint32_t>(n_vocab) ? static_cast<int>(w.y) : 0;
      meta->count = 0u;
      if (out_token) *out_token = tok;
      if (st) {
        st->token = tok;
        st->pos = st->pos + 1;
        if (out_tokens && st->step < st->n_out) out_tokens[st->step] = tok;
        st->step = st->step + 1;
      }
    }
  }
}

// Scratch layout: first, at offsets that do not depend on n, the sort-free
// path's state that must read zero at every call (bucket masses, the gather
// count; zeroed with the buffer at allocation and left zero by each call),
// its segment prefixes and totals; then e, p, key, key2, id, id2 (n each),
// pmax (nblk floats), bs (nblk doubles), the gathered elements and two
// candidate buffers (n each), the sort's scratch; every piece on a 256-byte
// boundary.
struct SmpLayout {
  size_t hm, pfx, seg, meta, e, p, key, key2, id, id2, pmax, bs, list, buf0, buf1, sort, end, sort_bytes;
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
  L.hm = take(static_cast<size_t>(SMP_HCOPY) * SMP_NBKT * 8);
  L.pfx = take(static_cast<size_t>(SMP_NBKT) * 8);
  L.seg = take(static_cast<size_t>(SMP_NBKT / SMP_B) * 8);
  L.meta = take(sizeof(SmpMeta));
  const size_t n4 = static_cast<size_t>(n) * 4;
  L.e = take(n4);
  L.p = take(n4);
  L.key = take(n4);
  L.key2 = take(n4);
  L.id = take(n4);
  L.id2 = take(n4);
  L.pmax = take(nblk * 4);
  L.bs = take(nblk * 8);
  L.list = take(static_cast<size_t>(n) * 8);
  L.buf0 = take(static_cast<size_t>(n) * 8);
  L.buf1 = take(static_cast<size_t>(n) * 8);
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
float sampler_sort_free_top_p() { return SMP_HIST_TOPP; }

hipError_t launch_sample(void* scratch, size_t scratch_bytes, const float* logits, int n, float temperature,
                         float top_p, float r, int* out_token, StepState* st, int* out_tokens, hipStream_t s,
                         const float* draws) {
  if (n <= 0 || n > SMP_REC * SMP_B || !logits || !scratch || (draws && !st)) return hipErrorInvalidValue;
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
  if (topp && top_p <= SMP_HIST_TOPP) {
    // exact masses: no sort (see k_smp_prob_hist)
    unsigned long long* hm = reinterpret_cast<unsigned long long*>(base + L.hm);
    unsigned long long* pfx = reinterpret_cast<unsigned long long*>(base + L.pfx);
    unsigned long long* seg = reinterpret_cast<unsigned long long*>(base + L.seg);
    SmpMeta* meta = reinterpret_cast<SmpMeta*>(base + L.meta);
    uint2* list = reinterpret_cast<uint2*>(base + L.list);
    uint2* buf0 = reinterpret_cast<uint2*>(base + L.buf0);
    uint2* buf1 = reinterpret_cast<uint2*>(base + L.buf1);
    hipLaunchKernelGGL(k_smp_prob_hist, dim3((n + SMP_HWG - 1) / SMP_HWG), dim3(SMP_B), 0, s, e, n, bs, nblk, key, hm);
    hipLaunchKernelGGL(k_smp_seg, dim3(SMP_NBKT / SMP_B), dim3(SMP_B), 0, s, hm, pfx, seg);
    hipLaunchKernelGGL(k_smp_gather<0>, dim3(nblk), dim3(SMP_B), 0, s, key, n, pfx, seg, top_p, r, list, meta,
                       draws, st);
    hipLaunchKernelGGL(k_smp_resolve<0>, dim3(1), dim3(SMP_B), 0, s, list, buf0, buf1, meta, n, top_p, r, out_token,
                       st, out_tokens, draws);
    hipLaunchKernelGGL(k_smp_gather<1>, dim3(nblk), dim3(SMP_B), 0, s, key, n, pfx, seg, top_p, r, list, meta,
                       draws, st);
    hipLaunchKernelGGL(k_smp_resolve<1>, dim3(1), dim3(SMP_B), 0, s, list, buf0, buf1, meta, n, top_p, r, out_token,
                       st, out_tokens, draws);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_smp_prob, dim3(nblk), dim3(SMP_B), 0, s, e, n, bs, nblk, topp, key, id, p);
  if (topp) {
    const hipError_t se = rocprim::radix_sort_pairs(sort_tmp, sort_bytes, key, key2, id, id2, n, 0, 32, s);
    if (se != hipSuccess) return se;
  }
  const uint32_t* kk = topp ? key2 : key;
  hipLaunchKernelGGL(k_smp_bsum, dim3(nblk), dim3(SMP_B), 0, s, kk, p, n, topp, bs);
  hipLaunchKernelGGL(k_smp_pick, dim3(1), dim3(SMP_B), 0, s, kk, id2, p, n, bs, nblk, topp, top_p, r, out_token, st,
                     out_tokens, draws);
  return hipGetLastError();
}

}  // namespace mcpm
