// mcpm_persist.h -- the decode layers of one token as one persistent launch
// (mcpm_persist.hip): its shape plan, shared by the engine (host) and the
// kernels.
#pragma once

#include <algorithm>
#include <cstring>
#include <initializer_list>

#include "mcpm_internal.h"

namespace mcpm {

// One weight matrix's rows of a work group inside a region of its slab (and
// of its LDS): byte offset in the region, rows allocated (the most any work
// group has; rows past a work group's own are zero) and ggml type.  Layout,
// nb blocks per row:
//   Q4_K  16-byte chunk c (0..7 quants, 8 header) of (block b, row i) at
//         ((b*9 + c)*R + i)*16
//   Q6_K  chunk c (0..7 ql, 8..11 qh, 12 scales) at ((b*13 + c)*R + i)*16,
//         then the fp16 d of (b, i) in the low half of dword b*R + i
// so that consecutive lanes on consecutive rows read consecutive 16 bytes.
struct PdSub {
  int off, R, type;
};

__host__ __device__ constexpr int pd_sub_bytes(int type, int R, int nb) {
  return type == MCPM_TYPE_Q4_K ? 144 * R * nb : 208 * R * nb + ((4 * R * nb + 15) & ~15);
}

constexpr int PD_XCDS = 8;     // work group b runs on XCD b % 8
constexpr int PD_NBX = 16;     // largest dim / 256
constexpr int PD_NBH = 32;     // largest ffn_pad / 256
constexpr int PD_NBQ = 9;      // largest n_heads * head_dim / 256
constexpr int PD_REC_BLK = 85; // records of one Q8_K block: d, 64 code dwords, 16 bsums, 4 bsum-pair words
constexpr int PD_REC_LINE = 16;  // records per 128-byte cache line
constexpr int PD_ATTN_LDS = ((ATTN_CHUNK * 68 + ATTN_CHUNK * 64 + 8 * 64 + 8 * ATTN_CHUNK) * 4 + 64 * 8 + 15) & ~15;

struct PdShape {
  int L, G, W;  // layers, work groups (one per CU), work groups per XCD
  int dim, nbx, qd, nbq, kvd, hd, group, gh, nkv, ffn, ffn_pad, nbh;
  int nq, nk;          // q rows, and k (= v) rows, of one work group
  int nh_max, np_max;  // rows of x and FFN pairs of a work group, at most
  float eps;
  PdSub sq, sk, sv, so, sg, su, sd;  // sub-regions: offsets within their region
  int reg_off[4], reg_sz[4];         // regions QKV, O, gate/up, down in a (layer, work group) slab and in LDS
  int wd_lds;                        // LDS bytes of the down region (the attention's staging shares it)
  int scr_off;                       // scratch region in LDS (bytes)
  // scratch, in dwords from scr_off: Q8_K activations (codes, d, bsum
  // pairs, bsums), the RMS tree, a union area (x staging / chain entries /
  // attention rows and combine), row values, own x and x after O, flags
  int s_xs, s_xd, s_xbp, s_xbs, s_red, s_u, s_vrow, s_ownx, s_ownx2, s_misc;
  int lds_bytes;
  int slab_stride;  // bytes per (layer, work group)
  int max_chunks;   // attention partial records per kv head
  int part_stride;  // record slots per chunk of partials: gh + 2*group in whole lines
};

// Per-layer pointers: norms and the weight planes (the slab builder's source).
struct PdLayer {
  const float* attn_norm;
  const float* ffn_norm;
  WView q, k, v, o, g, u, d;
};

// The launch's arguments (by value: pointers in kernel arguments are known to
// address global memory, so the kernel's accesses through them are global
// rather than flat, and none is loaded from memory).
struct PdArgs {
  PdShape s;
  const float* norms;     // [L][2][dim]: attention and FFN RMSNorm gains
  const uint8_t* slab;    // [L][G][slab_stride]
  float* kc;              // KV cache, [L][max_seq][kvd]
  float* vc;
  int max_seq;
  const float2* rope;     // [max_seq][hd/2] (cos, sin)
  const int* state;       // token, pos
  WView embd;
  // hand-off records (value bits, tag), 64-bit each
  uint64_t* rx;    // [dim]   x entering a layer
  uint64_t* rx2;   // [dim]   x after the O projection
  uint64_t* rh;    // [ffn]   SwiGLU output
  uint64_t* rqkv;  // [nkv][gh + 2*hd]  q of the head group, K and V rows at pos
  uint64_t* rpart; // [nkv][max_chunks][part_stride]  chunk partials o_c, m_c, z_c
  uint64_t* ratt;  // [nbq][PD_REC_BLK]  attention output as Q8_K blocks
  unsigned* epoch; // launch counter (tags), advanced by each launch
  unsigned* err;   // set when a wait passed spin_limit
  unsigned spin_limit;
  float* x_out;    // x after the last layer (plain stores, for the LM head)
  // 1 when every work group b runs on the XCD of work group b % 8 (checked
  // at set-up, and by each launch against xcc): the records read only on
  // their writer's XCD (a kv head's q/k/v rows, its chunks' partials) are
  // stored at workgroup scope and stay in that XCD's L2, where the readers'
  // agent-scope loads find them; 0: every record at agent scope
  int xcd_local;
  const int* xcc;  // [G] the XCD each work group ran on at set-up
};

// Rows of work group b.
struct PdRows {
  int hr0, nh;  // rows of x: O and down outputs, embedding values
  int fp0, np;  // FFN pairs (gate row, up row)
  int kvh, k;   // kv head (= XCD) and index within the XCD
  int qr0, kr0; // first q row, first k (and v) row
};

// FFN pairs of each of the 8 work groups b < 8 (index 0 in their XCDs, the
// owners of the first attention chunk): the fewest that leave every other
// work group at most np_max.  The owner of a context's only chunk finishes
// its head's attention and reaches O last; fewer gate/up rows leave it fewer
// weights to copy and less work before G's hand-off.
__host__ __device__ constexpr int pd_owner_pairs(const PdShape& s) {
  const int spare = s.ffn - s.np_max * (s.G - PD_XCDS);
  return spare <= 0 ? 0 : (spare + PD_XCDS - 1) / PD_XCDS;
}

__host__ __device__ inline PdRows pd_rows(const PdShape& s, int b) {
  PdRows r;
  r.hr0 = static_cast<int>((static_cast<int64_t>(b) * s.dim) / s.G);
  r.nh = static_cast<int>((static_cast<int64_t>(b + 1) * s.dim) / s.G) - r.hr0;
  const int p0 = pd_owner_pairs(s), rest = s.ffn - PD_XCDS * p0, g = s.G - PD_XCDS;
  if (b < PD_XCDS) {
    r.fp0 = b * p0;
    r.np = p0;
  } else {
    r.fp0 = PD_XCDS * p0 + static_cast<int>((static_cast<int64_t>(b - PD_XCDS) * rest) / g);
    r.np = PD_XCDS * p0 + static_cast<int>((static_cast<int64_t>(b + 1 - PD_XCDS) * rest) / g) - r.fp0;
  }
  r.kvh = b % PD_XCDS;
  r.k = b / PD_XCDS;
  r.qr0 = r.kvh * s.gh + r.k * s.nq;
  r.kr0 = r.kvh * s.hd + r.k * s.nk;
  return r;
}

// The gate and up sub-regions of work group b and the bytes of its gate/up
// region they fill: the plan's (np_max rows each, reg_sz[2]) or, on the
// first-chunk owners, rows for their own pairs only, so that their copy of
// the region is shorter.
struct PdGu {
  PdSub g, u;
  int bytes;
};

__host__ __device__ inline PdGu pd_gu(const PdShape& s, int b) {
  const int p0 = pd_owner_pairs(s);
  if (b < PD_XCDS && p0 < s.np_max) {
    const int gb = pd_sub_bytes(MCPM_TYPE_Q4_K, p0, s.nbx);
    return PdGu{PdSub{0, p0, MCPM_TYPE_Q4_K}, PdSub{gb, p0, MCPM_TYPE_Q4_K}, (2 * gb + 1023) / 1024 * 1024};
  }
  return PdGu{s.sg, s.su, s.reg_sz[2]};
}

// Where slab byte `off` (a multiple of 16) of work group b's layer slab comes
// from: tensor (0..6: q, k, v, o, gate, up, down; -1: padding, zeros) and
// either one 16-byte chunk of plane `plane` at byte src[0] (n = 1) or, for
// a Q6_K d array chunk, four fp16 d's of plane 3 at src[0..3] (n = 4;
// src[i] < 0: zero).  rows: the tensor's rows (its plane stride).
struct PdSrc {
  int tensor, plane, n;
  int64_t src[4];
};

__host__ __device__ inline PdSrc pd_slab_src(const PdShape& s, int b, int off, const int (&rows)[7]) {
  PdSrc out{-1, 0, 0, {-1, -1, -1, -1}};
  int r = 3;
  while (r > 0 && off < s.reg_off[r]) --r;
  const int o = off - s.reg_off[r];
  const PdRows me = pd_rows(s, b);
  PdSub sb[3];
  int tens[3], valid[3], row0[3], nsub, nb;
  if (r == 0) {
    sb[0] = s.sq; sb[1] = s.sk; sb[2] = s.sv;
    tens[0] = 0; tens[1] = 1; tens[2] = 2;
    valid[0] = s.nq; valid[1] = s.nk; valid[2] = s.nk;
    row0[0] = me.qr0; row0[1] = me.kr0; row0[2] = me.kr0;
    nsub = 3;
    nb = s.nbx;
  } else if (r == 1) {
    sb[0] = s.so; tens[0] = 3; valid[0] = me.nh; row0[0] = me.hr0;
    nsub = 1;
    nb = s.nbq;
  } else if (r == 2) {
    const PdGu gu = pd_gu(s, b);
    sb[0] = gu.g; sb[1] = gu.u;
    tens[0] = 4; tens[1] = 5;
    valid[0] = me.np; valid[1] = me.np;
    row0[0] = me.fp0; row0[1] = me.fp0;
    nsub = 2;
    nb = s.nbx;
  } else {
    sb[0] = s.sd; tens[0] = 6; valid[0] = me.nh; row0[0] = me.hr0;
    nsub = 1;
    nb = s.nbh;
  }
  for (int q = 0; q < nsub; ++q) {
    const int so = o - sb[q].off, R = sb[q].R;
    if (so < 0 || so >= pd_sub_bytes(sb[q].type, R, nb)) continue;
    const int64_t nrows = rows[tens[q]];
    const int kc = so / 16;
    if (sb[q].type == MCPM_TYPE_Q4_K) {
      const int row = kc % R, tt = kc / R, c = tt % 9, blk = tt / 9;
      if (row < valid[q]) {
        const int64_t gr = row0[q] + row;
        out.tensor = tens[q];
        out.n = 1;
        out.plane = c < 8 ? 0 : 1;
        out.src[0] = c < 8 ? ((static_cast<int64_t>(blk) * 8 + c) * nrows + gr) * 16 : (blk * nrows + gr) * 16;
      }
    } else if (kc < 13 * nb * R) {
      const int row = kc % R, tt = kc / R, c = tt % 13, blk = tt / 13;
      if (row < valid[q]) {
        const int64_t gr = row0[q] + row;
        out.tensor = tens[q];
        out.n = 1;
        out.plane = c < 8 ? 0 : c < 12 ? 1 : 2;
        out.src[0] = c < 8    ? ((static_cast<int64_t>(blk) * 8 + c) * nrows + gr) * 16
                     : c < 12 ? ((static_cast<int64_t>(blk) * 4 + (c - 8)) * nrows + gr) * 16
                              : (blk * nrows + gr) * 16;
      }
    } else {
      const int e0 = (kc - 13 * nb * R) * 4;
      out.tensor = tens[q];
      out.plane = 3;
      out.n = 4;
      for (int k = 0; k < 4; ++k) {
        const int e = e0 + k;
        if (e < nb * R) {
          const int blk = e / R, row = e % R;
          if (row < valid[q]) out.src[k] = (blk * nrows + row0[q] + row) * 2;
        }
      }
    }
  }
  return out;
}

// The plan for a model on n_cu CUs with a KV cache of max_seq positions and
// the given weight types; false (and *why) when the shape does not fit the
// persistent kernel: n_cu a multiple of 8, 8 kv heads of 64 (head h's rows
// and attention on XCD h), a head group of one Q8_K block (4 query heads),
// at most two attention chunks per work group, LDS within 160 KiB.
constexpr bool pd_plan(const mcpm_model_config& c, int n_cu, int max_seq, int tq, int tk, int tv, int to, int td,
                       PdShape& s, const char** why) {
  auto no = [&](const char* w) {
    if (why) *why = w;
    return false;
  };
  s = PdShape{};
  if (n_cu <= 0 || n_cu % PD_XCDS) return no("CU count not a multiple of 8");
  s.G = n_cu;
  s.W = n_cu / PD_XCDS;
  s.L = c.n_layers;
  s.dim = c.dim;
  s.nbx = c.dim / QK_K;
  s.hd = c.head_dim;
  s.nkv = c.n_kv_heads;
  s.group = c.n_kv_heads > 0 ? c.n_heads / c.n_kv_heads : 0;
  s.gh = s.group * s.hd;
  s.qd = c.n_heads * c.head_dim;
  s.nbq = s.qd / QK_K;
  s.kvd = s.nkv * s.hd;
  s.ffn = c.ffn;
  s.ffn_pad = c.ffn_pad;
  s.nbh = c.ffn_pad / QK_K;
  s.eps = c.eps;
  if (s.nkv != PD_XCDS || s.hd != 64) return no("needs 8 kv heads of 64");
  if (s.gh != QK_K) return no("head group not one Q8_K block");
  if (s.gh % (2 * s.W) || s.hd % (2 * s.W)) return no("head rows do not split into even runs per work group");
  if (c.dim % QK_K || s.nbx > PD_NBX || s.nbq > PD_NBQ || c.ffn_pad % QK_K || s.nbh > PD_NBH || c.ffn > c.ffn_pad)
    return no("dimensions outside the kernel's bounds");
  if (tq != MCPM_TYPE_Q4_K || tk != MCPM_TYPE_Q4_K) return no("q and k must be Q4_K");
  for (int ty : {tv, to, td})
    if (ty != MCPM_TYPE_Q4_K && ty != MCPM_TYPE_Q6_K) return no("weight type without a kernel");
  s.max_chunks = (max_seq + ATTN_CHUNK - 1) / ATTN_CHUNK;
  s.part_stride = (s.gh + 2 * s.group + PD_REC_LINE - 1) / PD_REC_LINE * PD_REC_LINE;
  if (s.max_chunks > 2 * s.W) return no("context longer than two chunks per work group");
  s.nq = s.gh / s.W;
  s.nk = s.hd / s.W;
  s.nh_max = (c.dim + s.G - 1) / s.G;
  s.np_max = (c.ffn + s.G - 1) / s.G;
  if (s.nq + 2 * s.nk > 64 || 2 * s.np_max > 64 || s.nh_max > 64) return no("too many rows per work group");
  auto sub = [](int off, int R, int type) { return PdSub{off, R, type}; };
  s.sq = sub(0, s.nq, tq);
  s.sk = sub(pd_sub_bytes(tq, s.nq, s.nbx), s.nk, tk);
  s.sv = sub(s.sk.off + pd_sub_bytes(tk, s.nk, s.nbx), s.nk, tv);
  const int qkv_bytes = s.sv.off + pd_sub_bytes(tv, s.nk, s.nbx);
  s.so = sub(0, s.nh_max, to);
  const int o_bytes = pd_sub_bytes(to, s.nh_max, s.nbq);
  s.sg = sub(0, s.np_max, MCPM_TYPE_Q4_K);
  s.su = sub(pd_sub_bytes(MCPM_TYPE_Q4_K, s.np_max, s.nbx), s.np_max, MCPM_TYPE_Q4_K);
  const int gu_bytes = 2 * pd_sub_bytes(MCPM_TYPE_Q4_K, s.np_max, s.nbx);
  s.sd = sub(0, s.nh_max, td);
  const int d_bytes = pd_sub_bytes(td, s.nh_max, s.nbh);
  const int kib = 1024;
  auto up = [&](int v) { return (v + kib - 1) / kib * kib; };
  s.reg_sz[0] = up(qkv_bytes);
  s.reg_sz[1] = up(o_bytes);
  s.reg_sz[2] = up(gu_bytes);
  s.reg_sz[3] = up(d_bytes);
  s.reg_off[0] = 0;
  for (int r = 1; r < 4; ++r) s.reg_off[r] = s.reg_off[r - 1] + s.reg_sz[r - 1];
  s.slab_stride = s.reg_off[3] + s.reg_sz[3];
  s.wd_lds = std::max(s.reg_sz[3], (PD_ATTN_LDS + 15) & ~15);
  s.scr_off = s.reg_off[3] + s.wd_lds;
  // scratch (dwords)
  const int nbm = std::max({s.nbx, s.nbq, s.nbh});
  auto a4 = [](int v) { return (v + 3) & ~3; };
  s.s_xs = 0;
  s.s_xd = nbm * 68;
  s.s_xbp = s.s_xd + a4(nbm);
  s.s_xbs = s.s_xbp + nbm * 4;
  s.s_red = s.s_xbs + nbm * 16;
  s.s_u = a4(s.s_red + 260);
  const int rq = s.nq + 2 * s.nk;
  // the attention's rows at pos, combined output, own o_c, every chunk's
  // (m_c, z_c)
  const int attn_words = 2 * s.hd + 3 * s.gh + 2 * 64 * ATTN_MAX_GROUP;
  // the down phase stages its hand-off in rounds of up to 16 blocks
  const int u_words = std::max({c.dim, rq * s.nbx * 12, s.nh_max * s.nbq * 12, 2 * s.np_max * s.nbx * 12,
                                s.nh_max * s.nbh * 12, attn_words, std::min(s.nbh, 16) * QK_K});
  s.s_vrow = a4(s.s_u + u_words);
  const int rmax = std::max({rq, s.nh_max, 2 * s.np_max});
  s.s_ownx = a4(s.s_vrow + rmax);
  s.s_ownx2 = a4(s.s_ownx + s.nh_max);
  s.s_misc = a4(s.s_ownx2 + s.nh_max);
  s.lds_bytes = s.scr_off + (s.s_misc + 24) * 4;  // abort flag, launch count, two vote sets, sub-region table
  if (s.lds_bytes > 160 * 1024 - 256) return no("LDS plan above 160 KiB");  // room for the runtime's own LDS words
  return true;
}

// The plan of the shape the launch has a compiled instance for, the
// 2.4B-shaped decoder (40 layers, hidden 2304, 32 query and 8 kv heads of 64,
// FFN 5760, Q4_K q/k/o/gate/up with Q6_K v and down, RMSNorm eps 1e-6) on 256
// CUs: that instance takes every field of the plan but the layer count and the
// chunk count as compile-time constants, which frees the registers and the
// instructions that reading them from the launch's arguments takes.
constexpr PdShape pd_fixed_plan() {
  mcpm_model_config c{};
  c.n_layers = 40;
  c.dim = 2304;
  c.n_heads = 32;
  c.n_kv_heads = 8;
  c.head_dim = 64;
  c.ffn = 5760;
  c.ffn_pad = 5888;
  c.eps = 1e-6f;
  PdShape s{};
  pd_plan(c, 256, 4096, MCPM_TYPE_Q4_K, MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K, MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K, s, nullptr);
  return s;
}

// True when s is pd_fixed_plan() in every field but the layer count and the
// chunk count (the plans hold ints and one float, no padding).
inline bool pd_fixed_shape(const PdShape& s) {
  PdShape f = pd_fixed_plan(), c = s;
  c.L = f.L;
  c.max_chunks = f.max_chunks;
  return std::memcmp(&c, &f, sizeof f) == 0;
}
// Copies every layer's weights into the slab layout (device gather).
hipError_t launch_build_slab(const PdShape& s, const PdLayer* d_layers, uint8_t* slab, hipStream_t st);
// Record buffer sizes (records) for the shape, every array starting on a
// cache line.
size_t pd_records(const PdShape& s);
// Points the record arrays of a at one allocation of pd_records(s) records.
void pd_bind_records(PdArgs& a, uint64_t* base);
// Writes the XCD that work group b of a G-wide launch runs on to xcc[b];
// same = every b on the XCD of b % 8.
hipError_t pd_probe_xcd(int G, int* xcc, hipStream_t st, bool& same);
// The launch's LDS attribute and the check that one work group fits a CU
// (outside any graph capture); then the launch.
hipError_t prepare_decode_persist(const PdShape& s);
hipError_t launch_decode_persist(const PdArgs& a, hipStream_t st);

}  // namespace mcpm
