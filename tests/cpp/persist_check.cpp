// Host-side check of the persistent decode kernel's plan and slab indexing
// (minicpm5.cpp_amd/csrc/mcpm_persist.{h,hip}), with no GPU: for each shape,
//  - the LDS plan: regions disjoint and in order, every phase's scratch use
//    (x staging, chain entries, attention rows) inside the union area, the
//    total within 160 KiB;
//  - the slab builder: for every work group and every 16-byte slab chunk,
//    the source (pd_slab_src, the builder's own code) lies inside its
//    plane, and every byte the kernel's lane-sum tasks read maps back to the
//    (row, block, chunk) of the weight it expects;
//  - the hand-offs: the row ranges of the work groups cover each consumer's
//    records exactly once, every record array starts on a cache line, and
//    the blocks stored at workgroup scope fill whole lines;
//  - shapes the kernel does not take are refused;
//  - the first-chunk owners' lighter FFN share (pd_owner_pairs);
//  - the plan the fixed-shape instance compiles in (pd_fixed_plan, evaluated
//    at compile time) equals the plan made at run time for that shape, and
//    pd_fixed_shape picks that instance for it at any layer count and KV
//    capacity the kernel takes, and for no other shape or weight type.
// Prints one line per shape; exit status 0 when every check holds.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "mcpm_persist.h"

using namespace mcpm;

static int failures = 0;
#define CHECK(cond, ...)                     \
  do {                                       \
    if (!(cond)) {                           \
      if (failures < 20) {                   \
        std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
        std::printf(__VA_ARGS__);            \
        std::printf("\n");                   \
      }                                      \
      ++failures;                            \
    }                                        \
  } while (0)

static mcpm_model_config cfg(int L, int dim, int nh, int nkv, int hd, int ffn) {
  mcpm_model_config c{};
  c.n_layers = L;
  c.dim = dim;
  c.n_heads = nh;
  c.n_kv_heads = nkv;
  c.head_dim = hd;
  c.ffn = ffn;
  c.ffn_pad = (ffn + 255) / 256 * 256;
  c.vocab = 1000;
  c.eps = 1e-6f;
  c.rope_base = 10000.0f;
  return c;
}

// bytes of plane p of a (rows x nb-block) tensor of the given type
static int64_t plane_bytes(int type, int64_t rows, int nb, int p) {
  if (type == MCPM_TYPE_Q4_K) return p == 0 ? nb * 8 * rows * 16 : p == 1 ? nb * rows * 16 : 0;
  return p == 0 ? nb * 8 * rows * 16 : p == 1 ? nb * 4 * rows * 16 : p == 2 ? nb * rows * 16 : nb * rows * 2;
}

static void check_shape(const char* name, const mcpm_model_config& c, int n_cu, int max_seq, int tv, int to, int td) {
  PdShape s{};
  const char* why = nullptr;
  const bool ok = pd_plan(c, n_cu, max_seq, MCPM_TYPE_Q4_K, MCPM_TYPE_Q4_K, tv, to, td, s, &why);
  CHECK(ok, "%s: plan refused (%s)", name, why ? why : "?");
  if (!ok) return;
  std::printf("%s: G=%d nq=%d nk=%d nh<=%d np<=%d regions %d/%d/%d/%d KiB slab %d B/WG/layer, LDS %d B\n", name, s.G,
              s.nq, s.nk, s.nh_max, s.np_max, s.reg_sz[0] >> 10, s.reg_sz[1] >> 10, s.reg_sz[2] >> 10,
              s.reg_sz[3] >> 10, s.slab_stride, s.lds_bytes);
  // LDS plan
  CHECK(s.reg_off[0] == 0, "%s: first region", name);
  for (int r = 1; r < 4; ++r) CHECK(s.reg_off[r] == s.reg_off[r - 1] + s.reg_sz[r - 1], "%s: region %d", name, r);
  for (int r = 0; r < 4; ++r) CHECK(s.reg_sz[r] % 1024 == 0 && s.reg_off[r] % 1024 == 0, "%s: region %d KiB", name, r);
  CHECK(s.wd_lds >= s.reg_sz[3] && s.wd_lds >= PD_ATTN_LDS, "%s: down/attention LDS", name);
  CHECK(s.scr_off == s.reg_off[3] + s.wd_lds && s.scr_off % 16 == 0, "%s: scratch offset", name);
  CHECK(s.lds_bytes == s.scr_off + (s.s_misc + 24) * 4 && s.lds_bytes <= 160 * 1024, "%s: LDS total", name);
  const int nbm = std::max(std::max(s.nbx, s.nbq), s.nbh);
  CHECK(s.s_xd >= s.s_xs + nbm * 68 && s.s_xbp >= s.s_xd + nbm && s.s_xbs >= s.s_xbp + 4 * nbm &&
            s.s_red >= s.s_xbs + 16 * nbm && s.s_u >= s.s_red + 256,
        "%s: activation areas", name);
  CHECK(s.s_xbp % 4 == 0 && s.s_xbs % 4 == 0 && s.s_u % 4 == 0, "%s: 16-byte alignment", name);
  const int u = s.s_vrow - s.s_u;
  const int rq = s.nq + 2 * s.nk;
  CHECK(u >= c.dim, "%s: x staging", name);
  CHECK(u >= std::min(s.nbh, 16) * 256, "%s: the down phase's hand-off staging (16 blocks a round)", name);
  CHECK(u >= rq * s.nbx * 12 && u >= s.nh_max * s.nbq * 12 && u >= 2 * s.np_max * s.nbx * 12 &&
            u >= s.nh_max * s.nbh * 12,
        "%s: chain entries", name);
  CHECK(u >= 2 * 64 + 3 * 256 + 2 * 64 * 8, "%s: attention rows and combine", name);
  CHECK(s.s_ownx - s.s_vrow >= std::max(rq, std::max(s.nh_max, 2 * s.np_max)), "%s: row values", name);
  CHECK(s.s_ownx2 - s.s_ownx >= s.nh_max && s.s_misc - s.s_ownx2 >= s.nh_max, "%s: own rows", name);
  CHECK(rq <= 64 && 2 * s.np_max <= 64 && s.nh_max <= 64, "%s: 4 lanes per chain row", name);
  CHECK(s.max_chunks <= 2 * s.W, "%s: chunks per work group", name);
  // rows: each consumer's records covered once
  std::vector<int> hx(c.dim, 0), fx(c.ffn, 0), qx(s.nkv * (s.gh + 2 * s.hd), 0);
  for (int b = 0; b < s.G; ++b) {
    const PdRows me = pd_rows(s, b);
    CHECK(me.nh <= s.nh_max && me.np <= s.np_max && me.nh >= 0 && me.np >= 0, "%s: rows of %d", name, b);
    for (int i = 0; i < me.nh; ++i) hx[me.hr0 + i]++;
    for (int i = 0; i < me.np; ++i) fx[me.fp0 + i]++;
    CHECK(me.qr0 % 2 == 0 && me.kr0 % 2 == 0 && s.nq % 2 == 0 && s.nk % 2 == 0, "%s: RoPE pairs of %d", name, b);
    for (int i = 0; i < s.nq; ++i) qx[me.kvh * (s.gh + 2 * s.hd) + (me.qr0 + i - me.kvh * s.gh)]++;
    for (int i = 0; i < s.nk; ++i) {
      qx[me.kvh * (s.gh + 2 * s.hd) + s.gh + (me.kr0 + i - me.kvh * s.hd)]++;
      qx[me.kvh * (s.gh + 2 * s.hd) + s.gh + s.hd + (me.kr0 + i - me.kvh * s.hd)]++;
    }
  }
  // records: every array on a cache line, in order, inside the allocation;
  // the blocks stored at workgroup scope (a kv head's q/k/v rows, a chunk's
  // partials) in whole lines, so no line holds two XCDs' blocks
  {
    std::vector<uint64_t> rec(pd_records(s));
    PdArgs a{};
    a.s = s;
    pd_bind_records(a, rec.data());
    const uint64_t* arr[6] = {a.rx, a.rx2, a.rh, a.rqkv, a.rpart, a.ratt};
    const size_t need[6] = {size_t(c.dim), size_t(c.dim), size_t(c.ffn), size_t(s.nkv) * (s.gh + 2 * s.hd),
                            size_t(s.nkv) * s.max_chunks * s.part_stride, size_t(s.nbq) * PD_REC_BLK};
    for (int i = 0; i < 6; ++i) {
      const size_t off = static_cast<size_t>(arr[i] - rec.data());
      const size_t end = i + 1 < 6 ? static_cast<size_t>(arr[i + 1] - rec.data()) : rec.size();
      CHECK(off % PD_REC_LINE == 0 && end >= off + need[i], "%s: record array %d", name, i);
    }
    CHECK((s.gh + 2 * s.hd) % PD_REC_LINE == 0 && s.part_stride % PD_REC_LINE == 0 &&
              s.part_stride >= s.gh + 2 * s.group,
          "%s: workgroup-scope record blocks in whole lines", name);
  }
  for (int v : hx) CHECK(v == 1, "%s: rows of x", name);
  for (int v : fx) CHECK(v == 1, "%s: FFN pairs", name);
  for (int v : qx) CHECK(v == 1, "%s: q/k/v records", name);
  // slab sources inside their planes
  const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
  const int rows[7] = {qd, kvd, kvd, c.dim, c.ffn, c.ffn, c.dim};
  const int types[7] = {MCPM_TYPE_Q4_K, MCPM_TYPE_Q4_K, tv, to, MCPM_TYPE_Q4_K, MCPM_TYPE_Q4_K, td};
  const int nbs[7] = {s.nbx, s.nbx, s.nbx, s.nbq, s.nbx, s.nbx, s.nbh};
  int64_t mapped = 0;
  for (int b = 0; b < s.G; ++b) {
    for (int off = 0; off < s.slab_stride; off += 16) {
      const PdSrc src = pd_slab_src(s, b, off, rows);
      if (src.tensor < 0) continue;
      const int64_t pb = plane_bytes(types[src.tensor], rows[src.tensor], nbs[src.tensor], src.plane);
      for (int k = 0; k < src.n; ++k)
        if (src.src[k] >= 0) {
          CHECK(src.src[k] + (src.n == 1 ? 16 : 2) <= pb && src.src[k] % (src.n == 1 ? 16 : 2) == 0,
                "%s: WG %d slab byte %d reads tensor %d plane %d at %lld of %lld", name, b, off, src.tensor,
                src.plane, static_cast<long long>(src.src[k]), static_cast<long long>(pb));
          ++mapped;
        }
    }
  }
  // every byte a task reads maps back to the expected (row, block, chunk)
  for (int b = 0; b < s.G; ++b) {
    const PdRows me = pd_rows(s, b);
    const PdGu gu = pd_gu(s, b);
    CHECK(gu.bytes <= s.reg_sz[2] && gu.u.off + pd_sub_bytes(gu.u.type, gu.u.R, s.nbx) <= gu.bytes,
          "%s: WG %d gate/up copy", name, b);
    struct Sub {
      int region, tensor, valid, row0, nb;
      PdSub sb;
    };
    const Sub subs[7] = {{0, 0, s.nq, me.qr0, s.nbx, s.sq},  {0, 1, s.nk, me.kr0, s.nbx, s.sk},
                         {0, 2, s.nk, me.kr0, s.nbx, s.sv},  {1, 3, me.nh, me.hr0, s.nbq, s.so},
                         {2, 4, me.np, me.fp0, s.nbx, gu.g}, {2, 5, me.np, me.fp0, s.nbx, gu.u},
                         {3, 6, me.nh, me.hr0, s.nbh, s.sd}};
    for (const Sub& q : subs) {
      const int R = q.sb.R, nc = q.sb.type == MCPM_TYPE_Q4_K ? 9 : 13;
      CHECK(q.valid <= R, "%s: valid rows", name);
      for (int row = 0; row < q.valid; ++row)
        for (int blk = 0; blk < q.nb; ++blk) {
          const int64_t gr = q.row0 + row, nrows = rows[q.tensor];
          for (int cc = 0; cc < nc; ++cc) {
            const int off = s.reg_off[q.region] + q.sb.off + ((blk * nc + cc) * R + row) * 16;
            const PdSrc src = pd_slab_src(s, b, off, rows);
            int plane;
            int64_t want;
            if (q.sb.type == MCPM_TYPE_Q4_K) {
              plane = cc < 8 ? 0 : 1;
              want = cc < 8 ? ((static_cast<int64_t>(blk) * 8 + cc) * nrows + gr) * 16 : (blk * nrows + gr) * 16;
            } else {
              plane = cc < 8 ? 0 : cc < 12 ? 1 : 2;
              want = cc < 8    ? ((static_cast<int64_t>(blk) * 8 + cc) * nrows + gr) * 16
                     : cc < 12 ? ((static_cast<int64_t>(blk) * 4 + cc - 8) * nrows + gr) * 16
                               : (blk * nrows + gr) * 16;
            }
            CHECK(src.tensor == q.tensor && src.plane == plane && src.n == 1 && src.src[0] == want,
                  "%s: WG %d tensor %d row %d block %d chunk %d", name, b, q.tensor, row, blk, cc);
          }
          if (q.sb.type == MCPM_TYPE_Q6_K) {
            const int e = blk * R + row;
            const int off = s.reg_off[q.region] + q.sb.off + 208 * R * q.nb + (e / 4) * 16;
            const PdSrc src = pd_slab_src(s, b, off, rows);
            CHECK(src.tensor == q.tensor && src.plane == 3 && src.n == 4 &&
                      src.src[e % 4] == (blk * nrows + gr) * 2,
                  "%s: WG %d tensor %d d of row %d block %d", name, b, q.tensor, row, blk);
          }
        }
    }
  }
  std::printf("%s: %lld slab sources checked\n", name, static_cast<long long>(mapped));
}

static void check_refused(const char* name, const mcpm_model_config& c, int n_cu, int max_seq) {
  PdShape s{};
  const char* why = nullptr;
  CHECK(!pd_plan(c, n_cu, max_seq, MCPM_TYPE_Q4_K, MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K, MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K,
                 s, &why),
        "%s: should be refused", name);
  std::printf("%s: refused (%s)\n", name, why ? why : "?");
}

static PdShape plan_of(const mcpm_model_config& c, int n_cu, int max_seq, int tv, int to, int td) {
  PdShape s{};
  if (!pd_plan(c, n_cu, max_seq, MCPM_TYPE_Q4_K, MCPM_TYPE_Q4_K, tv, to, td, s, nullptr)) s.G = -1;
  return s;
}

static void check_fixed_shape() {
  constexpr PdShape f = pd_fixed_plan();
  static_assert(f.G == 256 && f.dim == 2304 && f.nbh == 23, "the fixed plan is the 2.4B shape on 256 CUs");
  const int Q4 = MCPM_TYPE_Q4_K, Q6 = MCPM_TYPE_Q6_K;
  const PdShape r = plan_of(cfg(40, 2304, 32, 8, 64, 5760), 256, 4096, Q6, Q4, Q6);
  CHECK(r.G == 256 && std::memcmp(&r, &f, sizeof f) == 0, "compile-time plan differs from the run-time plan");
  for (int L : {1, 3, 40, 62})
    for (int ctx : {1, 64, 288, 1536, 4096})
      CHECK(pd_fixed_shape(plan_of(cfg(L, 2304, 32, 8, 64, 5760), 256, ctx, Q6, Q4, Q6)),
            "fixed shape not taken at %d layers, KV capacity %d", L, ctx);
  struct Other {
    const char* name;
    mcpm_model_config c;
    int n_cu, tv, to, td;
  };
  const Other others[] = {
      {"Q4_K v/down", cfg(40, 2304, 32, 8, 64, 5760), 256, Q4, Q4, Q4},
      {"Q4_K v", cfg(40, 2304, 32, 8, 64, 5760), 256, Q4, Q4, Q6},
      {"Q4_K down", cfg(40, 2304, 32, 8, 64, 5760), 256, Q6, Q4, Q4},
      {"FFN 5632", cfg(40, 2304, 32, 8, 64, 5632), 256, Q6, Q4, Q6},
      {"hidden 2048", cfg(40, 2048, 32, 8, 64, 5760), 256, Q6, Q4, Q6},
      {"small 8-kv", cfg(3, 1024, 32, 8, 64, 2816), 256, Q6, Q4, Q6},
  };
  for (const Other& o : others) {
    const PdShape s = plan_of(o.c, o.n_cu, 512, o.tv, o.to, o.td);
    CHECK(s.G > 0 && !pd_fixed_shape(s), "%s: %s", o.name, s.G > 0 ? "taken as the fixed shape" : "plan refused");
  }
  mcpm_model_config e = cfg(40, 2304, 32, 8, 64, 5760);
  e.eps = 1e-5f;
  CHECK(!pd_fixed_shape(plan_of(e, 256, 512, Q6, Q4, Q6)), "eps 1e-5 taken as the fixed shape");
  // the first-chunk owners' FFN pairs: the 56 the other 248 work groups
  // leave at 23 each, 7 per owner
  CHECK(pd_owner_pairs(f) == 7 && pd_rows(f, 0).np == 7 && pd_rows(f, 7).fp0 == 49 && pd_rows(f, 8).fp0 == 56 &&
            pd_rows(f, 8).np == 23 && pd_rows(f, 255).fp0 + pd_rows(f, 255).np == 5760,
        "owner FFN pairs of the fixed plan");
  std::printf("fixed-shape instance: plan %d B of LDS, taken for the 2.4B shape only; owners take %d FFN pairs\n",
              f.lds_bytes, pd_owner_pairs(f));
}

int main() {
  // the 2.4B shape on 256 CUs: the benchmark's context, the long-context
  // configuration's, and the longest the kernel takes
  const mcpm_model_config big = cfg(40, 2304, 32, 8, 64, 5760);
  check_shape("2.4B ctx 288", big, 256, 288, MCPM_TYPE_Q6_K, MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K);
  check_shape("2.4B ctx 1536", big, 256, 1536, MCPM_TYPE_Q6_K, MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K);
  check_shape("2.4B ctx 4096 Q4_K v/down", big, 256, 4096, MCPM_TYPE_Q4_K, MCPM_TYPE_Q4_K, MCPM_TYPE_Q4_K);
  // a small model with the same head geometry (the GPU tests' persistent case)
  check_shape("small 8-kv", cfg(3, 1024, 32, 8, 64, 2816), 256, 2304, MCPM_TYPE_Q6_K, MCPM_TYPE_Q4_K,
              MCPM_TYPE_Q6_K);
  check_shape("small 8-kv Q6_K o", cfg(2, 768, 32, 8, 64, 2000), 256, 512, MCPM_TYPE_Q4_K, MCPM_TYPE_Q6_K,
              MCPM_TYPE_Q4_K);
  // FFN sizes whose spare pairs give the first-chunk owners fewer rows than
  // the plan's (7 of 11, and none at all), in the gate/up layout of their own
  check_shape("small 8-kv ffn 2780", cfg(2, 1024, 32, 8, 64, 2780), 256, 512, MCPM_TYPE_Q6_K, MCPM_TYPE_Q4_K,
              MCPM_TYPE_Q6_K);
  check_shape("small 8-kv ffn 2600", cfg(2, 1024, 32, 8, 64, 2600), 256, 512, MCPM_TYPE_Q6_K, MCPM_TYPE_Q4_K,
              MCPM_TYPE_Q6_K);
  // FFN sizes past 16 Q8_K blocks: 20 blocks, whose 4 past the 16th fit the
  // 5 KiB of O weights a work group holds (one quantize round), and 23
  // blocks, whose 7 do not (two rounds)
  check_shape("small 8-kv ffn 5120", cfg(2, 1024, 32, 8, 64, 5120), 256, 512, MCPM_TYPE_Q6_K, MCPM_TYPE_Q4_K,
              MCPM_TYPE_Q6_K);
  check_shape("small 8-kv ffn 5888", cfg(2, 1024, 32, 8, 64, 5888), 256, 512, MCPM_TYPE_Q6_K, MCPM_TYPE_Q4_K,
              MCPM_TYPE_Q6_K);
  check_refused("2 kv heads", cfg(2, 512, 8, 2, 64, 1400), 256, 32);
  check_refused("head_dim 128", cfg(2, 2048, 16, 8, 128, 6144), 256, 64);
  check_refused("context past 2 chunks per work group", big, 256, 4160);
  check_refused("CU count not a multiple of 8", big, 252, 256);
  check_fixed_shape();
  if (failures) std::printf("%d check(s) failed\n", failures);
  else std::printf("all persistent-kernel plan checks passed\n");
  return failures ? 1 : 0;
}
