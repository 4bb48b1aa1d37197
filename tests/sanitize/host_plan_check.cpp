// CPU driver for the host-side argument checks and launch planning of
// libtrinix_attn.so (trinix_amd/csrc/host_plan.cpp), built by
// tests/test_host_sanitizers.py with AddressSanitizer and
// UndefinedBehaviorSanitizer (every report fatal).  It runs the status-code
// cases of the C ABI's validation, then a seeded fuzz over the whole range of
// every size, stride and window field (int64 extremes included), and checks
// the split-KV plan's invariants on every accepted decode call.  The bounds
// model (bounds_model.h) then walks the kernels' index maps for the
// BASELINE configurations and edge shapes (every work item and row where
// the grid is small enough) and for a share of the accepted fuzz cases.
// Exit status 0 and a final "ok" line mean no sanitizer report and no
// failed check.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>

#include "bounds_model.h"
#include "host_plan.h"

using namespace trinix;

static int failures = 0;
#define CHECK(cond, ...)                                 \
  do {                                                   \
    if (!(cond)) {                                       \
      std::fprintf(stderr, "check failed: " __VA_ARGS__); \
      std::fprintf(stderr, "\n");                        \
      ++failures;                                        \
    }                                                    \
  } while (0)

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {  // xorshift64*
  rng ^= rng >> 12;
  rng ^= rng << 25;
  rng ^= rng >> 27;
  return rng * 0x2545F4914F6CDD1Dull;
}
static int64_t pick(const int64_t* vals, int n) { return vals[next_u64() % (uint64_t)n]; }

static const int64_t kEdge[] = {std::numeric_limits<int64_t>::min(), -(1ll << 40), -65536, -1, 0, 1, 2, 3, 7, 8,
                                15, 16, 17, 63, 64, 65, 127, 128, 1000, 4096, 8192, 65535, 1ll << 20, (1ll << 22) - 8,
                                1ll << 22, (1ll << 30) - 1, 1ll << 30, 1ll << 40, std::numeric_limits<int64_t>::max()};
static const int kNEdge = sizeof(kEdge) / sizeof(kEdge[0]);

static int64_t rand_size() {
  switch (next_u64() % 4) {
    case 0: return pick(kEdge, kNEdge);
    case 1: return (int64_t)(next_u64() % 17);
    case 2: return (int64_t)(next_u64() % 100000);
    default: return (int64_t)next_u64();
  }
}

static trinix_attn_fwd_args valid_fwd() {
  trinix_attn_fwd_args a;
  std::memset(&a, 0, sizeof(a));
  a.q = a.k = a.v = a.out = (void*)4096;
  const int64_t st[4] = {8 * 64 * 128, 8 * 128, 128, 1};
  for (int i = 0; i < 4; ++i) a.q_stride[i] = a.k_stride[i] = a.v_stride[i] = a.out_stride[i] = st[i];
  a.batch = 1;
  a.seqlen_q = 64;
  a.seqlen_k = 64;
  a.nheads_q = 8;
  a.nheads_kv = 8;
  a.head_dim = 128;
  a.dtype = TRINIX_BF16;
  a.softmax_scale = 0.088f;
  return a;
}

template <class Args>
static void set_mask(Args& x, int64_t sb, int64_t sh, int64_t si, int64_t sj) {
  x.mask = (const void*)4096;
  x.mask_dtype = TRINIX_F32;
  x.mask_stride[0] = sb;
  x.mask_stride[1] = sh;
  x.mask_stride[2] = si;
  x.mask_stride[3] = sj;
}

static trinix_attn_bwd_args valid_bwd() {
  trinix_attn_bwd_args a;
  std::memset(&a, 0, sizeof(a));
  a.q = a.k = a.v = a.out = a.dout = (void*)4096;
  a.dq = a.dk = a.dv = (void*)8192;
  a.lse = (const float*)4096;
  a.delta = (float*)8192;
  const int64_t st[4] = {8 * 64 * 128, 8 * 128, 128, 1};
  for (int i = 0; i < 4; ++i)
    a.q_stride[i] = a.k_stride[i] = a.v_stride[i] = a.out_stride[i] = a.dout_stride[i] = a.dq_stride[i] =
        a.dk_stride[i] = a.dv_stride[i] = st[i];
  a.batch = 1;
  a.seqlen_q = 64;
  a.seqlen_k = 64;
  a.nheads_q = 8;
  a.nheads_kv = 8;
  a.head_dim = 128;
  a.dtype = TRINIX_BF16;
  a.softmax_scale = 0.088f;
  return a;
}

// Invariants of an accepted split plan: the chunks tile the visible keys,
// the grid fits int32, the workspace matches rows * chunks * (D + 1) floats.
static void check_plan(const trinix_attn_fwd_args& a, const SplitPlan& pl) {
  CHECK(pl.n_splits >= 1 && pl.chunk >= 64 && pl.chunk % 64 == 0, "plan chunking");
  CHECK(pl.klo >= 0 && pl.klo < pl.khi && pl.khi <= a.seqlen_k, "plan key range");
  const int64_t span = (int64_t)pl.khi - pl.klo;
  CHECK((int64_t)pl.n_splits * pl.chunk >= span && (int64_t)(pl.n_splits - 1) * pl.chunk < span, "plan covers");
  const int64_t items = a.batch * a.nheads_kv * pl.RG;
  CHECK(items * pl.n_splits < (1ll << 31), "plan grid");
  const int64_t rows = a.batch * a.nheads_kv * pl.M;
  CHECK(pl.ws_bytes == (pl.n_splits > 1 ? rows * pl.n_splits * (a.head_dim + 1) * 4 : 0), "plan workspace");
}

int main() {
  int cases = 0;
  // ---- status codes of the forward's validation
  {
    trinix_attn_fwd_args a = valid_fwd();
    CHECK(validate_fwd_args(&a) == TRINIX_OK, "valid fwd");
    CHECK(validate_fwd_args(nullptr) == TRINIX_ERR_NULL_POINTER, "null args");
    struct Case {
      void (*edit)(trinix_attn_fwd_args&);
      int code;
    } table[] = {
        {[](trinix_attn_fwd_args& x) { x.q = nullptr; }, TRINIX_ERR_NULL_POINTER},
        {[](trinix_attn_fwd_args& x) { x.dtype = 7; }, TRINIX_ERR_BAD_DTYPE},
        {[](trinix_attn_fwd_args& x) { x.head_dim = 96; }, TRINIX_ERR_BAD_HEAD_DIM},
        {[](trinix_attn_fwd_args& x) { x.nheads_kv = 3; }, TRINIX_ERR_BAD_SHAPE},
        {[](trinix_attn_fwd_args& x) { x.seqlen_q = 0; }, TRINIX_ERR_BAD_SHAPE},
        {[](trinix_attn_fwd_args& x) { x.batch = std::numeric_limits<int64_t>::max(); }, TRINIX_ERR_BAD_SHAPE},
        {[](trinix_attn_fwd_args& x) { x.nheads_kv = std::numeric_limits<int64_t>::min(); }, TRINIX_ERR_BAD_SHAPE},
        {[](trinix_attn_fwd_args& x) { x.q_stride[3] = 2; }, TRINIX_ERR_BAD_STRIDE},
        {[](trinix_attn_fwd_args& x) { x.k_stride[2] = 130; }, TRINIX_ERR_BAD_STRIDE},
        {[](trinix_attn_fwd_args& x) { x.k_stride[1] = 1ll << 22; }, TRINIX_ERR_BAD_STRIDE},
        {[](trinix_attn_fwd_args& x) { x.v_stride[1] = std::numeric_limits<int64_t>::min(); }, TRINIX_ERR_BAD_STRIDE},
        {[](trinix_attn_fwd_args& x) { x.out = (void*)4100; }, TRINIX_ERR_BAD_STRIDE},
        {[](trinix_attn_fwd_args& x) { x.dropout_p = 1.0f; }, TRINIX_ERR_BAD_ARGUMENT},
        {[](trinix_attn_fwd_args& x) { x.dropout_p = NAN; }, TRINIX_ERR_BAD_ARGUMENT},
        {[](trinix_attn_fwd_args& x) { x.mask_blockmap = (const uint8_t*)4096; }, TRINIX_ERR_BAD_ARGUMENT},
        {[](trinix_attn_fwd_args& x) { x.rope_cos = (void*)4096; }, TRINIX_ERR_NULL_POINTER},
        {[](trinix_attn_fwd_args& x) { x.mask = (void*)4096; x.mask_dtype = 9; }, TRINIX_ERR_BAD_DTYPE},
        {[](trinix_attn_fwd_args& x) { x.q_norm_weight = (void*)4096; x.dropout_p = 0.1f; }, TRINIX_ERR_BAD_ARGUMENT},
        // mask strides: non-negative; a 32-row sub-tile's rows at 32-bit offsets
        {[](trinix_attn_fwd_args& x) { set_mask(x, 0, 0, -64, 1); }, TRINIX_ERR_BAD_STRIDE},
        {[](trinix_attn_fwd_args& x) { set_mask(x, -4096, 0, 64, 1); }, TRINIX_ERR_BAD_STRIDE},
        {[](trinix_attn_fwd_args& x) { set_mask(x, 0, 0, 1ll << 27, 1); }, TRINIX_ERR_BAD_STRIDE},
        {[](trinix_attn_fwd_args& x) { set_mask(x, 0, 0, (1ll << 31) / 31, 1); }, TRINIX_OK},
        {[](trinix_attn_fwd_args& x) { set_mask(x, 0, 0, 64, 1ll << 26); }, TRINIX_ERR_BAD_STRIDE},
        {[](trinix_attn_fwd_args& x) { x.seqlen_q = 1; set_mask(x, 0, 0, 1ll << 40, 1); }, TRINIX_OK},
    };
    for (const Case& c : table) {
      trinix_attn_fwd_args x = valid_fwd();
      c.edit(x);
      const int rc = validate_fwd_args(&x);
      CHECK(rc == c.code, "fwd case %d: got %d, want %d", cases, rc, c.code);
      ++cases;
    }
  }
  // ---- status codes of the backward's validation
  {
    trinix_attn_bwd_args a = valid_bwd();
    CHECK(validate_bwd_args(&a) == TRINIX_OK, "valid bwd");
    a.dtype = TRINIX_F32;
    a.q = (void*)4098;
    CHECK(validate_bwd_args(&a) == TRINIX_ERR_BAD_STRIDE, "bwd fp32 misaligned");
    a = valid_bwd();
    a.delta = nullptr;
    CHECK(validate_bwd_args(&a) == TRINIX_ERR_NULL_POINTER, "bwd delta");
    a = valid_bwd();
    a.dropout_p = -0.5f;
    CHECK(validate_bwd_args(&a) == TRINIX_ERR_BAD_ARGUMENT, "bwd dropout");
    a = valid_bwd();
    a.dk_stride[1] = std::numeric_limits<int64_t>::max();
    CHECK(validate_bwd_args(&a) == TRINIX_ERR_BAD_STRIDE, "bwd stride");
    // the dK/dV kernel reads a mask sub-tile's 32 rows at 32-bit offsets
    // r * row_stride from its first row (64-bit): (Sq = 64) 31 * stride < 2^31
    a = valid_bwd();
    set_mask(a, 0, 0, (1ll << 31) / 31 + 1, 1);
    CHECK(validate_bwd_args(&a) == TRINIX_ERR_BAD_STRIDE, "bwd mask row stride");
    a = valid_bwd();
    set_mask(a, 0, 0, (1ll << 31) / 31, 1);
    CHECK(validate_bwd_args(&a) == TRINIX_OK, "bwd mask row stride at the limit");
    a = valid_bwd();
    set_mask(a, 0, 0, -1, 1);
    CHECK(validate_bwd_args(&a) == TRINIX_ERR_BAD_STRIDE, "bwd negative mask row stride");
    a = valid_bwd();
    a.seqlen_q = a.seqlen_k = 70000;  // a contiguous mask beyond 2^32 elements
    set_mask(a, 0, 0, 70000, 1);
    CHECK(validate_bwd_args(&a) == TRINIX_OK, "bwd contiguous mask of 70000^2");
    cases += 9;
  }
  // ---- the tuning override TRINIX_ATTN_CFG="nw,occ,bn[,ks]": ks 0 (the
  // per-item split), 1 and 2 are taken, anything else leaves the planner's
  // choice
  {
    auto forced = [](const char* v) {
      setenv("TRINIX_ATTN_CFG", v, 1);
      const Cfg16 c = pick_cfg16(64, 1, 4, 512, true, true, true);
      unsetenv("TRINIX_ATTN_CFG");
      return c;
    };
    const Cfg16 dflt = pick_cfg16(64, 1, 4, 512, true, true, true);
    Cfg16 c = forced("4,2,64,0");
    CHECK(c.nw == 4 && c.occ == 2 && c.bn == 64 && c.ks == 0, "override ks 0");
    c = forced("4,2,64,2");
    CHECK(c.ks == 2, "override ks 2");
    c = forced("8,2,128");
    CHECK(c.nw == 8 && c.bn == 128 && c.ks == 1, "override without ks");
    c = forced("4,2,64,3");
    CHECK(c.nw == dflt.nw && c.bn == dflt.bn && c.ks == dflt.ks, "override ks 3 rejected");
    c = forced("3,2,64,2");
    CHECK(c.nw == dflt.nw && c.ks == dflt.ks, "override nw not a multiple of ks rejected");
    cases += 5;
  }
  // ---- fuzz: every field over its whole range
  int accepted = 0, planned = 0;
  for (int it = 0; it < 200000; ++it) {
    trinix_attn_fwd_args a = valid_fwd();
    a.batch = rand_size();
    a.seqlen_q = next_u64() % 3 ? (int64_t)(next_u64() % 20) : rand_size();
    a.seqlen_k = rand_size();
    a.nheads_kv = next_u64() % 2 ? (int64_t)(1 + next_u64() % 8) : rand_size();
    const bool small_kv = a.nheads_kv > 0 && a.nheads_kv <= (1 << 20);
    a.nheads_q = small_kv && next_u64() % 2 ? a.nheads_kv * (int64_t)(1 + next_u64() % 8) : rand_size();
    if (a.nheads_kv > 0 && a.nheads_q > 0 && a.nheads_q % a.nheads_kv) a.nheads_q = a.nheads_kv;
    a.head_dim = next_u64() % 5 ? (int64_t)(64 << (next_u64() % 3)) : rand_size();
    a.dtype = (int32_t)(next_u64() % 4);
    a.causal = (int32_t)(next_u64() % 2);
    a.has_window = (int32_t)(next_u64() % 2);
    a.window_left = rand_size();
    a.window_right = rand_size();
    for (int i = 0; i < 3; ++i) {
      if (next_u64() % 8 == 0) a.q_stride[i] = rand_size();
      if (next_u64() % 8 == 0) a.k_stride[i] = rand_size();
      if (next_u64() % 8 == 0) a.v_stride[i] = rand_size();
    }
    if (next_u64() % 16 == 0) a.dropout_p = (float)(next_u64() % 1000) / 900.f;
    const int rc = validate_fwd_args(&a);
    if (rc != TRINIX_OK) continue;
    ++accepted;
    const bool plain = !a.mask && a.dropout_p == 0.f;
    const bool split_ok = plain && a.causal && !a.has_window;
    const Cfg16 c = pick_cfg16(a.head_dim, a.batch, a.nheads_q, a.seqlen_q, a.causal || a.has_window, plain,
                               split_ok);
    CHECK((c.nw == 4 && c.bn == 64 && (c.ks == 1 || c.ks == 2)) ||
              (c.nw == 4 && c.bn == 64 && c.ks == 0 && a.head_dim == 64 && split_ok) ||
              (c.nw == 8 && c.bn == 128 && c.ks == 1 && a.head_dim == 128 && plain), "tile config");
    if (c.ks == 0) {
      uint8_t items[kMaxRowItems];
      const int n = plan_split_rows(a.seqlen_q, a.seqlen_k, a.batch * a.nheads_q, 128, 64, items, kMaxRowItems);
      CHECK(n >= 0 && n <= kMaxRowItems, "split items");
      // every 128-row block appears once whole or as both halves
      int seen[64] = {0};
      for (int k = 0; k < n; ++k) seen[items[k] >> 2] += (items[k] & 2) ? 1 : 2;
      const int64_t nb = (a.seqlen_q + 127) / 128;
      for (int64_t rb = 0; n > 0 && rb < nb; ++rb) CHECK(seen[rb] == 2, "split items cover every row block");
    }
    SplitPlan pl;
    if (make_split_plan(&a, &pl)) {
      ++planned;
      check_plan(a, pl);
      CHECK(a.seqlen_q <= kDecodeMaxSq, "plan only for decode shapes");
      CHECK(pl.ws_bytes <= (int64_t)TRINIX_SPLITKV_SCRATCH_BYTES, "default plan fits the static scratch");
    }
  }
  for (int it = 0; it < 50000; ++it) {
    trinix_attn_bwd_args a = valid_bwd();
    a.batch = rand_size();
    a.seqlen_q = rand_size();
    a.seqlen_k = rand_size();
    a.nheads_kv = rand_size();
    a.nheads_q = rand_size();
    a.head_dim = next_u64() % 3 ? (int64_t)(64 << (next_u64() % 3)) : rand_size();
    a.dtype = (int32_t)(next_u64() % 4);
    for (int i = 0; i < 4; ++i)
      if (next_u64() % 4 == 0) a.dk_stride[i] = rand_size();
    if (next_u64() % 2 == 0) set_mask(a, rand_size(), rand_size(), rand_size(), rand_size());
    if (validate_bwd_args(&a) != TRINIX_OK) continue;
    if (a.mask) {
      // what the kernels' mask addressing relies on (see mask_strides_ok)
      for (int i = 0; i < 4; ++i) CHECK(a.mask_stride[i] >= 0, "accepted mask stride >= 0");
      const int64_t rows = a.seqlen_q - 1 < 31 ? a.seqlen_q - 1 : 31;
      CHECK((__int128)rows * a.mask_stride[2] < ((__int128)1 << 31), "sub-tile row offsets fit 31 bits");
      CHECK((__int128)(a.seqlen_k - 1) * a.mask_stride[3] < ((__int128)1 << 31), "key offsets fit 31 bits");
    }
    const bool masked = next_u64() % 2 == 0;
    if (pick_dq_wide(a.head_dim, a.batch, a.nheads_q, a.seqlen_q, a.causal || a.has_window, masked))
      CHECK(a.head_dim == 128 && !masked, "wide dQ only at head_dim 128 without a mask");
  }
  // ---- bounds model: curated shapes (every item and row where small), then
  // a share of the fuzz's accepted argument sets (sampled items)
  bounds::Report BR;
  int modelled = 0;
  auto model_one = [&](const trinix_attn_fwd_args& f, int64_t limit) {
    if (validate_fwd_args(&f) != TRINIX_OK || f.dtype == TRINIX_F32) return;
    FwdPlan fp;
    if (plan_fwd(&f, &fp) == TRINIX_OK) bounds::model_fwd16(BR, f, fp, limit);
    SplitPlan sp;
    if (make_split_plan(&f, &sp)) bounds::model_decode(BR, f, sp, limit);
    if (f.head_dim <= 128 && f.q_norm_weight == nullptr) {
      trinix_attn_bwd_args b = valid_bwd();
      b.batch = f.batch, b.seqlen_q = f.seqlen_q, b.seqlen_k = f.seqlen_k, b.nheads_q = f.nheads_q;
      b.nheads_kv = f.nheads_kv, b.head_dim = f.head_dim, b.dtype = f.dtype, b.causal = f.causal;
      b.has_window = f.has_window, b.window_left = f.window_left, b.window_right = f.window_right;
      b.mask = f.mask, b.mask_dtype = f.mask_dtype, b.mask_blockmap = f.mask_blockmap, b.dropout_p = f.dropout_p;
      b.dropout_keep_map = f.dropout_keep_map;
      for (int i = 0; i < 4; ++i) {
        b.q_stride[i] = b.dout_stride[i] = b.out_stride[i] = b.dq_stride[i] = f.q_stride[i];
        b.k_stride[i] = b.dk_stride[i] = f.k_stride[i];
        b.v_stride[i] = b.dv_stride[i] = f.v_stride[i];
        b.mask_stride[i] = f.mask_stride[i];
      }
      BwdPlan bp;
      if (validate_bwd_args(&b) == TRINIX_OK && plan_bwd(&b, &bp) == TRINIX_OK) bounds::model_bwd16(BR, b, bp, limit);
    }
    ++modelled;
  };
  auto shape = [](int64_t B, int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D, int dtype) {
    trinix_attn_fwd_args a = valid_fwd();
    a.batch = B, a.seqlen_q = Sq, a.seqlen_k = Sk, a.nheads_q = Hq, a.nheads_kv = Hkv, a.head_dim = D, a.dtype = dtype;
    const int64_t q[4] = {Sq * Hq * D, Hq * D, D, 1}, kv[4] = {Sk * Hkv * D, Hkv * D, D, 1};
    for (int i = 0; i < 4; ++i) a.q_stride[i] = a.out_stride[i] = q[i], a.k_stride[i] = a.v_stride[i] = kv[i];
    return a;
  };
  {
    const int64_t kAll = 1 << 16;  // list every work item / row up to this many
    std::vector<trinix_attn_fwd_args> cur;
    auto add = [&](trinix_attn_fwd_args a) { cur.push_back(a); };
    trinix_attn_fwd_args a;
    a = shape(4, 1024, 1024, 12, 12, 64, TRINIX_BF16), a.causal = 1, add(a);          // C2
    a = shape(1, 8192, 8192, 32, 8, 128, TRINIX_BF16), a.causal = 1, add(a);          // C3
    a = shape(2, 16384, 16384, 32, 8, 128, TRINIX_BF16), a.causal = 1;                // C4
    a.has_window = 1, a.window_left = 4096, a.window_right = 0, add(a);
    a = shape(8, 2048, 2048, 16, 16, 64, TRINIX_F16);                                 // C5a, mask + block map
    a.mask = (void*)4096, a.mask_dtype = TRINIX_F32, a.mask_blockmap = (const uint8_t*)4096;
    a.mask_stride[0] = a.mask_stride[1] = 0, a.mask_stride[2] = 2048, a.mask_stride[3] = 1, add(a);
    a.nheads_kv = 1, a.k_stride[2] = a.v_stride[2] = 0, add(a);                       // C5b (expanded KV)
    for (int64_t D : {64, 128, 256})
      for (int64_t Sq : {1, 17, 100, 128, 300})
        for (int64_t Sk : {1, 63, 64, 65, 300})
          for (int c = 0; c < 6; ++c) {
            a = shape(2, Sq, Sk, 4, c % 2 ? 1 : 2, D, c % 3 ? TRINIX_BF16 : TRINIX_F16);
            a.causal = c & 1;
            if (c >= 2) a.has_window = 1, a.window_left = c == 4 ? -3 : 40, a.window_right = c == 5 ? (1ll << 62) : 7;
            if (c == 3) a.mask = (void*)4096, a.mask_dtype = TRINIX_BF16, a.mask_blockmap = (const uint8_t*)4096,
                        a.mask_stride[2] = Sk, a.mask_stride[3] = 1;
            if (c == 5) a.dropout_p = 0.25f, a.dropout_keep_map = D <= 128 ? (void*)4096 : nullptr;
            add(a);
          }
    a = shape(4, 1024, 1024, 12, 12, 64, TRINIX_BF16), a.causal = 1;                     // C2, C3 with dropout
    a.dropout_p = 0.1f, a.dropout_keep_map = (void*)4096, add(a);
    a = shape(1, 8192, 8192, 32, 8, 128, TRINIX_BF16), a.causal = 1;
    a.dropout_p = 0.1f, a.dropout_keep_map = (void*)4096, add(a);
    a = shape(3, 300, 77, 6, 2, 64, TRINIX_F16), a.dropout_p = 0.3f, a.dropout_keep_map = (void*)4096, add(a);
    a = shape(1, 40000, 40000, 2, 1, 64, TRINIX_BF16), a.causal = 1, a.has_window = 1;  // long, two-sided window
    a.window_left = 8192, a.window_right = 300, add(a);
    a = shape(3, 9, 70000, 32, 8, 128, TRINIX_BF16), a.causal = 1, add(a);              // decode shapes
    a = shape(16, 1, 8192, 32, 8, 128, TRINIX_BF16), add(a);
    a = shape(1, 5, 777, 8, 2, 64, TRINIX_F16), a.has_window = 1, a.window_left = 100, a.window_right = -2, add(a);
    a = shape(1, 64, 64, 8, 8, 128, TRINIX_BF16), a.has_window = 1;                       // extreme windows
    a.window_left = std::numeric_limits<int64_t>::min(), a.window_right = std::numeric_limits<int64_t>::max(), add(a);
    a.window_left = std::numeric_limits<int64_t>::max(), a.window_right = std::numeric_limits<int64_t>::min(), add(a);
    for (const auto& f : cur) model_one(f, kAll);
    cases += (int)cur.size();
  }
  {
    // fuzz share: 1 in 40 accepted 16-bit argument sets, sampled items
    bounds::g_sample_ends = 3, bounds::g_sample_inner = 6;
    rng = 0x1234567887654321ull;
    int ran = 0;
    for (int it = 0; it < 400000 && ran < 1500; ++it) {
      trinix_attn_fwd_args a = valid_fwd();
      a.batch = next_u64() % 3 ? (int64_t)(1 + next_u64() % 8) : rand_size();
      a.seqlen_q = next_u64() % 2 ? (int64_t)(1 + next_u64() % 20) : rand_size();
      a.seqlen_k = rand_size();
      a.nheads_kv = (int64_t)(1 + next_u64() % 8);
      a.nheads_q = a.nheads_kv * (int64_t)(1 + next_u64() % 8);
      a.head_dim = (int64_t)(64 << (next_u64() % 3));
      a.dtype = next_u64() % 2 ? TRINIX_BF16 : TRINIX_F16;
      a.causal = (int32_t)(next_u64() % 2);
      a.has_window = (int32_t)(next_u64() % 2);
      a.window_left = rand_size();
      a.window_right = rand_size();
      if (next_u64() % 2) a.window_left = (int64_t)(next_u64() % 3000) - 1000;  // small, both signs
      if (next_u64() % 2) a.window_right = (int64_t)(next_u64() % 3000) - 1000;
      const int64_t kvs = next_u64() % 2 ? a.nheads_kv * a.head_dim : (int64_t)(8 * (next_u64() % (1 << 19)));
      a.k_stride[1] = a.v_stride[1] = kvs;
      if (next_u64() % 3 == 0) {
        a.mask = (void*)4096, a.mask_dtype = (int32_t)(next_u64() % 4);
        a.mask_blockmap = next_u64() % 2 ? (const uint8_t*)4096 : nullptr;
        a.mask_stride[0] = rand_size(), a.mask_stride[1] = rand_size();
        a.mask_stride[2] = rand_size(), a.mask_stride[3] = next_u64() % 2 ? 1 : rand_size();
      }
      if (next_u64() % 4 == 0) {
        a.dropout_p = 0.1f;
        if (a.head_dim <= 128) a.dropout_keep_map = (void*)4096;
      }
      if (validate_fwd_args(&a) != TRINIX_OK) continue;
      model_one(a, 4096);
      ++ran;
    }
    cases += ran;
  }
  std::printf("bounds model: %d argument sets, %ld checks, %ld failures\n", modelled, BR.checks, BR.failures);
  failures += (int)BR.failures;
  std::printf("cases %d, fuzz accepted %d, planned %d, failures %d\n", cases, accepted, planned, failures);
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
