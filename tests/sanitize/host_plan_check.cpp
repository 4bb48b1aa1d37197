// CPU driver for the host-side argument checks and launch planning of
// libtrinix_attn.so (trinix_amd/csrc/host_plan.cpp), built by
// tests/test_host_sanitizers.py with AddressSanitizer and
// UndefinedBehaviorSanitizer (every report fatal).  It runs the status-code
// cases of the C ABI's validation, then a seeded fuzz over the whole range of
// every size, stride and window field (int64 extremes included), and checks
// the split-KV plan's invariants on every accepted decode call.  Exit status
// 0 and a final "ok" line mean no sanitizer report and no failed check.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>

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
  std::printf("cases %d, fuzz accepted %d, planned %d, failures %d\n", cases, accepted, planned, failures);
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
