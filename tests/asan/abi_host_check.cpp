// Host-side check of the C ABI (include/fused_tq.h) under AddressSanitizer and
// UndefinedBehaviorSanitizer.  Built by run_host_asan.sh from the library's own
// sources with host-only compilation (no device code: every kernel launch
// fails with a HIP error), linked into this one executable.
//
// What it drives:
//   * every size / heuristic helper over a grid of ordinary and extreme
//     arguments (INT_MIN .. INT_MAX): no overflow, and -1 or a sane value;
//   * ftq_codebook_class on heap arrays of exactly 2^bits + 1 boundaries, so a
//     read past the table is reported;
//   * every compute entry point with each argument error its checks name
//     (dims, widths, dtypes, counts, strides up to INT64_MAX, misaligned and
//     null pointers, short workspaces): -1 and a NUL-terminated message;
//     empty inputs: 0;
//   * when no GPU is visible (the build container), the same entry points
//     with valid arguments on host buffers: the launch fails and the HIP
//     error comes back as a positive status with its message.  With a GPU
//     present this part is skipped (host pointers must never reach a real
//     launch).
// Exit status 0 when every expectation holds; a sanitizer report aborts.

#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "fused_tq.h"

static int g_fail = 0, g_checks = 0;

#define EXPECT(cond, ...)                                              \
  do {                                                                 \
    ++g_checks;                                                        \
    if (!(cond)) {                                                     \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);        \
      std::fprintf(stderr, __VA_ARGS__);                               \
      std::fputc('\n', stderr);                                        \
      ++g_fail;                                                        \
    }                                                                  \
  } while (0)

static void message_ok(const char* what) {
  const char* m = ftq_last_error();
  EXPECT(m != nullptr, "%s: null error string", what);
  if (m) {
    const size_t n = strnlen(m, 1024);
    EXPECT(n > 0 && n < 512, "%s: error string length %zu", what, n);
  }
}

static void arg_error(int rc, const char* what) {
  EXPECT(rc == FTQ_ERR_ARG, "%s: rc %d, want -1 (%s)", what, rc, ftq_last_error());
  message_ok(what);
}

static void hip_error(int rc, const char* what) {
  EXPECT(rc > 0, "%s: rc %d, want a HIP error (%s)", what, rc, ftq_last_error());
  message_ok(what);
}

// 16-byte aligned host buffer; freed at exit
struct Buf {
  std::vector<void*> all;
  uint8_t* get(size_t n) {
    void* p = std::aligned_alloc(64, (n + 63) / 64 * 64);
    std::memset(p, 0, (n + 63) / 64 * 64);
    all.push_back(p);
    return static_cast<uint8_t*>(p);
  }
  ~Buf() {
    for (void* p : all) std::free(p);
  }
};

static const int kInts[] = {INT_MIN, -65536, -1, 0, 1, 2, 3, 4, 7, 8, 16, 63, 64, 96, 128, 255, 256, 512,
                            1024, 4096, 65536, 1 << 20, INT_MAX / 2, INT_MAX};

static void sizes() {
  for (int d : kInts)
    for (int a : {-1, 0, 1, 2, 3, 4, 5, 8, 9})
      for (int b : {-1, 0, 1, 2, 3, 4, 5, 8, 9}) {
        const int64_t p = ftq_paged_subblock_bytes(d, a, b);
        EXPECT(p == -1 || (p > 0 && p < (int64_t)1 << 32), "paged_subblock_bytes(%d,%d,%d) = %lld", d, a, b,
               (long long)p);
        const int64_t s = ftq_v1_slot_bytes(d, a, b);
        EXPECT(s == -1 || (s > 0 && s < (int64_t)1 << 32), "v1_slot_bytes(%d,%d,%d) = %lld", d, a, b,
               (long long)s);
        for (int f : {-1, 0, 1, 2, 3, 4, 7, 8, 15, 16}) {
          const int64_t t = ftq_v1_slot_bytes_flags(d, a, b, f);
          EXPECT(t == -1 || (t > 0 && t < (int64_t)1 << 32), "v1_slot_bytes_flags(%d,%d,%d,%d) = %lld", d, a,
                 b, f, (long long)t);
        }
      }
  for (int d : kInts) {
    const int64_t r = ftq_raw_slot_bytes(d);
    EXPECT(r == -1 || r == 4 * (int64_t)d, "raw_slot_bytes(%d) = %lld", d, (long long)r);
  }
  for (int b : kInts)
    for (int h : kInts)
      for (int d : {-1, 0, 64, 128, 256, INT_MAX})
        for (int s : {INT_MIN, -1, 0, 1, 8, 1024, 1025, INT_MAX}) {
          int64_t w[3] = {ftq_paged_workspace_bytes(b, h, d, s), ftq_v1_workspace_bytes(b, h, d, s),
                          ftq_raw_workspace_bytes(b, h, d, s)};
          for (int k = 0; k < 3; ++k)
            EXPECT(w[k] >= -1, "workspace_bytes[%d](%d,%d,%d,%d) = %lld", k, b, h, d, s, (long long)w[k]);
        }
  for (int b : kInts)
    for (int h : kInts)
      for (int L : kInts) {
        const int s[3] = {ftq_paged_default_splits(b, h, L), ftq_v1_default_splits(b, h, L),
                          ftq_raw_default_splits(b, h, L)};
        for (int k = 0; k < 3; ++k)
          EXPECT(s[k] >= 1 && s[k] <= 1024, "default_splits[%d](%d,%d,%d) = %d", k, b, h, L, s[k]);
        for (int hq : {1, 4, 8, 32, INT_MAX})
          for (int d : {64, 128, 256}) {
            const int c = ftq_paged_choose_splits(b, hq, h, d, L);
            EXPECT(c >= 1 && c <= 1024, "choose_splits(%d,%d,%d,%d,%d) = %d", b, hq, h, d, L, c);
            // widths in and out of the matrix-core range, flags with and without the VALU bit
            for (int kb : {1, 2, 4, 8})
              for (int fl : {0, 3, 8}) {
                const int v = ftq_v1_choose_splits(b, hq, h, d, kb, kb == 8 ? 8 : 6 - kb, fl, L);
                EXPECT(v >= 1 && v <= 1024, "v1_choose_splits(%d,%d,%d,%d,%d,%d,%d) = %d", b, hq, h, d, kb, fl, L, v);
              }
          }
      }
  EXPECT(ftq_v1_scratch_bytes() > 0, "scratch bytes");
  EXPECT(ftq_version() == FTQ_ABI_VERSION, "version");
}

static void codebook_class() {
  for (int bits = 2; bits <= 4; ++bits) {
    const int n = (1 << bits) + 1;
    // exactly n floats on the heap: a read of boundaries[n] is reported
    float* sym = static_cast<float*>(std::malloc(sizeof(float) * n));
    for (int k = 0; k < n; ++k) sym[k] = (float)(k - (n - 1) / 2) * 0.25f;
    sym[0] = -INFINITY;
    sym[n - 1] = INFINITY;
    EXPECT(ftq_codebook_class(sym, bits) == FTQ_CB_SYMMETRIC, "symmetric table, bits %d", bits);
    sym[1] -= 0.01f;
    EXPECT(ftq_codebook_class(sym, bits) == FTQ_CB_ANY, "asymmetric table, bits %d", bits);
    sym[2] = NAN;
    EXPECT(ftq_codebook_class(sym, bits) == FTQ_CB_ANY, "NaN table, bits %d", bits);
    std::free(sym);
  }
  float t[17] = {};
  for (int bits : {INT_MIN, -1, 0, 1, 5, 8, INT_MAX}) arg_error(ftq_codebook_class(t, bits), "codebook_class bits");
  arg_error(ftq_codebook_class(nullptr, 3), "codebook_class null");
}

static void codec(bool launch) {
  Buf B;
  const int64_t n = 4;
  uint8_t* x = B.get(n * 256 * 4);
  float* signs = reinterpret_cast<float*>(B.get(4096 * 4));
  float* bnd = reinterpret_cast<float*>(B.get(17 * 4));
  uint8_t* packed = B.get(n * 256);
  uint16_t* norms = reinterpret_cast<uint16_t*>(B.get(n * 2));
  uint8_t* y = B.get(n * 256 * 4);
  // encode / encode_cb / encode_kv
  for (int d : {INT_MIN, -128, 0, 4, 100, 8192, INT_MAX}) {
    arg_error(ftq_encode(x, FTQ_BF16, n, d, signs, bnd, 3, packed, norms, nullptr), "encode d");
    arg_error(ftq_encode_kv(x, x, FTQ_BF16, n, d, signs, bnd, 3, 0, packed, norms, packed, norms, nullptr),
              "encode_kv d");
    arg_error(ftq_decode(packed, norms, n, d, bnd, signs, 3, y, FTQ_F32, nullptr), "decode d");
    arg_error(ftq_rht(x, FTQ_F32, n, d, signs, 0, y, FTQ_F32, nullptr), "rht d");
  }
  for (int bits : {INT_MIN, 0, 1, 5, INT_MAX}) {
    arg_error(ftq_encode(x, FTQ_BF16, n, 128, signs, bnd, bits, packed, norms, nullptr), "encode bits");
    arg_error(ftq_decode(packed, norms, n, 128, bnd, signs, bits, y, FTQ_F32, nullptr), "decode bits");
  }
  for (int dt : {INT_MIN, -1, 3, INT_MAX}) {
    arg_error(ftq_encode(x, dt, n, 128, signs, bnd, 3, packed, norms, nullptr), "encode dtype");
    arg_error(ftq_decode(packed, norms, n, 128, bnd, signs, 3, y, dt, nullptr), "decode dtype");
    arg_error(ftq_rht(x, dt, n, 128, signs, 0, y, FTQ_F32, nullptr), "rht dtype");
    arg_error(ftq_rht(x, FTQ_F32, n, 128, signs, 0, y, dt, nullptr), "rht out dtype");
  }
  for (int64_t bad_n : {INT64_MIN, (int64_t)-1})
    arg_error(ftq_encode(x, FTQ_BF16, bad_n, 128, signs, bnd, 3, packed, norms, nullptr), "encode n");
  for (int cls : {-1, 2, 7}) {
    arg_error(ftq_encode_cb(x, FTQ_BF16, n, 128, signs, bnd, 3, cls, packed, norms, nullptr), "encode_cb class");
    arg_error(ftq_encode_kv(x, x, FTQ_BF16, n, 128, signs, bnd, 3, cls, packed, norms, packed, norms, nullptr),
              "encode_kv class");
  }
  arg_error(ftq_encode(nullptr, FTQ_BF16, n, 128, signs, bnd, 3, packed, norms, nullptr), "encode null x");
  arg_error(ftq_encode(x, FTQ_BF16, n, 128, nullptr, bnd, 3, packed, norms, nullptr), "encode null signs");
  arg_error(ftq_encode(x + 2, FTQ_BF16, n, 128, signs, bnd, 3, packed, norms, nullptr), "encode misaligned x");
  arg_error(ftq_encode_kv(x, x + 8, FTQ_BF16, n, 128, signs, bnd, 3, 0, packed, norms, packed, norms, nullptr),
            "encode_kv misaligned v");
  arg_error(ftq_encode_kv(x, x, FTQ_BF16, n, 128, signs, bnd, 3, 0, packed, norms, packed, nullptr, nullptr),
            "encode_kv null v norms");
  arg_error(ftq_decode(packed, norms, n, 128, bnd, signs, 3, y + 4, FTQ_F32, nullptr), "decode misaligned out");
  arg_error(ftq_decode(nullptr, norms, n, 128, bnd, signs, 3, y, FTQ_F32, nullptr), "decode null packed");
  arg_error(ftq_rht(x, FTQ_F32, n, 128, signs, 0, y + 4, FTQ_F32, nullptr), "rht misaligned out");
  // empty inputs need no pointers
  EXPECT(ftq_encode(nullptr, FTQ_BF16, 0, 128, nullptr, nullptr, 3, nullptr, nullptr, nullptr) == 0, "encode n=0");
  EXPECT(ftq_encode_kv(nullptr, nullptr, FTQ_BF16, 0, 128, nullptr, nullptr, 3, 0, nullptr, nullptr, nullptr,
                       nullptr, nullptr) == 0,
         "encode_kv n=0");
  EXPECT(ftq_decode(nullptr, nullptr, 0, 64, nullptr, nullptr, 2, nullptr, FTQ_F16, nullptr) == 0, "decode n=0");
  EXPECT(ftq_rht(nullptr, FTQ_F32, 0, 256, nullptr, 1, nullptr, FTQ_BF16, nullptr) == 0, "rht n=0");
  if (!launch) return;
  for (int d : {64, 128, 256, 32, 512}) {  // 32 and 512: the any-dimension kernels
    for (int bits = 2; bits <= 4; ++bits) {
      hip_error(ftq_encode(x, FTQ_BF16, n, d, signs, bnd, bits, packed, norms, nullptr), "encode launch");
      hip_error(ftq_encode_cb(x, FTQ_F16, n, d, signs, bnd, bits, FTQ_CB_SYMMETRIC, packed, norms, nullptr),
                "encode_cb launch");
      hip_error(ftq_decode(packed, norms, n, d, bnd, signs, bits, y, FTQ_BF16, nullptr), "decode launch");
    }
    hip_error(ftq_encode_kv(x, x, FTQ_F32, n, d, signs, bnd, 3, 0, packed, norms, packed, norms, nullptr),
              "encode_kv launch");
    hip_error(ftq_rht(x, FTQ_F32, n, d, signs, 1, y, FTQ_F16, nullptr), "rht launch");
  }
}

static void paged(bool launch) {
  Buf B;
  const int nt = 5, hkv = 2, hq = 8, d = 128, page = 16, bk = 3, bv = 3;
  const int64_t nb = 4;
  const int64_t sub = ftq_paged_subblock_bytes(d, bk, bv);
  EXPECT(sub > 0, "subblock bytes");
  uint8_t* kv = B.get(nt * hkv * 256 * 4);
  float* signs = reinterpret_cast<float*>(B.get(256 * 4));
  float* bnd = reinterpret_cast<float*>(B.get(17 * 4));
  int64_t* slots = reinterpret_cast<int64_t*>(B.get(nt * 8));
  uint8_t* cache = B.get(nb * (page / 16) * hkv * sub + 64);
  // store
  for (int dd : {64, 100, 512})
    arg_error(ftq_paged_store(kv, kv, FTQ_BF16, nt, hkv, dd, signs, signs, bnd, bnd, bk, bv, slots, cache, page, nb,
                              nullptr),
              "paged_store d");
  for (int ps : {0, 8, 24})
    arg_error(ftq_paged_store(kv, kv, FTQ_BF16, nt, hkv, d, signs, signs, bnd, bnd, bk, bv, slots, cache, ps, nb,
                              nullptr),
              "paged_store page");
  arg_error(ftq_paged_store(kv, kv, FTQ_BF16, nt, 0, d, signs, signs, bnd, bnd, bk, bv, slots, cache, page, nb, nullptr),
            "paged_store heads");
  arg_error(ftq_paged_store(kv, kv, FTQ_BF16, nt, hkv, d, signs, signs, bnd, bnd, 1, bv, slots, cache, page, nb, nullptr),
            "paged_store bits");
  arg_error(ftq_paged_store(kv, kv, FTQ_BF16, nt, hkv, d, signs, signs, bnd, bnd, bk, bv, nullptr, cache, page, nb,
                            nullptr),
            "paged_store null slots");
  arg_error(ftq_paged_store(kv, kv, FTQ_BF16, nt, hkv, d, signs, signs, bnd, bnd, bk, bv, slots, cache + 4, page, nb,
                            nullptr),
            "paged_store misaligned cache");
  EXPECT(ftq_paged_store(nullptr, nullptr, FTQ_BF16, 0, hkv, d, nullptr, nullptr, nullptr, nullptr, bk, bv, nullptr,
                         nullptr, page, 0, nullptr) == 0,
         "paged_store n=0");
  // attention
  const int B_ = 2, mb = 3, S = 2;
  uint8_t* q = B.get(B_ * hq * d * 4);
  int32_t* bt = reinterpret_cast<int32_t*>(B.get(B_ * mb * 4));
  int32_t* sl = reinterpret_cast<int32_t*>(B.get(B_ * 4));
  float* lev = reinterpret_cast<float*>(B.get(16 * 4));
  const int64_t wsb = ftq_paged_workspace_bytes(B_, hq, d, S);
  EXPECT(wsb > 0, "paged workspace bytes");
  uint8_t* ws = B.get(wsb);
  uint8_t* out = B.get(B_ * hq * d * 4);
  auto attn = [&](int bb, int hq_, int hkv_, int d_, int page_, int mb_, int64_t nb_, int bk_, int bv_, int s_,
                  void* ws_, int64_t wsb_, const void* q_, void* out_, int qt, int ot, bool valu) {
    return valu ? ftq_paged_decode_attention_valu(q_, qt, cache, bt, sl, bb, hq_, hkv_, d_, page_, mb_, nb_, signs,
                                                  signs, lev, lev, bk_, bv_, 0.1f, s_, ws_, wsb_, out_, ot, nullptr)
                : ftq_paged_decode_attention(q_, qt, cache, bt, sl, bb, hq_, hkv_, d_, page_, mb_, nb_, signs, signs,
                                             lev, lev, bk_, bv_, 0.1f, s_, ws_, wsb_, out_, ot, nullptr);
  };
  for (bool valu : {false, true}) {
    arg_error(attn(B_, hq, hkv, 64, page, mb, nb, bk, bv, S, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu), "paged d");
    arg_error(attn(B_, hq, 3, d, page, mb, nb, bk, bv, S, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu), "paged gqa");
    arg_error(attn(B_, hq, 0, d, page, mb, nb, bk, bv, S, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu), "paged hkv 0");
    arg_error(attn(B_, hq, hkv, d, page, mb, nb, 5, bv, S, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu), "paged bits");
    arg_error(attn(B_, hq, hkv, d, page, mb, nb, bk, bv, 0, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu), "paged S=0");
    arg_error(attn(B_, hq, hkv, d, page, mb, nb, bk, bv, 2000, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu),
              "paged S big");
    arg_error(attn(B_, hq, hkv, d, page, mb, nb, bk, bv, S, ws, wsb - 4, q, out, FTQ_BF16, FTQ_F32, valu),
              "paged short workspace");
    arg_error(attn(B_, hq, hkv, d, page, mb, nb, bk, bv, S, nullptr, wsb, q, out, FTQ_BF16, FTQ_F32, valu),
              "paged null workspace");
    arg_error(attn(B_, hq, hkv, d, page, mb, nb, bk, bv, S, ws, wsb, q + 2, out, FTQ_BF16, FTQ_F32, valu),
              "paged misaligned q");
    arg_error(attn(B_, hq, hkv, d, page, mb, nb, bk, bv, S, ws, wsb, q, out, 5, FTQ_F32, valu), "paged dtype");
    arg_error(attn(B_, hq, hkv, d, 24, mb, nb, bk, bv, S, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu), "paged page");
    arg_error(attn(-1, hq, hkv, d, page, mb, nb, bk, bv, S, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu), "paged B<0");
    arg_error(attn(B_, INT_MAX, 1, d, page, mb, nb, bk, bv, S, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu),
              "paged hq huge");
    EXPECT(attn(0, hq, hkv, d, page, mb, nb, bk, bv, S, nullptr, 0, nullptr, nullptr, FTQ_BF16, FTQ_F32, valu) == 0,
           "paged B=0");
    if (launch)
      hip_error(attn(B_, hq, hkv, d, page, mb, nb, bk, bv, S, ws, wsb, q, out, FTQ_BF16, FTQ_F32, valu),
                "paged launch");
  }
  if (launch) {
    hip_error(ftq_paged_store(kv, kv, FTQ_BF16, nt, hkv, d, signs, signs, bnd, bnd, bk, bv, slots, cache, page, nb,
                              nullptr),
              "paged_store launch");
    hip_error(attn(B_, hq, hkv, 256, page, mb, nb, 4, 2, 1, ws, wsb * 2, q, out, FTQ_F32, FTQ_F16, false),
              "paged launch d256");
  }
}

// v1 / raw slot caches: [num_blocks][block_size][hkv][slot]
static void v1(bool launch) {
  Buf B;
  const int nt = 5, hkv = 2, hq = 8, d = 128, bs = 16, kb = 3, vb = 3;
  const int64_t nb = 2, sh = 128, sp = sh * hkv, sbk = sp * bs;
  uint8_t* kv = B.get(nt * hkv * 256 * 4);
  float* mids = reinterpret_cast<float*>(B.get(256 * 4));
  int64_t* slots = reinterpret_cast<int64_t*>(B.get(nt * 8));
  uint8_t* cache = B.get(nb * sbk * 2 + 64);
  float* rot = reinterpret_cast<float*>(B.get(256 * 256 * 4));
  auto store = [&](int dd, int kb_, int vb_, int vr, int64_t n_, int h_, int64_t nb_, int bs_, int64_t sb_,
                   int64_t sp_, int64_t sh_, const void* k, uint8_t* c, const int64_t* sl) {
    return ftq_v1_store(k, k, FTQ_BF16, n_, h_, dd, mids, kb_, vb_, vr, sl, c, nb_, bs_, sb_, sp_, sh_, nullptr);
  };
  for (int dd : {0, 96, 512}) arg_error(store(dd, kb, vb, 0, nt, hkv, nb, bs, sbk, sp, sh, kv, cache, slots), "v1_store d");
  for (int w : {0, 5, 9}) arg_error(store(d, w, vb, 0, nt, hkv, nb, bs, sbk, sp, sh, kv, cache, slots), "v1_store kb");
  for (int vr : {-1, 8, INT_MAX})
    arg_error(store(d, kb, vb, vr, nt, hkv, nb, bs, sbk, sp, sh, kv, cache, slots), "v1_store flags");
  arg_error(store(d, kb, vb, 0, nt, hkv, nb, bs, sbk, sp, 32, kv, cache, slots), "v1_store stride_head < slot");
  arg_error(store(d, kb, vb, 0, nt, hkv, nb, bs, sbk, sh, sh, kv, cache, slots), "v1_store stride_pos");
  arg_error(store(d, kb, vb, 0, nt, hkv, nb, bs, sbk, sp, 130, kv, cache, slots), "v1_store stride % 4");
  // strides whose products overflow int64
  arg_error(store(d, kb, vb, 0, nt, hkv, nb, bs, INT64_MAX, INT64_MAX / 2, INT64_MAX / 4, kv, cache, slots),
            "v1_store huge strides");
  arg_error(store(d, kb, vb, 0, nt, 1 << 30, nb, bs, INT64_MAX, INT64_MAX / 8 * 4, INT64_MAX / 16 * 4, kv, cache, slots),
            "v1_store huge strides x heads");
  // each stride fits, but num_blocks * stride_block does not
  arg_error(store(d, kb, vb, 0, nt, hkv, 8, 1 << 30, INT64_MAX / 4 * 4, sp, sh, kv, cache, slots),
            "v1_store cache span past int64");
  arg_error(store(d, kb, vb, 0, nt, hkv, nb, bs, sbk, sp, sh, nullptr, cache, slots), "v1_store null key");
  arg_error(store(d, kb, vb, 0, nt, 0, nb, bs, sbk, sp, sh, kv, cache, slots), "v1_store heads");
  arg_error(store(d, kb, vb, 0, -1, hkv, nb, bs, sbk, sp, sh, kv, cache, slots), "v1_store n<0");
  arg_error(ftq_v1_store_blockdiag(kv, kv, FTQ_BF16, nt, hkv, d, mids, kb, vb, 0, slots, cache, nb, bs, sbk, sp, sh,
                                   rot, 5, nullptr),
            "v1_store_blockdiag block");
  arg_error(ftq_v1_store_rot(kv, kv, FTQ_BF16, nt, hkv, d, mids, kb, vb, 0, slots, cache, nb, bs, sbk, sp, sh,
                             reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(rot) + 2), nullptr),
            "v1_store_rot misaligned rotation");
  EXPECT(store(d, kb, vb, 0, 0, hkv, nb, bs, sbk, sp, sh, nullptr, nullptr, nullptr) == 0, "v1_store n=0");

  const int B_ = 2, mb = 2, S = 2;
  uint8_t* q = B.get(B_ * hq * d * 4);
  int32_t* bt = reinterpret_cast<int32_t*>(B.get(B_ * mb * 4));
  int32_t* sl = reinterpret_cast<int32_t*>(B.get(B_ * 4));
  float* cent = reinterpret_cast<float*>(B.get(256 * 4));
  float* lse = reinterpret_cast<float*>(B.get(B_ * hq * 4));
  const int64_t wsb = ftq_v1_workspace_bytes(B_, hq, d, S);
  EXPECT(wsb > 0, "v1 workspace bytes");
  uint8_t* ws = B.get(wsb);
  uint8_t* out = B.get(B_ * hq * d * 4);
  struct A {
    int bb, hq, hkv, d, kb, vb, vr, S, bs, mb;
    int64_t nb, sb, sp, sh, wsb;
    const void* q;
    void* out;
    void* ws;
    int qt, ot;
  };
  const A ok{B_, hq, hkv, d, kb, vb, 1, S, bs, mb, nb, sbk, sp, sh, wsb, q, out, ws, FTQ_BF16, FTQ_F32};
  auto run = [&](const A& a, int form) {
    switch (form) {
      case 0:
        return ftq_v1_decode_attention(a.q, a.qt, cache, a.nb, a.bs, a.sb, a.sp, a.sh, bt, a.mb, sl, nullptr, a.bb,
                                       a.hq, a.hkv, a.d, cent, a.kb, a.vb, 0.1f, a.vr, a.S, a.ws, a.wsb, a.out, a.ot,
                                       nullptr);
      case 1:
        return ftq_v1_decode_attention_lse(a.q, a.qt, cache, a.nb, a.bs, a.sb, a.sp, a.sh, bt, a.mb, sl, sl, a.bb,
                                           a.hq, a.hkv, a.d, cent, a.kb, a.vb, 0.1f, a.vr, a.S, a.ws, a.wsb, a.out,
                                           a.ot, lse, nullptr);
      case 2:
        return ftq_v1_decode_attention_rot(a.q, a.qt, cache, a.nb, a.bs, a.sb, a.sp, a.sh, bt, a.mb, sl, nullptr,
                                           a.bb, a.hq, a.hkv, a.d, cent, a.kb, a.vb, 0.1f, a.vr, a.S, a.ws, a.wsb,
                                           a.out, a.ot, lse, rot, nullptr);
      default:
        return ftq_v1_decode_attention_noalloc(a.q, a.qt, cache, a.nb, a.bs, a.sb, a.sp, a.sh, bt, a.mb, sl,
                                               nullptr, a.bb, a.hq, a.hkv, a.d, cent, a.kb, a.vb, 0.1f, a.vr, a.S,
                                               a.out, a.ot, nullptr);
    }
  };
  for (int form = 0; form < 4; ++form) {
    A a = ok;
    a.d = 96; arg_error(run(a, form), "v1 attn d");
    a = ok; a.kb = 5; arg_error(run(a, form), "v1 attn kb");
    a = ok; a.kb = 8; arg_error(run(a, form), "v1 attn kb 8 without fp8 keys");
    a = ok; a.vr = 16; arg_error(run(a, form), "v1 attn flags");
    a = ok; a.bs = 24; arg_error(run(a, form), "v1 attn block_size");
    a = ok; a.bs = 8192; arg_error(run(a, form), "v1 attn block_size big");
    a = ok; a.hkv = 3; arg_error(run(a, form), "v1 attn gqa");
    a = ok; a.hq = 64; a.hkv = 2; arg_error(run(a, form), "v1 attn gqa > 16");
    a = ok; a.S = 0; arg_error(run(a, form), "v1 attn S=0");
    a = ok; a.S = 1025; arg_error(run(a, form), "v1 attn S big");
    a = ok; a.sh = 64; arg_error(run(a, form), "v1 attn stride_head");
    a = ok; a.sp = INT64_MAX / 8 * 4; a.sb = INT64_MAX / 4 * 4; arg_error(run(a, form), "v1 attn stride_pos big");
    a = ok; a.sh = INT64_MAX / 4 * 4; a.sp = INT64_MAX / 4 * 4; a.sb = INT64_MAX / 4 * 4;
    arg_error(run(a, form), "v1 attn huge strides");
    a = ok; a.sb = INT64_MAX / 4 * 4; a.nb = 3; arg_error(run(a, form), "v1 attn cache span past int64");
    a = ok; a.qt = 3; arg_error(run(a, form), "v1 attn dtype");
    a = ok; a.mb = -1; arg_error(run(a, form), "v1 attn max_blocks");
    a = ok; a.bb = -1; arg_error(run(a, form), "v1 attn B<0");
    a = ok; a.nb = 0; arg_error(run(a, form), "v1 attn no blocks");
    a = ok; a.q = q + 4; arg_error(run(a, form), "v1 attn misaligned q");
    a = ok; a.out = nullptr; arg_error(run(a, form), "v1 attn null out");
    if (form < 3) {
      a = ok; a.wsb = wsb - 1; arg_error(run(a, form), "v1 attn short workspace");
      a = ok; a.ws = out + 4; arg_error(run(a, form), "v1 attn misaligned workspace");
    } else {
      a = ok; a.bb = 1 << 20; a.S = 1024; arg_error(run(a, form), "v1 noalloc beyond scratch");
    }
    a = ok; a.bb = 0; a.q = nullptr; a.out = nullptr; a.ws = nullptr; a.wsb = 0;
    if (form < 3) EXPECT(run(a, form) == 0, "v1 attn B=0 (form %d)", form);
    if (launch) {
      for (int S1 : {1, S}) {
        a = ok; a.S = S1; hip_error(run(a, form), "v1 attn launch");
        a.d = 256; a.wsb = ftq_v1_workspace_bytes(B_, hq, 256, S1);
        a.ws = B.get(a.wsb);
        a.out = B.get(B_ * hq * 256 * 4);
        a.q = B.get(B_ * hq * 256 * 4);
        a.sh = 256; a.sp = 512; a.sb = 512 * bs;
        hip_error(run(a, form), "v1 attn launch d256 (VALU kernel)");
      }
    }
  }
  if (launch) {
    for (int vr : {0, 1, 3})
      hip_error(store(d, kb, vb, vr, nt, hkv, nb, bs, sbk, sp, sh, kv, cache, slots), "v1_store launch");
    const int64_t f8 = (ftq_v1_slot_bytes_flags(d, 8, 8, FTQ_V1_KFP8) + 3) / 4 * 4;
    EXPECT(f8 > 0, "fp8 slot bytes");
    hip_error(store(d, 8, 8, FTQ_V1_KFP8, nt, hkv, nb, bs, f8 * hkv * bs, f8 * hkv, f8, kv, B.get(nb * f8 * hkv * bs),
                    slots),
              "v1_store fp8 launch");
    hip_error(ftq_v1_store_rot(kv, kv, FTQ_F16, nt, hkv, d, mids, kb, vb, 1, slots, cache, nb, bs, sbk, sp, sh, rot,
                               nullptr),
              "v1_store_rot launch");
    for (int blk : {2, 3, 4})
      hip_error(ftq_v1_store_blockdiag(kv, kv, FTQ_F32, nt, hkv, d, mids, kb, vb, 1, slots, cache, nb, bs, sbk, sp, sh,
                                       rot, blk, nullptr),
                "v1_store_blockdiag launch");
  }
}

static void raw(bool launch) {
  Buf B;
  const int nt = 5, hkv = 2, hq = 8, d = 128, bs = 16;
  const int64_t nb = 2, sh = 4 * d, sp = sh * hkv, sbk = sp * bs;
  uint8_t* kv = B.get(nt * hkv * d * 4);
  int64_t* slots = reinterpret_cast<int64_t*>(B.get(nt * 8));
  uint8_t* cache = B.get(nb * sbk + 64);
  arg_error(ftq_raw_store(kv, kv, FTQ_BF16, nt, hkv, 96, slots, cache, nb, bs, sbk, sp, sh, nullptr), "raw_store d");
  arg_error(ftq_raw_store(kv, kv, FTQ_BF16, nt, hkv, d, slots, cache, nb, bs, sbk, sp, 256, nullptr),
            "raw_store stride_head");
  arg_error(ftq_raw_store(kv, kv, FTQ_BF16, nt, hkv, d, slots, cache, nb, bs, INT64_MAX / 16 * 16,
                          INT64_MAX / 32 * 16, INT64_MAX / 64 * 16, nullptr),
            "raw_store huge strides");
  arg_error(ftq_raw_store(kv, kv, FTQ_BF16, nt, hkv, d, slots, cache + 8, nb, bs, sbk, sp, sh, nullptr),
            "raw_store misaligned cache");
  EXPECT(ftq_raw_store(nullptr, nullptr, FTQ_F32, 0, hkv, d, nullptr, nullptr, nb, bs, sbk, sp, sh, nullptr) == 0,
         "raw_store n=0");
  const int B_ = 2, mb = 2, S = 3;
  uint8_t* q = B.get(B_ * hq * d * 4);
  int32_t* bt = reinterpret_cast<int32_t*>(B.get(B_ * mb * 4));
  int32_t* sl = reinterpret_cast<int32_t*>(B.get(B_ * 4));
  float* lse = reinterpret_cast<float*>(B.get(B_ * hq * 4));
  const int64_t wsb = ftq_raw_workspace_bytes(B_, hq, d, S);
  uint8_t* ws = B.get(wsb);
  uint8_t* out = B.get(B_ * hq * d * 4);
  auto run = [&](int d_, int hq_, int hkv_, int S_, int64_t wsb_, int64_t sh_, int64_t sp_, int64_t sb_, int bs_,
                 const void* q_) {
    return ftq_raw_decode_attention_lse(q_, FTQ_BF16, cache, nb, bs_, sb_, sp_, sh_, bt, mb, sl, sl, B_, hq_, hkv_,
                                        d_, 0.1f, S_, ws, wsb_, out, FTQ_F32, lse, nullptr);
  };
  arg_error(run(96, hq, hkv, S, wsb, sh, sp, sbk, bs, q), "raw attn d");
  arg_error(run(d, 32, 2, S, wsb, sh, sp, sbk, bs, q), "raw attn gqa");
  arg_error(run(d, hq, hkv, 0, wsb, sh, sp, sbk, bs, q), "raw attn S");
  arg_error(run(d, hq, hkv, S, wsb - 1, sh, sp, sbk, bs, q), "raw attn workspace");
  arg_error(run(d, hq, hkv, S, wsb, 256, sp, sbk, bs, q), "raw attn stride_head");
  arg_error(run(d, hq, hkv, S, wsb, INT64_MAX / 64 * 16, INT64_MAX / 32 * 16, INT64_MAX / 16 * 16, bs, q),
            "raw attn huge strides");
  arg_error(run(d, hq, hkv, S, wsb, sh, sp, sbk, 48, q), "raw attn block_size");
  arg_error(run(d, hq, hkv, S, wsb, sh, sp, sbk, bs, q + 8), "raw attn misaligned q");
  if (launch) {
    hip_error(run(d, hq, hkv, S, wsb, sh, sp, sbk, bs, q), "raw attn launch");
    hip_error(ftq_raw_decode_attention(q, FTQ_F16, cache, nb, bs, sbk, sp, sh, bt, mb, sl, nullptr, B_, hq, hkv, d,
                                       0.1f, S, ws, wsb, out, FTQ_BF16, nullptr),
              "raw attn launch (no lse)");
    hip_error(ftq_raw_store(kv, kv, FTQ_BF16, nt, hkv, d, slots, cache, nb, bs, sbk, sp, sh, nullptr),
              "raw_store launch");
  }
}

int main() {
  int ndev = 0;
  const hipError_t e = hipGetDeviceCount(&ndev);
  const bool launch = e != hipSuccess || ndev == 0;  // host buffers reach the launch only without a GPU
  std::printf("[asan] devices visible: %d (%s); launch-path checks %s\n", e == hipSuccess ? ndev : 0,
              hipGetErrorString(e), launch ? "on" : "skipped");
  sizes();
  codebook_class();
  codec(launch);
  paged(launch);
  v1(launch);
  raw(launch);
  std::printf("[asan] %d checks, %d failed\n", g_checks, g_fail);
  return g_fail == 0 ? 0 : 1;
}
