// Host-side fuzzing of the library's CPU code under AddressSanitizer and
// UndefinedBehaviorSanitizer (TEST INFRASTRUCTURE; built by this folder's
// Makefile with the sanitizers on the host pass only, run by
// tests/test_sanitize.py).  No GPU call is made.
//
//  * SDEC headers (model_load_weights' header, model.cu:89-179): valid
//    headers of versions 1-5 mutated (bit flips, byte stores, random
//    fields, truncation) go through sde_model_read_header; its status and
//    fields must equal this file's own restatement of the header rules.
//  * Arena sizing: sde_model_weights_bytes of every parsed header and of
//    random configurations (negative, zero, huge fields) against a 128-bit
//    restatement of the tensor plan (model.cu:230-252).
//  * KV configurations: sde_kv_config_validate / sde_kv_pool_bytes on random
//    configurations around every limit, against a 128-bit restatement;
//    every accepted configuration's pool size must be representable.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>
#include <unistd.h>

#include "sde_paged_kv.h"

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint64_t next_u64() {  // xorshift64*
  g_state ^= g_state >> 12;
  g_state ^= g_state << 25;
  g_state ^= g_state >> 27;
  return g_state * 0x2545F4914F6CDD1Dull;
}
uint32_t rnd(uint32_t n) { return (uint32_t)(next_u64() % n); }

int g_failures = 0;
#define EXPECT(cond, ...)                                          \
  do {                                                             \
    if (!(cond)) {                                                 \
      if (++g_failures <= 20) {                                    \
        std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);  \
        std::fprintf(stderr, __VA_ARGS__);                         \
        std::fprintf(stderr, "\n");                                \
      }                                                            \
    }                                                              \
  } while (0)

// A value that stresses the header's bounds: small, a power of two near a
// limit, the limits themselves, or random.
uint32_t interesting_u32() {
  static const uint32_t v[] = {0u, 1u, 2u, 3u, 4u, 7u, 8u, 32u, 40u, 41u, 64u, 4096u,
                               (1u << 30) - 1, 1u << 30, (1u << 30) + 1, 1u << 31,
                               0x7FFFFFFFu, 0xFFFFFFFFu};
  return rnd(3) == 0 ? (uint32_t)next_u64() : v[rnd(sizeof(v) / sizeof(v[0]))];
}

void put_u32(std::vector<uint8_t>& b, uint32_t x) {
  uint8_t t[4];
  std::memcpy(t, &x, 4);
  b.insert(b.end(), t, t + 4);
}
void put_f32(std::vector<uint8_t>& b, float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  put_u32(b, u);
}

std::vector<uint8_t> valid_header(uint32_t version) {
  std::vector<uint8_t> b = {'S', 'D', 'E', 'C'};
  put_u32(b, version);
  const uint32_t nh = 1u << rnd(6), g = 1u << rnd(3);
  const uint32_t nkv = nh / g ? nh / g : 1;
  const uint32_t dph = 8u << rnd(5);
  put_u32(b, rnd(41));           // n_layers
  put_u32(b, nh * dph);          // d_model
  put_u32(b, nh);                // n_heads
  if (version >= 3) put_u32(b, nkv);
  put_u32(b, 4 * nh * dph);      // d_ff
  put_u32(b, 256 + rnd(200000));  // vocab
  if (version >= 2) put_f32(b, 500000.f);
  if (version >= 3) {
    put_u32(b, rnd(3));
    put_f32(b, 8.f);
  }
  if (version >= 4) put_u32(b, 0);
  if (version >= 5) put_u32(b, rnd(2));
  return b;
}

void mutate(std::vector<uint8_t>& b) {
  const int n = 1 + (int)rnd(4);
  for (int i = 0; i < n && !b.empty(); i++) {
    switch (rnd(5)) {
      case 0: b[rnd((uint32_t)b.size())] ^= (uint8_t)(1u << rnd(8)); break;
      case 1: b[rnd((uint32_t)b.size())] = (uint8_t)next_u64(); break;
      case 2: {  // a whole field after the magic
        if (b.size() >= 8) {
          const uint32_t f = 4 + 4 * rnd((uint32_t)(b.size() - 4) / 4);
          const uint32_t x = f == 4 ? rnd(7) : interesting_u32();
          std::memcpy(&b[f], &x, 4);
        }
        break;
      }
      case 3: b.resize(rnd((uint32_t)b.size() + 1)); break;
      default: b.push_back((uint8_t)next_u64()); break;
    }
  }
}

struct Expect {
  int status;
  sde_model_config cfg;
};

// The header rules, restated from the byte stream.
Expect restate(const std::vector<uint8_t>& b) {
  Expect e{};
  size_t at = 0;
  auto take = [&](void* dst) {
    if (at + 4 > b.size()) return false;
    std::memcpy(dst, &b[at], 4);
    at += 4;
    return true;
  };
  char magic[4];
  if (!take(magic)) return {SDE_ERR_IO, {}};
  if (std::memcmp(magic, "SDEC", 4) != 0) return {SDE_ERR_FORMAT, {}};
  uint32_t ver;
  if (!take(&ver)) return {SDE_ERR_IO, {}};
  if (ver < 1 || ver > 5) return {SDE_ERR_FORMAT, {}};
  uint32_t f[6];
  const int nf = ver <= 2 ? 5 : 6;
  for (int i = 0; i < nf; i++)
    if (!take(&f[i])) return {SDE_ERR_IO, {}};
  uint32_t L = f[0], d = f[1], nh = f[2], nkv, dff, V;
  if (ver <= 2) {
    nkv = nh, dff = f[3], V = f[4];
  } else {
    nkv = f[3], dff = f[4], V = f[5];
  }
  float theta = 10000.f, sf = 1.f;
  int32_t st = 0, at_type = 0, bias = 0;
  if (ver >= 2 && !take(&theta)) return {SDE_ERR_IO, {}};
  if (ver >= 3 && (!take(&st) || !take(&sf))) return {SDE_ERR_IO, {}};
  if (ver >= 4 && !take(&at_type)) return {SDE_ERR_IO, {}};
  if (ver >= 5 && !take(&bias)) return {SDE_ERR_IO, {}};
  if (L > 40 || nh == 0 || nkv == 0 || d % nh != 0 || nh % nkv != 0) return {SDE_ERR_FORMAT, {}};
  if (d > (1u << 30) || dff > (1u << 30) || V > (1u << 30)) return {SDE_ERR_FORMAT, {}};
  e.status = SDE_OK;
  e.cfg.n_layers = (int32_t)L;
  e.cfg.d_model = (int32_t)d;
  e.cfg.n_heads = (int32_t)nh;
  e.cfg.n_kv_heads = (int32_t)nkv;
  e.cfg.d_ff = (int32_t)dff;
  e.cfg.vocab_size = (int32_t)V;
  e.cfg.rope_theta = theta;
  e.cfg.rope_scaling_type = st;
  e.cfg.rope_scaling_factor = sf;
  e.cfg.attention_type = at_type;
  e.cfg.has_qkv_bias = bias != 0;
  e.cfg.version = (int32_t)ver;
  return e;
}

bool same_bits(float a, float b) { return std::memcmp(&a, &b, 4) == 0; }

// The arena size of a configuration (model.cu:230-252 tensor order; each
// tensor 256-byte aligned), 0 when invalid or not representable.
size_t restate_arena(const sde_model_config& c) {
  if (c.n_layers < 0 || c.n_layers > 40 || c.d_model <= 0 || c.n_heads <= 0 ||
      c.n_kv_heads <= 0 || c.d_model % c.n_heads != 0 || c.n_heads % c.n_kv_heads != 0 ||
      c.d_ff < 0 || c.vocab_size < 0)
    return 0;
  using u128 = unsigned __int128;
  const u128 d = (u128)c.d_model, kd = (u128)c.n_kv_heads * (u128)(c.d_model / c.n_heads),
             dff = (u128)c.d_ff, V = (u128)c.vocab_size;
  std::vector<u128> n = {V * d, d, d * V};
  for (int l = 0; l < c.n_layers; l++) {
    for (u128 x : {d, d * d, d * kd, d * kd, d * d, d, d * dff, d * dff, dff * d}) n.push_back(x);
    if (c.has_qkv_bias)
      for (u128 x : {d, kd, kd}) n.push_back(x);
  }
  u128 total = 0;
  for (u128 x : n) {
    if (x > (u128)UINT32_MAX) return 0;
    total += (x * 2 + 255) / 256 * 256;
  }
  return total > (u128)SIZE_MAX ? 0 : (size_t)total;
}

void fuzz_headers(int iters) {
  char path[] = "/tmp/sde_fuzz_XXXXXX";
  const int fd = mkstemp(path);
  if (fd < 0) {
    std::perror("mkstemp");
    std::exit(2);
  }
  close(fd);
  int ok = 0;
  for (int i = 0; i < iters; i++) {
    std::vector<uint8_t> b = valid_header(1 + rnd(5));
    if (i % 8 != 0) mutate(b);  // every 8th header stays valid
    FILE* f = std::fopen(path, "wb");
    if (!b.empty()) std::fwrite(b.data(), 1, b.size(), f);
    std::fclose(f);
    sde_model_config cfg;
    std::memset(&cfg, 0xA5, sizeof(cfg));
    const int st = sde_model_read_header(path, &cfg);
    const Expect e = restate(b);
    EXPECT(st == e.status, "header %d: status %d, restated %d", i, st, e.status);
    if (st != SDE_OK || e.status != SDE_OK) continue;
    ok++;
    const sde_model_config& x = e.cfg;
    EXPECT(cfg.n_layers == x.n_layers && cfg.d_model == x.d_model && cfg.n_heads == x.n_heads &&
               cfg.n_kv_heads == x.n_kv_heads && cfg.d_ff == x.d_ff &&
               cfg.vocab_size == x.vocab_size && cfg.version == x.version &&
               cfg.rope_scaling_type == x.rope_scaling_type &&
               cfg.attention_type == x.attention_type && cfg.has_qkv_bias == x.has_qkv_bias &&
               same_bits(cfg.rope_theta, x.rope_theta) &&
               same_bits(cfg.rope_scaling_factor, x.rope_scaling_factor),
           "header %d: fields differ", i);
    const size_t bytes = sde_model_weights_bytes(&cfg);
    EXPECT(bytes == restate_arena(cfg), "header %d: arena %zu, restated %zu", i, bytes,
           restate_arena(cfg));
  }
  std::remove(path);
  EXPECT(ok > iters / 16, "too few headers parsed (%d)", ok);
  std::printf("sdec headers: %d fuzzed, %d parsed\n", iters, ok);
}

int32_t interesting_i32() {
  static const int32_t v[] = {INT32_MIN, -1, 0, 1, 2, 3, 8, 16, 40, 41, 64, 1024, 1025,
                              1 << 20, 1 << 30, INT32_MAX - 1, INT32_MAX};
  return rnd(3) == 0 ? (int32_t)next_u64() : v[rnd(sizeof(v) / sizeof(v[0]))];
}

void fuzz_arena(int iters) {
  for (int i = 0; i < iters; i++) {
    sde_model_config c{};
    c.n_layers = rnd(2) ? (int32_t)rnd(42) : interesting_i32();
    c.n_heads = rnd(2) ? (int32_t)(1u << rnd(7)) : interesting_i32();
    c.n_kv_heads = rnd(2) && c.n_heads > 0 ? c.n_heads >> rnd(4) : interesting_i32();
    c.d_model = rnd(2) && c.n_heads > 0 && c.n_heads <= (1 << 20)
                    ? c.n_heads * (int32_t)(1u << rnd(8))
                    : interesting_i32();
    c.d_ff = interesting_i32();
    c.vocab_size = interesting_i32();
    c.has_qkv_bias = (int32_t)rnd(2);
    const size_t got = sde_model_weights_bytes(&c);
    EXPECT(got == restate_arena(c), "config %d: arena %zu, restated %zu", i, got,
           restate_arena(c));
  }
  EXPECT(sde_model_weights_bytes(nullptr) == 0, "null config");
  std::printf("arena sizing: %d configurations\n", iters);
}

void fuzz_kv(int iters) {
  int valid = 0;
  for (int i = 0; i < iters; i++) {
    sde_kv_config c{};
    c.n_layers = rnd(2) ? 1 + (int32_t)rnd(128) : interesting_i32();
    c.kv_dim = rnd(2) ? (int32_t)(64u << rnd(6)) : interesting_i32();
    c.max_blocks_per_layer = rnd(2) ? 1 + (int32_t)rnd(1 << 16) : interesting_i32();
    c.block_size = rnd(2) ? (int32_t)(1u << rnd(11)) : interesting_i32();
    c.pool_blocks = rnd(2) ? 0 : interesting_i32();
    // The rules: positive sizes, block_size <= 1024, pool of at least one
    // layer's blocks that fits int32, positions that fit int32, and a pool
    // whose byte size fits ptrdiff_t.
    using i128 = __int128;
    bool want = c.n_layers >= 1 && c.kv_dim >= 1 && c.max_blocks_per_layer >= 1 &&
                c.block_size >= 1 && c.block_size <= 1024 && c.pool_blocks >= 0;
    i128 pool = 0;
    if (want) {
      pool = c.pool_blocks ? (i128)c.pool_blocks : (i128)c.n_layers * c.max_blocks_per_layer;
      want = pool <= INT32_MAX && pool >= c.max_blocks_per_layer &&
             (i128)c.max_blocks_per_layer * c.block_size <= INT32_MAX &&
             pool * 2 * c.block_size * c.kv_dim * 2 <= (i128)PTRDIFF_MAX;
    }
    const int st = sde_kv_config_validate(&c);
    const size_t bytes = sde_kv_pool_bytes(&c);
    EXPECT((st == SDE_OK) == want, "kv config %d (%d %d %d %d %d): status %d", i, c.n_layers,
           c.kv_dim, c.max_blocks_per_layer, c.block_size, c.pool_blocks, st);
    if (want && st == SDE_OK) {
      valid++;
      EXPECT((i128)bytes == pool * 2 * c.block_size * c.kv_dim * 2, "kv config %d: bytes %zu",
             i, bytes);
    } else {
      EXPECT(bytes == 0, "kv config %d: invalid but %zu bytes", i, bytes);
    }
  }
  EXPECT(sde_kv_config_validate(nullptr) != SDE_OK && sde_kv_pool_bytes(nullptr) == 0,
         "null kv config");
  std::printf("kv configurations: %d checked, %d valid\n", iters, valid);
}

}  // namespace

int main(int argc, char** argv) {
  const int scale = argc > 1 ? std::atoi(argv[1]) : 1;
  g_state ^= (uint64_t)(argc > 2 ? std::atoll(argv[2]) : 1);
  fuzz_headers(20000 * scale);
  fuzz_arena(200000 * scale);
  fuzz_kv(200000 * scale);
  if (g_failures) {
    std::fprintf(stderr, "%d failures\n", g_failures);
    return 1;
  }
  std::printf("host fuzz: all checks passed\n");
  return 0;
}
