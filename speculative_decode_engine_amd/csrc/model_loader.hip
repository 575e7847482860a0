// SDEC weight files onto the GPU: the reference's model_load_weights
// (model.cu:68-260; format written by tools/export_model.py:19-35, 170-210)
// behind the C-ABI of sde_paged_kv.h.
//
// The header is validated field by field as the reference does.  The
// weights go to one device arena (tensors 256-byte aligned, so the GEMV's
// 16-byte row loads and the attention's pool-independent pointers stay
// aligned); the file is streamed through two pinned staging buffers on a
// stream of its own: while one buffer's host-to-device copy runs, the
// next chunk of the file is read into the other.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include "sde_paged_kv.h"

struct sde_model {
  sde_model_config cfg;
  int device = 0;
  void* arena = nullptr;
  size_t arena_bytes = 0;
  sde_model_globals globals{};
  std::vector<sde_layer_weights> layers;
};

namespace {

constexpr int kMaxLayers = 40;                 // MAX_LAYERS, config.h:21
constexpr size_t kAlign = 256;
constexpr size_t kStageBytes = 32u << 20;       // per pinned staging buffer

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct File {
  FILE* f = nullptr;
  explicit File(const char* path) : f(path ? std::fopen(path, "rb") : nullptr) {}
  ~File() {
    if (f) std::fclose(f);
  }
  bool read(void* dst, size_t n) { return std::fread(dst, 1, n, f) == n; }
};

int kv_dim_of(const sde_model_config& c) { return c.n_kv_heads * (c.d_model / c.n_heads); }

// model.cu:89-179 (+ guards against zero head counts, which the reference
// would divide by).
int parse_header(File& file, sde_model_config* cfg) {
  char magic[4];
  if (!file.read(magic, 4)) return SDE_ERR_IO;
  if (std::memcmp(magic, "SDEC", 4) != 0) return SDE_ERR_FORMAT;
  uint32_t version = 0;
  if (!file.read(&version, 4)) return SDE_ERR_IO;
  if (version < 1u || version > 5u) return SDE_ERR_FORMAT;
  uint32_t n_layers, d_model, n_heads, n_kv_heads, d_ff, vocab;
  if (version <= 2u) {
    uint32_t h[5];
    if (!file.read(h, sizeof(h))) return SDE_ERR_IO;
    n_layers = h[0], d_model = h[1], n_heads = h[2], d_ff = h[3], vocab = h[4];
    n_kv_heads = n_heads;  // expanded GQA
  } else {
    uint32_t h[6];
    if (!file.read(h, sizeof(h))) return SDE_ERR_IO;
    n_layers = h[0], d_model = h[1], n_heads = h[2], n_kv_heads = h[3], d_ff = h[4],
    vocab = h[5];
  }
  float rope_theta = 10000.f;
  if (version >= 2u && !file.read(&rope_theta, 4)) return SDE_ERR_IO;
  int32_t scaling_type = 0;
  float scaling_factor = 1.f;
  if (version >= 3u && (!file.read(&scaling_type, 4) || !file.read(&scaling_factor, 4)))
    return SDE_ERR_IO;
  int32_t attention_type = 0;
  if (version >= 4u && !file.read(&attention_type, 4)) return SDE_ERR_IO;
  int32_t has_bias = 0;
  if (version >= 5u && !file.read(&has_bias, 4)) return SDE_ERR_IO;

  if (n_layers > (uint32_t)kMaxLayers) return SDE_ERR_FORMAT;
  if (n_heads == 0 || n_kv_heads == 0 || d_model % n_heads != 0 || n_heads % n_kv_heads != 0)
    return SDE_ERR_FORMAT;
  if (d_model > (1u << 30) || d_ff > (1u << 30) || vocab > (1u << 30)) return SDE_ERR_FORMAT;
  cfg->n_layers = (int32_t)n_layers;
  cfg->d_model = (int32_t)d_model;
  cfg->n_heads = (int32_t)n_heads;
  cfg->n_kv_heads = (int32_t)n_kv_heads;
  cfg->d_ff = (int32_t)d_ff;
  cfg->vocab_size = (int32_t)vocab;
  cfg->rope_theta = rope_theta;
  cfg->rope_scaling_type = scaling_type;
  cfg->rope_scaling_factor = scaling_factor;
  cfg->attention_type = attention_type;
  cfg->has_qkv_bias = has_bias != 0;
  cfg->version = version;
  return SDE_OK;
}

// The tensors of a file in order (model.cu:230-252): destination slot and
// element count.
struct TensorSlot {
  const uint16_t** dst;
  size_t n;
};

std::vector<TensorSlot> tensor_plan(sde_model* m) {
  const sde_model_config& c = m->cfg;
  const size_t d = (size_t)c.d_model, kd = (size_t)kv_dim_of(c), dff = (size_t)c.d_ff,
               V = (size_t)c.vocab_size;
  std::vector<TensorSlot> t;
  t.push_back({&m->globals.token_embedding, V * d});
  t.push_back({&m->globals.rms_final_weight, d});
  t.push_back({&m->globals.output_proj, d * V});
  m->layers.assign((size_t)c.n_layers, sde_layer_weights{});
  for (auto& L : m->layers) {
    t.push_back({&L.rms_attn_weight, d});
    t.push_back({&L.Wq, d * d});
    t.push_back({&L.Wk, d * kd});
    t.push_back({&L.Wv, d * kd});
    t.push_back({&L.Wo, d * d});
    t.push_back({&L.rms_mlp_weight, d});
    t.push_back({&L.W_gate, d * dff});
    t.push_back({&L.W_up, d * dff});
    t.push_back({&L.W_down, dff * d});
    if (c.has_qkv_bias) {
      t.push_back({&L.Wq_bias, d});
      t.push_back({&L.Wk_bias, kd});
      t.push_back({&L.Wv_bias, kd});
    }
  }
  return t;
}

// Arena bytes of a plan.  SDE_ERR_FORMAT when a tensor has more elements
// than the file's uint32 count can state (no file can match it) or the sum
// would wrap: the header bounds (each dimension up to 2^30) allow both, and
// the arena is allocated from this sum before any tensor is read.
int arena_bytes_of(const std::vector<TensorSlot>& t, size_t* bytes) {
  size_t b = 0;
  for (const auto& s : t) {
    if (s.n > (size_t)UINT32_MAX) return SDE_ERR_FORMAT;
    const size_t add = align_up(s.n * 2);
    if (add > SIZE_MAX - b) return SDE_ERR_FORMAT;
    b += add;
  }
  *bytes = b;
  return SDE_OK;
}

// Two pinned buffers and a stream: chunk i is read while chunk i-1 copies.
class Stager {
 public:
  int init() {
    if (hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking) != hipSuccess) return SDE_ERR_HIP;
    for (int b = 0; b < 2; b++) {
      if (hipHostMalloc(&buf_[b], kStageBytes, hipHostMallocDefault) != hipSuccess ||
          hipEventCreateWithFlags(&done_[b], hipEventDisableTiming) != hipSuccess)
        return SDE_ERR_HIP;
      pending_[b] = false;
    }
    return SDE_OK;
  }
  ~Stager() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (int b = 0; b < 2; b++) {
      if (buf_[b]) (void)hipHostFree(buf_[b]);
      if (done_[b]) (void)hipEventDestroy(done_[b]);
    }
    if (stream_) (void)hipStreamDestroy(stream_);
  }
  // n bytes of the file to device address dst.
  int copy(File& file, char* dst, size_t n) {
    while (n > 0) {
      const size_t c = n < kStageBytes ? n : kStageBytes;
      if (pending_[next_] && hipEventSynchronize(done_[next_]) != hipSuccess) return SDE_ERR_HIP;
      if (!file.read(buf_[next_], c)) return SDE_ERR_IO;
      if (hipMemcpyAsync(dst, buf_[next_], c, hipMemcpyHostToDevice, stream_) != hipSuccess ||
          hipEventRecord(done_[next_], stream_) != hipSuccess)
        return SDE_ERR_HIP;
      pending_[next_] = true;
      next_ ^= 1;
      dst += c;
      n -= c;
    }
    return SDE_OK;
  }
  int finish() { return hipStreamSynchronize(stream_) == hipSuccess ? SDE_OK : SDE_ERR_HIP; }

 private:
  hipStream_t stream_ = nullptr;
  void* buf_[2] = {nullptr, nullptr};
  hipEvent_t done_[2] = {nullptr, nullptr};
  bool pending_[2] = {false, false};
  int next_ = 0;
};

bool valid_config(const sde_model_config* c) {
  return c && c->n_layers >= 0 && c->n_layers <= kMaxLayers && c->d_model > 0 &&
         c->n_heads > 0 && c->n_kv_heads > 0 && c->d_model % c->n_heads == 0 &&
         c->n_heads % c->n_kv_heads == 0 && c->d_ff >= 0 && c->vocab_size >= 0;
}

}  // namespace

extern "C" {

int sde_model_read_header(const char* path, sde_model_config* cfg) {
  if (!path || !cfg) return SDE_ERR_INVALID_ARGUMENT;
  File file(path);
  if (!file.f) return SDE_ERR_IO;
  return parse_header(file, cfg);
}

size_t sde_model_weights_bytes(const sde_model_config* cfg) {
  if (!valid_config(cfg)) return 0;
  try {  // no C++ exception crosses the C-ABI
    sde_model m;
    m.cfg = *cfg;
    size_t bytes = 0;
    return arena_bytes_of(tensor_plan(&m), &bytes) == SDE_OK ? bytes : 0;
  } catch (...) {
    return 0;
  }
}

int sde_model_load(const char* path, sde_model** out, sde_model_config* cfg_out) {
  if (!path || !out) return SDE_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  File file(path);
  if (!file.f) return SDE_ERR_IO;
  sde_model* m = new (std::nothrow) sde_model();
  if (!m) return SDE_ERR_HIP;
  int st = parse_header(file, &m->cfg);
  if (st != SDE_OK) {
    delete m;
    return st;
  }
  if (hipGetDevice(&m->device) != hipSuccess) {
    delete m;
    return SDE_ERR_NO_DEVICE;
  }
  std::vector<TensorSlot> plan;
  try {  // host allocation failure: no C++ exception crosses the C-ABI
    plan = tensor_plan(m);
  } catch (...) {
    delete m;
    return SDE_ERR_HIP;
  }
  st = arena_bytes_of(plan, &m->arena_bytes);
  if (st != SDE_OK) {
    delete m;
    return st;
  }
  if (m->arena_bytes > 0 && hipMalloc(&m->arena, m->arena_bytes) != hipSuccess) {
    delete m;
    return SDE_ERR_HIP;
  }
  {
    Stager stage;
    st = stage.init();
    char* at = static_cast<char*>(m->arena);
    for (size_t i = 0; st == SDE_OK && i < plan.size(); i++) {
      uint32_t n = 0;
      if (!file.read(&n, 4)) {
        st = SDE_ERR_IO;
      } else if ((size_t)n != plan[i].n) {
        st = SDE_ERR_FORMAT;
      } else {
        *plan[i].dst = reinterpret_cast<const uint16_t*>(at);
        st = stage.copy(file, at, plan[i].n * 2);
        at += align_up(plan[i].n * 2);
      }
    }
    const int fin = stage.finish();
    if (st == SDE_OK) st = fin;
  }
  if (st != SDE_OK) {
    if (m->arena) (void)hipFree(m->arena);
    delete m;
    return st;
  }
  if (cfg_out) *cfg_out = m->cfg;
  *out = m;
  return SDE_OK;
}

int sde_model_get_config(const sde_model* model, sde_model_config* cfg) {
  if (!model || !cfg) return SDE_ERR_INVALID_ARGUMENT;
  *cfg = model->cfg;
  return SDE_OK;
}

int sde_model_get_layer(const sde_model* model, int layer, sde_layer_weights* out) {
  if (!model || !out || layer < 0 || layer >= model->cfg.n_layers) return SDE_ERR_INVALID_ARGUMENT;
  *out = model->layers[(size_t)layer];
  return SDE_OK;
}

int sde_model_get_globals(const sde_model* model, sde_model_globals* out) {
  if (!model || !out) return SDE_ERR_INVALID_ARGUMENT;
  *out = model->globals;
  return SDE_OK;
}

int sde_model_free(sde_model* model) {
  if (!model) return SDE_ERR_INVALID_ARGUMENT;
  int st = SDE_OK;
  if (model->arena && hipFree(model->arena) != hipSuccess) st = SDE_ERR_HIP;
  delete model;
  return st;
}

}  // extern "C"
