// The persistent speculative decoding loop on gfx950: one cooperative
// launch runs round after round of self-speculative decoding over a paged
// KV cache -- greedy, or speculative sampling -- with every token decision
// and every rewind made on the device.
//
// Reference (arkhamHack/speculative_decode_engine):
//   cuda/src/kernels.cu:2864-3106  megakernel_speculative_kernel: draft k
//                                  tokens, verify the window [last, drafts]
//                                  in one batched pass, greedy accept,
//                                  rewind target / draft seq_len
//   cuda/src/kernels.cu:3108-3481  megakernel_speculative_stochastic_kernel:
//                                  drafts sampled at a draft temperature
//                                  (adapted per round toward a target
//                                  acceptance), speculative-sampling accept
//                                  with the corrected or bonus sample
//   cuda/src/model.cu:838-890      self-speculative verify: layers
//                                  [n_draft, n_layers) over the saved
//                                  hiddens of the prefix layers
//   cuda/src/kernels.cu:2727-2739  the megakernel's attention (block 0)
//
// What differs from the reference by design: attention runs on every block
// (device_flash_attention_gqa_grid) instead of block 0, the output head on
// every block (over a panel-packed copy of its weights, whole output
// columns per block, with the greedy argmax reduced from per-panel
// candidates), and the window's appends on one block per window row.  The model is the paged-KV path's own: layer l
// of token t reads q, k, v rows from per-layer embedding tables, q adds the
// previous layer's attention output (a residual stream through the
// attention), and fp16 head weights map the last layer's attention output to
// logits.  K/V bytes therefore depend on (token, position) alone, so greedy
// speculation must leave exactly the greedy decoder's bytes below seq_len.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "sde/attention_device.hpp"
#include "sde/matvec_packed.hpp"
#include "sde/spec_device.hpp"
#include "sde_internal.hpp"

namespace sde {
namespace loop {

constexpr int kThreads = 512;
constexpr uint32_t kSpinLimit = 1u << 18;  // polls of a grid barrier before it gives up
constexpr int kMaxWindow = 16;  // k + 1 rows (two passes of the packed head)

// Words of d_state.
enum : int {
  kAnchor = 0,    // in: the last emitted token (not yet in the cache); out: updated
  kEmitted = 1,   // tokens written to d_emitted
  kRounds = 2,    // rounds run
  kStatus = 3,    // first error (SDE_OK when none)
  kProposed = 4,  // drafts proposed
  kAccepted = 5,  // drafts accepted
  kTemp = 6,      // sampling loop: the draft temperature (float bits), in and out
  kEwma = 7,      // sampling loop: the acceptance-rate average (float bits, < 0: none yet)
  kStateWords = 8
};

// Grid barrier words: the XCDs' leaders' arrivals and the generation, then
// per XCD (on a 128-byte line of its own) the arrivals of its blocks and the
// number of blocks the launch placed on it.
enum : int {
  kBarArrive = 0,
  kBarGen = 1,
  kBarXcd = 32,   // + 32 x: arrivals of XCD x's blocks
  kBarCount = 48, // + 32 x: blocks on XCD x (counted once, at the kernel's start)
  kBarWords = 32 * 9
};
constexpr size_t kBarBytes = kBarWords * sizeof(uint32_t);

// One model of the loop over its cache: the target (whose prefix layers
// also draft in the self-speculative form), or a separate draft model.
struct Side {
  sde_kv_view kv;
  sde_loop_model m;
  int d;    // n_heads * head_dim
  int cap;  // positions every layer's table maps
  const uint4* head_packed;  // the head's panel-packed copy (made by the launch)
};

struct LoopArgs {
  Side t;      // the target model and cache
  Side dr;     // the draft model and its cache (when `two`)
  int two;     // a separate draft model and cache (kernels.cu:2864-2875, shared_kv false)
  int eos;     // stop after a round whose bonus is this token; < 0: never
  int k;
  int n_draft;
  int max_new;
  int32_t* state;
  int32_t* emitted;   // [max_new + k]
  int32_t* accepted;  // [max_new], per round
  float* q_buf;       // [k+1][d] (the separate q phase of the generic shapes)
  float* h_buf;       // two [k+1][d] halves: layer l's attention output in half l % 2
  size_t h_half;      // floats per half
  int fused;          // the attention builds the window itself (tile-path shapes)
  float* logits;      // [k+1][vocab]
  int32_t* tokens;    // [2(k+1) + 2]: window tokens, the target's tokens, kCatchUp, kDone
  void* attn_ws;
  size_t attn_ws_bytes;
  uint2* cand;               // [kMaxWindow][panels]: each panel's (max logit, column) per row
  uint32_t* cand_arrivals;   // the head's items done (zero at rest)
  uint32_t* bar;  // grid barrier words (kBar*), zero at rest
  // speculative sampling (sde_spec_loop_stochastic)
  float* dlogits;      // [k][vocab]: the draft rows' logits
  int32_t* sres;       // [k+5]: the acceptance's result
  int32_t* dres;       // [8]: a draft sample's result, then a scratch seq_len word
  uint32_t* sscratch;  // the stochastic device function's workspace (counters zero at rest)
  uint64_t* offset;    // the random stream's call index (device, caller-owned)
  sde_loop_sampling smp;
};

// Workspace layout: attention workspace (counters first), the loop's
// buffers, then the heads' packed copies, each 256-byte aligned.
struct Layout {
  size_t attn, q, h, logits, tokens, bar, dlogits, sres, dres, sscratch, head, dhead, cand, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// A model's attention shape and its cache's positions.
struct Shape {
  int nh, nkv, dph, cap;
};

// tokens[] words after the window's and the target's tokens.
__host__ __device__ inline int catch_up_slot(int k) { return 2 * (k + 1); }  // the draft catch-up's token
__host__ __device__ inline int done_slot(int k) { return 2 * (k + 1) + 1; }  // 1 once an EOS bonus is out

inline Layout layout(const Shape& t, const Shape* d, int vocab, int k) {
  Layout l;
  const int M = k + 1;
  const size_t dt = (size_t)t.nh * t.dph;
  const size_t dd = d ? (size_t)d->nh * d->dph : 0;
  const size_t dmax = dt > dd ? dt : dd;
  // The target's window calls and the draft's one-query calls share the
  // attention workspace (a grid barrier separates them).
  size_t ws = grid_attention_workspace_size(t.nh, t.nkv, t.dph, M, t.cap);
  if (d) {
    const size_t wd = grid_attention_workspace_size(d->nh, d->nkv, d->dph, 1, d->cap);
    if (wd > ws) ws = wd;
  }
  l.attn = 0;
  l.q = align256(ws);
  l.h = l.q + align256(M * dmax * sizeof(float));
  l.logits = l.h + align256(2 * M * dmax * sizeof(float));
  l.tokens = l.logits + align256((size_t)M * vocab * sizeof(float));
  l.bar = l.tokens + align256((2 * M + 2) * sizeof(int32_t));
  l.dlogits = l.bar + align256(kBarBytes);
  l.sres = l.dlogits + align256((size_t)(k > 0 ? k : 1) * vocab * sizeof(float));
  l.dres = l.sres + align256((k + 5) * sizeof(int32_t));
  l.sscratch = l.dres + 256;
  l.head = l.sscratch + align256(spec_stochastic_workspace_size());
  l.dhead = l.head + align256(mvp::packed_shape((int)dt, vocab).units * 16);
  l.cand = l.dhead + (d ? align256(mvp::packed_shape((int)dd, vocab).units * 16) : 0);
  l.total = l.cand + 256 + align256((size_t)kMaxWindow * (vocab / 8) * sizeof(uint2));
  return l;
}

__device__ __forceinline__ uint32_t xcd_id() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x & 7u;
}

// Whether an error has been recorded (the launch is ending).
__device__ __forceinline__ bool failed(const LoopArgs& a) {
  return __hip_atomic_load(a.state + kStatus, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) !=
         SDE_OK;
}

// Waits for the barrier generation to move past `gen`.  Returns at once
// once an error is recorded, so after one broken barrier (which records
// SDE_ERR_HIP when its spin budget runs out) every later wait of the launch
// returns immediately instead of spending a budget of its own: the blocks
// reach the next round check, see the status and leave together.
__device__ __forceinline__ void wait_generation(const LoopArgs& a, uint32_t gen) {
  uint32_t polls = 0;
  while (__hip_atomic_load(a.bar + kBarGen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen) {
    if (failed(a)) break;
    if (++polls == kSpinLimit) {
      atomicCAS(reinterpret_cast<int*>(a.state + kStatus), SDE_OK, SDE_ERR_HIP);
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Grid barrier between the loop's phases, two levels deep.  Each wave
// waits for its stores (s_waitcnt: acknowledged by its XCD's L2), the block
// synchronizes, and one thread per block arrives on its XCD's counter.  The
// last block of an XCD to arrive writes that XCD's L2 back to the device
// coherence point with one device-scope release fence -- every block of the
// XCD has its stores in that L2 by then -- and arrives on the grid counter;
// the last XCD leader moves the generation.  Every block then waits for the
// generation to move and drops stale lines of its CU's L1 and its XCD's L2
// with a device-scope acquire fence.  One writeback per XCD instead of one
// per block: measured on MI355X with 256 blocks of 512 threads, 6.1 us per
// barrier and phase against 12.7 for a release fence in every block (9.4 vs
// 24.9 with 16 KiB written per block), and no stale read in either.  A wait
// gives up after kSpinLimit polls and records SDE_ERR_HIP, so a broken
// barrier ends the launch instead of hanging it; once a status is recorded
// the barrier does not wait at all (every later round check sees the status
// and exits; the barrier words are cleared by the next launch's init).
__device__ __forceinline__ void barrier(const LoopArgs& a) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0 && !failed(a)) {
    const uint32_t gen =
        __hip_atomic_load(a.bar + kBarGen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t x = xcd_id();
    uint32_t* xa = a.bar + kBarXcd + 32 * x;
    const uint32_t n_x =
        __hip_atomic_load(a.bar + kBarCount + 32 * x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t p = __hip_atomic_fetch_add(xa, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (p == n_x - 1) {
      __hip_atomic_store(xa, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      uint32_t n_xcds = 0;
      for (int i = 0; i < 8; i++)
        n_xcds += __hip_atomic_load(a.bar + kBarCount + 32 * i, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) > 0u;
      const uint32_t q =
          __hip_atomic_fetch_add(a.bar + kBarArrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (q == n_xcds - 1) {
        __hip_atomic_store(a.bar + kBarArrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.bar + kBarGen, gen + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        wait_generation(a, gen);
      }
    } else {
      wait_generation(a, gen);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

// At the kernel's start: every block counts itself on its XCD, then a
// one-level barrier (a release fence in every block) publishes the counts.
__device__ __forceinline__ void register_blocks(const LoopArgs& a) {
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(a.bar + kBarCount + 32 * xcd_id(), 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t gen =
        __hip_atomic_load(a.bar + kBarGen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const uint32_t p =
        __hip_atomic_fetch_add(a.bar + kBarArrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (p == gridDim.x * gridDim.y * gridDim.z - 1) {
      __hip_atomic_store(a.bar + kBarArrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.bar + kBarGen, gen + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      wait_generation(a, gen);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

// The loop's control words (seq_len, tokens emitted, status) are written
// and read with device-scope atomics, so every block takes the same exits
// whatever the caches hold: a block that left the loop early would leave the
// others waiting at a grid barrier.
__device__ __forceinline__ int load_word(const int32_t* p) {
  return __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

__device__ __forceinline__ void store_word(int32_t* p, int x) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void note_error(const LoopArgs& a, int st) {
  if (st != SDE_OK && threadIdx.x == 0)
    atomicCAS(reinterpret_cast<int*>(a.state + kStatus), SDE_OK, st);
}

// Layer l's attention output rows (layer l - 1's are layer l's residual:
// two halves, so a layer's attention never writes what its q rows read).
__device__ __forceinline__ float* hbuf(const LoopArgs& a, int l) {
  return a.h_buf + (size_t)(l & 1) * a.h_half;
}

// q rows [r0, r0+n) of layer l of model s: the token's embedding, plus the
// previous layer's attention output of the row (residual), by the whole grid.
__device__ void build_q(const LoopArgs& a, const Side& s, int l, int r0, int n, bool residual) {
  const int d = s.d, V = s.m.vocab;
  const int total = n * d;
  for (int i = blockIdx.x * blockDim.x + attn::item_tid(); i < total;
       i += gridDim.x * blockDim.x) {
    const int m = r0 + i / d, e = i - (i / d) * d;
    const int tok = a.tokens[m];
    float x = s.m.emb_q[((size_t)l * V + tok) * d + e];
    if (residual) x += hbuf(a, l - 1)[(size_t)m * d + e];
    a.q_buf[(size_t)m * d + e] = x;
  }
}

// Window rows [r0, r0+n) of layer l appended at pos0 + row, one block per
// row: kv_cache_append (kv_cache.cu:70-93), fp32 -> fp16 round to nearest
// even.  The host checked that every position the loop reaches is mapped.
// (Thread indices here and below come through attn::item_tid(), so the
// compiler cannot keep them live across the attention's register-heavy
// tile loop.)
// Token tok's K/V rows of layer l of model s at position pos, by the
// calling block.
__device__ __forceinline__ void append_token(const Side& s, int l, int tok, int pos) {
  const int kvd = s.kv.kv_dim, V = s.m.vocab;
  const float* k = s.m.emb_k + ((size_t)l * V + tok) * kvd;
  const float* v = s.m.emb_v + ((size_t)l * V + tok) * kvd;
  const int lb = pos / s.kv.block_size;
  const int pb = s.kv.block_tables[(size_t)l * s.kv.max_blocks_per_layer + lb];
  uint16_t* kd = s.kv.pool + ((size_t)pb * 2u * s.kv.block_size + (pos - lb * s.kv.block_size)) *
                                 (size_t)kvd;
  uint16_t* vd = kd + (size_t)s.kv.block_size * kvd;
  for (int i = attn::item_tid(); i < kvd; i += blockDim.x) {
    kd[i] = __builtin_bit_cast(uint16_t, (_Float16)k[i]);
    vd[i] = __builtin_bit_cast(uint16_t, (_Float16)v[i]);
  }
}

__device__ void append_rows(const LoopArgs& a, const Side& s, int l, int r0, int n, int pos0) {
  for (int r = r0 + blockIdx.x; r < r0 + n; r += gridDim.x)
    append_token(s, l, a.tokens[r], pos0 + r);
}

// The draft model's catch-up forward of megakernel_speculative_kernel
// (kernels.cu:3079-3093) as the draft cache sees it: token
// tokens[catch_up_slot] (the last draft when all were accepted, else the
// bonus) at position pos in every draft layer, one block per layer.  (The
// loop model's K/V depend on the token and the position alone; the
// forward's logits are unused.)
__device__ void catch_up(const LoopArgs& a, int pos) {
  const int tok = a.tokens[catch_up_slot(a.k)];
  for (int l = blockIdx.x; l < a.dr.kv.n_layers; l += gridDim.x) append_token(a.dr, l, tok, pos);
}

// The grid attention of layer l over window rows [r0, r0+n) at positions
// pos0 + row, as a function of its own: its tile loop gets the whole register
// budget instead of sharing it with the values the loops around it keep.
// 4-wave staging (64 KiB of LDS): the 8-wave form is off in the loop (see
// the design notes on the loop's attention).  Tile-path shapes take the
// window straight from the model's tables (device_attention_grid_gathered:
// q rows, residual and the window's K / V appends inside the attention);
// the generic shapes attend to the q rows and appends of the phase before.
__device__ __attribute__((noinline)) int layer_attention(const LoopArgs& a, const Side& s, int l,
                                                         int r0, int n, int pos0) {
  float* out = hbuf(a, l) + (size_t)r0 * s.d;
  if (a.fused) {
    const size_t V = (size_t)s.m.vocab;
    attn::GatherArgs g;
    g.tok = a.tokens + r0;
    g.q_table = s.m.emb_q + (size_t)l * V * s.d;
    g.q_add = l > 0 ? hbuf(a, l - 1) + (size_t)r0 * s.d : nullptr;
    g.k_table = s.m.emb_k + (size_t)l * V * s.kv.kv_dim;
    g.v_table = s.m.emb_v + (size_t)l * V * s.kv.kv_dim;
    g.pool = s.kv.pool;
    return device_attention_grid_gathered(g, out, s.kv, l, s.m.n_heads, s.m.n_kv_heads,
                                          s.m.head_dim, pos0 + r0, n, a.attn_ws,
                                          a.attn_ws_bytes);
  }
  return device_flash_attention_gqa_grid<4>(
      a.q_buf + (size_t)r0 * s.d, out, s.kv, l, s.m.n_heads, s.m.n_kv_heads, s.m.head_dim,
      pos0 + r0, n, a.attn_ws, a.attn_ws_bytes);
}

// Layers [lo, hi) of model s on window rows [r0, r0+n) at positions pos0 +
// row: (append, q, grid barrier,) grid attention, grid barrier; layer hi-1's
// output rows are then in hbuf(a, hi - 1).
__device__ __forceinline__ void run_layers(const LoopArgs& a, const Side& s, int lo, int hi,
                                           int r0, int n, int pos0) {
  for (int l = lo; l < hi; l++) {
    if (!a.fused) {
      append_rows(a, s, l, r0, n, pos0);
      build_q(a, s, l, r0, n, l > 0);
      barrier(a);
    }
    note_error(a, layer_attention(a, s, l, r0, n, pos0));
    barrier(a);
  }
}

// The output head over its panel-packed copy (sde_matvec_packed's
// workgroup body): every block takes (panel, pass) items in turn and writes
// whole output columns -- no partials, no arrival counters, no combining
// block.  A function of its own: the kernels keep their register budget
// for their loops.  Rows n <= 16 (two passes above 9).
// The greedy loop's argmax rides on the head (the lowest column among equal
// maxima, NaN never winning, all-NaN rows giving token 0): after an item,
// one thread per
// row of its pass scans the panel's logits it just wrote (visible to the
// block after the barrier) and publishes the panel's (max, column) with a
// device-scope store; the last item to arrive reduces every panel's
// candidates, in panel (column) order, into tokens[dst + row].
struct HeadArgmax {
  int dst;     // tokens[dst + row]; < 0: no argmax
  int accept;  // the greedy loop's verify: the argmax's block then accepts (accept_in_block)
  int P, D, round;
};

__device__ void accept_in_block(const LoopArgs& a, const HeadArgmax& am);

__device__ __forceinline__ bool arg_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

template <int PW>
__device__ __forceinline__ void panel_candidates(const LoopArgs& a, const mvp::PackedArgs& pa,
                                                 int panel, int pass, int panels) {
  const int m0 = pass * pa.pass_rows;
  const int mc = min(pa.pass_rows, pa.M - m0);
  const int t = (int)threadIdx.x;
  if (t < mc) {
    const float* row = pa.out + (size_t)(m0 + t) * pa.d_out + (size_t)panel * PW;
    float best = -INFINITY;
    int bi = pa.d_out;
#pragma unroll
    for (int c = 0; c < PW; c++) {
      const float v = row[c];
      if (v > best) {
        best = v;
        bi = panel * PW + c;
      }
    }
    const uint64_t bits = (uint64_t)__builtin_bit_cast(uint32_t, best) |
                          ((uint64_t)(uint32_t)bi << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(a.cand + (size_t)(m0 + t) * panels + panel),
                       bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The last item's block: row r's winner over its panels' candidates.
__device__ __forceinline__ void reduce_candidates(const LoopArgs& a, int n, int panels, int V,
                                                  int dst) {
  __shared__ float s_val[kThreads / 64];
  __shared__ int s_idx[kThreads / 64];
  const int tid = (int)threadIdx.x;
  for (int r = 0; r < n; r++) {
    float best = -INFINITY;
    int bi = V;
    for (int p = tid; p < panels; p += blockDim.x) {  // ascending panels per thread
      const uint64_t bits = __hip_atomic_load(
          reinterpret_cast<uint64_t*>(a.cand + (size_t)r * panels + p), __ATOMIC_RELAXED,
          __HIP_MEMORY_SCOPE_AGENT);
      const float v = __builtin_bit_cast(float, (uint32_t)bits);
      const int i = (int)(uint32_t)(bits >> 32);
      if (arg_better(v, i, best, bi)) {
        best = v;
        bi = i;
      }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(best, off);
      const int oi = __shfl_xor(bi, off);
      if (arg_better(ov, oi, best, bi)) {
        best = ov;
        bi = oi;
      }
    }
    if ((tid & 63) == 0) {
      s_val[tid >> 6] = best;
      s_idx[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < (int)(blockDim.x >> 6); w++)
        if (arg_better(s_val[w], s_idx[w], best, bi)) {
          best = s_val[w];
          bi = s_idx[w];
        }
      a.tokens[dst + r] = bi < V ? bi : 0;  // all NaN: token 0
    }
    __syncthreads();
  }
}

// The head's cross-wave sums: one LDS array for every row count (9 rows,
// 8 waves, 16-column panels) instead of one per instantiation.
__device__ __forceinline__ float* head_red() {
  __shared__ float buf[9 * mvp::kWaves * 16];
  return buf;
}

template <int MB, int LPR, bool ACCEPT>
__device__ __forceinline__ void head_items(const LoopArgs& a, const mvp::PackedArgs& pa,
                                           int panels, int passes, HeadArgmax am) {
  constexpr int PW = 8 * LPR;
  __shared__ int s_last;
  const int blk = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int nblk = gridDim.x * gridDim.y * gridDim.z;
  const int items = panels * passes;
  for (int it = blk; it < items; it += nblk) {
    const int panel = it % panels, pass = it / panels;
    static_assert(MB <= 9 && LPR <= 2, "head_red holds 9 rows of 16-column panels");
    mvp::packed_item<MB, LPR, (MB == 1 ? 8 : 4), true>(pa, panel, pass, head_red());
    __syncthreads();  // the item's logits are written; its LDS sums are read
    if (am.dst >= 0) {
      panel_candidates<PW>(a, pa, panel, pass, panels);
      __builtin_amdgcn_s_waitcnt(0);  // the candidates reached the coherence point
      __syncthreads();
      if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(a.cand_arrivals, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == (uint32_t)(items - 1);
        if (last)
          __hip_atomic_store(a.cand_arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
      }
      __syncthreads();
      if (s_last) {
        reduce_candidates(a, pa.M, panels, pa.d_out, am.dst);
        if constexpr (ACCEPT) {
          if (am.accept) accept_in_block(a, am);
        }
      }
    }
  }
}

template <int LPR, bool ACCEPT>
__device__ __forceinline__ void head_rows(const LoopArgs& a, const mvp::PackedArgs& pa,
                                          int panels, int passes, HeadArgmax am) {
  switch (pa.pass_rows) {
    case 1: head_items<1, LPR, ACCEPT>(a, pa, panels, passes, am); break;
    case 2: head_items<2, LPR, ACCEPT>(a, pa, panels, passes, am); break;
    case 3: head_items<3, LPR, ACCEPT>(a, pa, panels, passes, am); break;
    case 4: head_items<4, LPR, ACCEPT>(a, pa, panels, passes, am); break;
    case 5: head_items<5, LPR, ACCEPT>(a, pa, panels, passes, am); break;
    case 6: head_items<6, LPR, ACCEPT>(a, pa, panels, passes, am); break;
    case 7: head_items<7, LPR, ACCEPT>(a, pa, panels, passes, am); break;
    case 8: head_items<8, LPR, ACCEPT>(a, pa, panels, passes, am); break;
    default: head_items<9, LPR, ACCEPT>(a, pa, panels, passes, am); break;
  }
}

// ACCEPT: the greedy loop's form (its verify's argmax block accepts).
template <bool ACCEPT>
__device__ __attribute__((noinline)) void head_logits(const LoopArgs& a, const Side& s, int layer,
                                                      int r0, int n, float* logits,
                                                      HeadArgmax am) {
  const int d = wave_uniform(s.d), V = wave_uniform(s.m.vocab);
  n = wave_uniform(n);
  const mvp::PackedShape sh = mvp::packed_shape(d, V);
  mvp::PackedArgs pa;
  pa.W = wave_uniform(s.head_packed);
  pa.x = wave_uniform(hbuf(a, wave_uniform(layer)) + (size_t)wave_uniform(r0) * d);
  pa.out = wave_uniform(logits);
  pa.d_in = d;
  pa.d_out = V;
  pa.M = n;
  pa.pass_rows = mvp::packed_pass_rows(n);
  pa.n_batches = sh.n_batches;
  pa.accumulate = 0;
  const int passes = mvp::packed_passes(n);
  am.dst = wave_uniform(am.dst);
  am.accept = wave_uniform(am.accept);
  if (sh.lpr == 2)
    head_rows<2, ACCEPT>(a, pa, sh.panels, passes, am);
  else
    head_rows<1, ACCEPT>(a, pa, sh.panels, passes, am);
}

// Logits of window rows [r0, r0+n) from their h_buf rows (model s's head),
// then their argmaxes into tokens[dst + row].
__device__ __forceinline__ void decide(const LoopArgs& a, const Side& s, int layer, int r0, int n,
                                       int dst, HeadArgmax am = HeadArgmax{0, 0, 0, 0, 0}) {
  am.dst = dst;
  head_logits<true>(a, s, layer, r0, n, a.logits, am);
  barrier(a);
}

// Step s of a round's n_steps: the draft steps 0..n_steps-2 (window row s
// alone, layers [0, n_draft)), then the verify step (every window row,
// layers [n_draft, n_layers)).
struct Step {
  int lo, hi, r0, n;
  bool verify;
};

__device__ __forceinline__ Step round_step(const LoopArgs& a, int s, int n_steps, int n_layers) {
  const bool verify = s == n_steps - 1;
  return verify ? Step{a.n_draft, n_layers, 0, a.k + 1, true} : Step{0, a.n_draft, s, 1, false};
}

// Before the loop (the launch before it on the stream): the device
// functions' arrival counters and the barrier's arrivals at zero, the state
// words cleared, window token 0 = the anchor.
__global__ void spec_loop_init_kernel(LoopArgs a) {
  uint32_t* c = static_cast<uint32_t*>(a.attn_ws);
  for (int i = threadIdx.x; i < kGridCounters; i += blockDim.x) c[i] = 0u;
  for (int i = threadIdx.x; i < kBarWords; i += blockDim.x) a.bar[i] = 0u;
  if (threadIdx.x == 0) *a.cand_arrivals = 0u;
  if (a.offset) {  // the sampling loop: its device function's counters, its state words
    for (int i = threadIdx.x; i < kSpecScratchWords; i += blockDim.x) a.sscratch[i] = 0u;
  }
  if (threadIdx.x == 0) {
    // The anchor indexes the embedding tables: one outside the vocabulary
    // stops the launch at its first round check, before any table read.
    const int anchor = a.state[kAnchor];
    const bool ok = anchor >= 0 && anchor < a.t.m.vocab;
    a.tokens[0] = ok ? anchor : 0;
    a.tokens[done_slot(a.k)] = 0;
    for (int i = kEmitted; i < kStateWords; i++) a.state[i] = 0;
    if (!ok) a.state[kStatus] = SDE_ERR_INVALID_ARGUMENT;
    if (a.offset) {
      a.state[kTemp] = __float_as_int(a.smp.draft_temp);
      a.state[kEwma] = __float_as_int(-1.f);
    }
  }
}

// The round's opening checks, the same in every block: stop when max_new
// tokens are out, on a recorded status or after an EOS bonus; a window past
// the mapped positions records SDE_ERR_CAPACITY and stops.
__device__ __forceinline__ bool round_open(const LoopArgs& a, int P, int D) {
  if (load_word(a.state + kEmitted) >= a.max_new || load_word(a.state + kStatus) != SDE_OK ||
      load_word(a.tokens + done_slot(a.k)) != 0)
    return false;
  const int M = a.k + 1;
  if (P < 0 || P + M > a.t.cap || (a.two && (D < 0 || D + M > a.dr.cap))) {
    if (blockIdx.x == 0 && threadIdx.x == 0) store_word(a.state + kStatus, SDE_ERR_CAPACITY);
    return false;
  }
  return true;
}

// After the accept (block 0, thread 0): the two-cache loop's catch-up token
// and draft seq_len (draft_save + n + 1, the catch-up's position + 1), and
// the EOS flag.
__device__ __forceinline__ void round_close(const LoopArgs& a, int n, int bonus, int draft_seq) {
  if (a.two) {
    a.tokens[catch_up_slot(a.k)] = n == a.k ? a.tokens[a.k] : bonus;
    store_word(a.dr.kv.seq_len, draft_seq + 1);
  }
  if (a.eos >= 0 && bonus == a.eos) store_word(a.tokens + done_slot(a.k), 1);
}

__global__ __launch_bounds__(kThreads) void spec_loop_kernel(LoopArgs a) {
  const int M = a.k + 1;
  const int n_layers = a.t.kv.n_layers;
  register_blocks(a);

  for (int round = 0;; round++) {
    // Every block reads the same words after the barrier: the loop's exits
    // are uniform over the grid, so every block meets every barrier.
    const int P = load_word(a.t.kv.seq_len);
    const int D = a.two ? load_word(a.dr.kv.seq_len) : P;
    if (!round_open(a, P, D)) break;
    if (a.two) {
      // Draft (kernels.cu:2948-2958): the draft model, all its layers, window
      // token s at D+s; its argmax proposes token s+1.  Verify
      // (model_batch_forward_logits, model.cu:657-714): the target, all
      // layers, the whole window at P; the target's token for every row.
      for (int s = 0; s < a.k; s++) {
        run_layers(a, a.dr, 0, a.dr.kv.n_layers, s, 1, D);
        decide(a, a.dr, a.dr.kv.n_layers - 1, s, 1, s + 1);
      }
      run_layers(a, a.t, 0, n_layers, 0, M, P);
      decide(a, a.t, n_layers - 1, 0, M, M, HeadArgmax{0, 1, P, D, round});
    } else {
      // Draft (kernels.cu:2960-3006), steps 0..k when k > 0: the prefix
      // layers for window token s at P+s, one token at a time; the first k
      // outputs propose window token s+1.  Verify (model.cu:838-890), the
      // last step: the remaining layers over the whole window, then the
      // target's token for every row.
      const int n_steps = a.k > 0 ? M + 1 : 1;
      for (int s = 0; s < n_steps; s++) {
        const Step t = round_step(a, s, n_steps, n_layers);
        run_layers(a, a.t, t.lo, t.hi, t.r0, t.n, P);
        if (t.verify)
          decide(a, a.t, t.hi - 1, t.r0, t.n, M, HeadArgmax{0, 1, P, D, round});
        else if (s < a.k)
          decide(a, a.t, t.hi - 1, t.r0, t.n, s + 1);
      }
    }
    // (the verify's decide accepted, rewound and caught up: accept_in_block)
  }
}

// Greedy accept and O(1) rewinds (kernels.cu:3050-3076), by the block that
// reduced the verify's argmax, right after it (the target's tokens are its
// own stores): thread 0 accepts; with a draft model the block then appends
// the catch-up token's K / V at draft_save + n in every draft layer
// (kernels.cu:3079-3093).  The decide's grid barrier follows, so the round
// needs no barrier of its own for the accept or the catch-up.
__device__ void accept_in_block(const LoopArgs& a, const HeadArgmax& am) {
  __shared__ int s_pos;
  const int M = a.k + 1;
  if (threadIdx.x == 0) {
    const int E = a.state[kEmitted];
    const SpecAccept r = spec_accept_greedy(a.tokens + 1, a.tokens + M, a.k, am.P, am.D, a.t.kv,
                                            a.two ? &a.dr.kv : nullptr, a.emitted + E);
    store_word(a.t.kv.seq_len, r.target_seq);  // (spec_accept_greedy wrote it plainly)
    store_word(a.state + kEmitted, E + r.n_accepted + 1);
    a.state[kAnchor] = r.bonus;
    a.state[kRounds] = am.round + 1;
    a.state[kProposed] += a.k;
    a.state[kAccepted] += r.n_accepted;
    a.accepted[am.round] = r.n_accepted;
    a.tokens[0] = r.bonus;
    round_close(a, r.n_accepted, r.bonus, r.draft_seq);
    s_pos = r.draft_seq;
  }
  __syncthreads();
  if (a.two) {
    const int tok = a.tokens[catch_up_slot(a.k)];
    for (int l = 0; l < a.dr.kv.n_layers; l++) append_token(a.dr, l, tok, s_pos);
  }
}

// The grid barrier as the stochastic device function's `sync`.
struct GridSync {
  const LoopArgs* a;
  __device__ void operator()() const { barrier(*a); }
};

// The draft temperature's update after a round (kernels.cu:3441-3458): an
// exponential average of the round's acceptance rate, moved toward the
// target rate by `gain`, clamped to [min_temp, max_temp].
__device__ void adapt_temperature(const LoopArgs& a, int n_accepted) {
  if (!a.smp.adaptive || a.k < 1) return;
  const float mix = fminf(fmaxf(a.smp.ewma_mix, 1e-6f), 1.f - 1e-6f);
  const float rr = (float)n_accepted / (float)a.k;
  float ewma = __int_as_float(a.state[kEwma]);
  ewma = ewma < 0.f ? rr : (1.f - mix) * ewma + mix * rr;
  float t = __int_as_float(a.state[kTemp]);
  t += a.smp.gain * (ewma - a.smp.target_accept);
  t = fmaxf(a.smp.min_temp, fminf(a.smp.max_temp, t));
  a.state[kEwma] = __float_as_int(ewma);
  a.state[kTemp] = __float_as_int(t);
}

// A draft sample's token into window slot `slot`, on the thread that drew
// it (a token outside the vocabulary would index the tables out of bounds:
// record an error and continue with token 0).
struct DraftTokenHook {
  const LoopArgs* a;
  int slot;
  __device__ void operator()(int, int tok, int, int) const {
    const bool ok = tok >= 0 && tok < a->t.m.vocab;
    a->tokens[slot] = ok ? tok : 0;
    if (!ok) atomicCAS(reinterpret_cast<int*>(a->state + kStatus), SDE_OK, SDE_ERR_HIP);
  }
};

// The round's bookkeeping after the sampling accept, on the thread that
// decided it (emitted tokens: the accepted drafts, then the corrected or
// bonus token), then the temperature update and the round's close.
struct AcceptHook {
  const LoopArgs* a;
  int P, D, round;
  __device__ void operator()(int n, int tok, int t_seq, int d_seq) const {
    const LoopArgs& la = *a;
    const int E = load_word(la.state + kEmitted);
    if (n < 0 || n > la.k || tok < 0 || tok >= la.t.m.vocab || t_seq != P + n + 1 ||
        (la.two && d_seq != D + n)) {
      // not a result of the acceptance: stop with an error, caches untouched
      atomicCAS(reinterpret_cast<int*>(la.state + kStatus), SDE_OK, SDE_ERR_HIP);
      store_word(la.t.kv.seq_len, P);
      if (la.two) store_word(la.dr.kv.seq_len, D);
      return;
    }
    for (int j = 0; j < n; j++) la.emitted[E + j] = la.tokens[1 + j];
    la.emitted[E + n] = tok;
    store_word(la.t.kv.seq_len, t_seq);
    store_word(la.state + kEmitted, E + n + 1);
    la.state[kAnchor] = tok;
    la.state[kRounds] = round + 1;
    la.state[kProposed] += la.k;
    la.state[kAccepted] += n;
    la.accepted[round] = n;
    la.tokens[0] = tok;
    adapt_temperature(la, n);
    round_close(la, n, tok, D + n);
  }
};

// Speculative sampling over the same rounds (megakernel_speculative_
// stochastic_kernel, kernels.cu:3108-3481, self-speculative): draft token
// i+1 is sampled from softmax(draft logits of row i / T_d) by the
// stochastic device function with no drafts (its bonus row); the window's
// target logits and every draft row's logits then go to the same function
// for the accept tests and the corrected or bonus sample (target temperature
// 1, as the reference), which also rewinds seq_len; T_d adapts per round.
// Unlike the reference, the draft rows' logits are kept from drafting
// instead of recomputed after a rejection (the same values).
__global__ __launch_bounds__(kThreads) void spec_loop_stochastic_kernel(LoopArgs a) {
  const int M = a.k + 1;
  const int V = a.t.m.vocab;
  const int n_layers = a.t.kv.n_layers;
  const GridSync sync{&a};
  const size_t sbytes = spec_stochastic_workspace_size();
  sde_kv_view dv = a.t.kv;  // draft samples rewind nothing: their seq_len word is scratch
  dv.seq_len = a.dres + 7;
  register_blocks(a);

  for (int round = 0;; round++) {
    const int P = load_word(a.t.kv.seq_len);
    const int D = a.two ? load_word(a.dr.kv.seq_len) : P;
    if (!round_open(a, P, D)) break;
    const float temp = __int_as_float(load_word(a.state + kTemp));
    // The greedy loop's steps: drafts 0..k-1 sample the next window token
    // from their logits (the self-speculative draft step k only appends),
    // the last step verifies; with a draft model, its k steps draft and the
    // target verifies.
    const int n_steps = a.two ? M : (a.k > 0 ? M + 1 : 1);
    for (int s = 0; s < n_steps; s++) {
      const Step t = a.two ? (s < a.k ? Step{0, a.dr.kv.n_layers, s, 1, false}
                                      : Step{0, n_layers, 0, M, true})
                           : round_step(a, s, n_steps, n_layers);
      const Side& sd = a.two && !t.verify ? a.dr : a.t;
      run_layers(a, sd, t.lo, t.hi, t.r0, t.n, t.verify ? P : (a.two ? D : P));
      if (!t.verify && s >= a.k) continue;
      float* lg = t.verify ? a.logits : a.dlogits + (size_t)s * V;
      head_logits<false>(a, sd, t.hi - 1, t.r0, t.n, lg, HeadArgmax{-1, 0, 0, 0, 0});
      barrier(a);
      if (t.verify) break;
      int st = device_spec_accept_stochastic_grid(lg, nullptr, nullptr, 0, V, temp, 1.f, a.smp.seed,
                                              a.offset, 0, 0, dv, nullptr, a.dres, a.sscratch,
                                              sbytes, sync, DraftTokenHook{&a, s + 1});
      note_error(a, st);
      barrier(a);
    }
    int st = device_spec_accept_stochastic_grid(a.logits, a.dlogits, a.tokens + 1, a.k, V, 1.f, temp,
                                            a.smp.seed, a.offset, P, D, a.t.kv,
                                            a.two ? &a.dr.kv : nullptr, a.sres, a.sscratch, sbytes,
                                            sync, AcceptHook{&a, P, D, round});
    note_error(a, st);
    barrier(a);
    if (a.two && load_word(a.state + kStatus) == SDE_OK) {  // the draft's catch-up
      catch_up(a, load_word(a.dr.kv.seq_len) - 1);
      barrier(a);
    }
  }
}

}  // namespace loop
}  // namespace sde

namespace {

// A loop model's checks against its cache (the same for the target and a
// draft model).
int check_model(const sde_kv_cache* cache, const sde_loop_model* model) {
  if (!cache || !model) return SDE_ERR_INVALID_ARGUMENT;
  const sde_loop_model& m = *model;
  if (!m.emb_q || !m.emb_k || !m.emb_v || !m.head) return SDE_ERR_INVALID_ARGUMENT;
  if (m.n_heads < 1 || m.n_kv_heads < 1 || m.n_heads % m.n_kv_heads != 0 ||
      m.n_kv_heads * m.head_dim != cache->cfg.kv_dim || m.vocab < 8)
    return SDE_ERR_INVALID_ARGUMENT;
  // Head sizes 64 / 128 with block sizes that are multiples of 8 run the
  // tile path of the grid attention, the others (head_dim up to 512) its
  // generic path; the packed head needs n_heads * head_dim and the
  // vocabulary to be multiples of 8.
  if (m.head_dim > sde::gen::kMaxDph || (m.n_heads * m.head_dim) % 8 != 0 || m.vocab % 8 != 0 ||
      (reinterpret_cast<uintptr_t>(m.head) & 15u) != 0)
    return SDE_ERR_UNSUPPORTED;
  return SDE_OK;
}

// A model's attention shape over its cache (the attention workspace is
// sized for the cache's whole table).
sde::loop::Shape shape_of(const sde_kv_cache* cache, const sde_loop_model* m) {
  return {m->n_heads, m->n_kv_heads, m->head_dim,
          cache->cfg.max_blocks_per_layer * cache->cfg.block_size};
}

// Positions every layer of the cache maps to a physical block.
int mapped_positions(const sde_kv_cache* cache) {
  int cap = cache->cfg.max_blocks_per_layer * cache->cfg.block_size;
  for (int l = 0; l < cache->cfg.n_layers; l++) {
    const int mapped = (int)sde::mapped_tokens(cache, l);
    if (mapped < cap) cap = mapped;
  }
  return cap;
}

// The workspace layout for a configuration (its shapes checked by the caller).
sde::loop::Layout config_layout(const sde_kv_cache* cache, const sde_loop_model* model,
                                const sde_spec_loop_config& c) {
  const sde::loop::Shape t = shape_of(cache, model);
  if (c.draft_cache) {
    const sde::loop::Shape d = shape_of(c.draft_cache, c.draft_model);
    return sde::loop::layout(t, &d, model->vocab, c.k);
  }
  return sde::loop::layout(t, nullptr, model->vocab, c.k);
}

sde::loop::Side make_side(const sde_kv_view& kv, const sde_loop_model& m, int cap,
                          const char* packed) {
  sde::loop::Side s;
  s.kv = kv;
  s.m = m;
  s.d = m.n_heads * m.head_dim;
  s.cap = cap;
  s.head_packed = reinterpret_cast<const uint4*>(packed);
  return s;
}

// The head's panel-packed copy for this launch (a one-time re-layout per
// call, amortized over its rounds).
int pack_head(const sde_loop_model& m, char* dst, int n_cus, hipStream_t stream) {
  const int d = m.n_heads * m.head_dim;
  const sde::mvp::PackedShape hs = sde::mvp::packed_shape(d, m.vocab);
  if (hs.panels == 0) return SDE_ERR_UNSUPPORTED;
  const size_t pack_blocks = (hs.units + 255) / 256;
  const int pb = (int)(pack_blocks < (size_t)n_cus * 16 ? pack_blocks : (size_t)n_cus * 16);
  sde::mvp::matvec_pack_kernel<<<pb, 256, 0, stream>>>(m.head, reinterpret_cast<uint4*>(dst), d,
                                                       m.vocab);
  return hipGetLastError() == hipSuccess ? SDE_OK : SDE_ERR_HIP;
}

// The checks and the launch shared by the greedy and the sampling loops,
// self-speculative or with a draft model over a cache of its own.
int launch_loop(sde_kv_cache* cache, const sde_loop_model* model, const sde_spec_loop_config* cfg,
                int32_t* d_state, int32_t* d_emitted, int32_t* d_accepted, void* d_workspace,
                size_t workspace_bytes, sde_stream_t stream, const sde_loop_sampling* smp,
                uint64_t* d_offset) {
  using namespace sde::loop;
  if (!cfg || !d_state || !d_emitted || !d_accepted || !d_workspace)
    return SDE_ERR_INVALID_ARGUMENT;
  const sde_spec_loop_config c = *cfg;
  int st = check_model(cache, model);
  if (st != SDE_OK) return st;
  const sde_loop_model& m = *model;
  if (c.max_new < 1) return SDE_ERR_INVALID_ARGUMENT;
  if (c.k < 0 || c.k + 1 > kMaxWindow) return SDE_ERR_RANGE;
  const int n_layers = cache->cfg.n_layers;
  const bool two = c.draft_cache != nullptr || c.draft_model != nullptr;
  if (two) {
    // A draft model over its own cache (kernels.cu:3593-3627, not
    // self_speculative): the same vocabulary, another cache on the device.
    if (!c.draft_cache || !c.draft_model || c.draft_cache == cache || c.k < 1)
      return SDE_ERR_INVALID_ARGUMENT;
    st = check_model(c.draft_cache, c.draft_model);
    if (st != SDE_OK) return st;
    if (c.draft_model->vocab != m.vocab || c.draft_cache->device != cache->device)
      return SDE_ERR_INVALID_ARGUMENT;
  } else if (c.k > 0 && (c.n_draft < 1 || c.n_draft >= n_layers)) {
    return SDE_ERR_INVALID_ARGUMENT;
  }
  if (smp) {
    if (!d_offset || !std::isfinite(smp->draft_temp) || !std::isfinite(smp->min_temp) ||
        !std::isfinite(smp->max_temp) || !std::isfinite(smp->target_accept) ||
        !std::isfinite(smp->gain) || !std::isfinite(smp->ewma_mix) ||
        (smp->adaptive && smp->min_temp > smp->max_temp))
      return SDE_ERR_INVALID_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(d_offset) & 7u) != 0) return SDE_ERR_INVALID_ARGUMENT;
  }
  const Layout lay = config_layout(cache, model, c);
  if (workspace_bytes < lay.total) return SDE_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(d_workspace) & 255u) != 0) return SDE_ERR_INVALID_ARGUMENT;

  sde::DeviceGuard guard(cache->device);
  if (!guard.ok()) return SDE_ERR_HIP;
  const void* kernel = smp ? reinterpret_cast<const void*>(spec_loop_stochastic_kernel)
                           : reinterpret_cast<const void*>(spec_loop_kernel);
  int coop = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, cache->device) !=
          hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0) != hipSuccess)
    return SDE_ERR_HIP;
  if (!coop || per_cu < 1) return SDE_ERR_UNSUPPORTED;

  char* ws = static_cast<char*>(d_workspace);
  sde_kv_view tv, dv{};
  if (sde_kv_get_view(cache, &tv) != SDE_OK) return SDE_ERR_INVALID_ARGUMENT;
  if (two && sde_kv_get_view(c.draft_cache, &dv) != SDE_OK) return SDE_ERR_INVALID_ARGUMENT;
  LoopArgs a;
  // Every position the loop can reach must have a physical block.
  a.t = make_side(tv, m, mapped_positions(cache), ws + lay.head);
  a.dr = two ? make_side(dv, *c.draft_model, mapped_positions(c.draft_cache), ws + lay.dhead)
             : a.t;
  a.two = two ? 1 : 0;
  a.eos = c.eos_token < 0 ? -1 : c.eos_token;
  a.k = c.k;
  a.n_draft = two || c.k == 0 ? 0 : c.n_draft;
  a.max_new = c.max_new;
  a.state = d_state;
  a.emitted = d_emitted;
  a.accepted = d_accepted;
  a.attn_ws = ws + lay.attn;
  a.attn_ws_bytes = lay.q - lay.attn;
  a.cand_arrivals = reinterpret_cast<uint32_t*>(ws + lay.cand);
  a.cand = reinterpret_cast<uint2*>(ws + lay.cand + 256);
  a.q_buf = reinterpret_cast<float*>(ws + lay.q);
  a.h_buf = reinterpret_cast<float*>(ws + lay.h);
  a.h_half = (size_t)(c.k + 1) * (size_t)(two ? (a.t.d > a.dr.d ? a.t.d : a.dr.d) : a.t.d);
  // The gathered attention serves the tile-path shapes; every side must
  // have one (the loop's phases are uniform over the grid).
  a.fused = !sde::gen::needs_generic(m.head_dim, cache->cfg.block_size) &&
            (!two || !sde::gen::needs_generic(c.draft_model->head_dim,
                                              c.draft_cache->cfg.block_size));
  a.logits = reinterpret_cast<float*>(ws + lay.logits);
  a.tokens = reinterpret_cast<int32_t*>(ws + lay.tokens);
  a.bar = reinterpret_cast<uint32_t*>(ws + lay.bar);
  a.dlogits = reinterpret_cast<float*>(ws + lay.dlogits);
  a.sres = reinterpret_cast<int32_t*>(ws + lay.sres);
  a.dres = reinterpret_cast<int32_t*>(ws + lay.dres);
  a.sscratch = reinterpret_cast<uint32_t*>(ws + lay.sscratch);
  a.offset = smp ? d_offset : nullptr;
  a.smp = smp ? *smp : sde_loop_sampling{};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  st = pack_head(m, ws + lay.head, cache->n_cus, s);
  if (st == SDE_OK && two) st = pack_head(*c.draft_model, ws + lay.dhead, cache->n_cus, s);
  if (st != SDE_OK) return st;
  spec_loop_init_kernel<<<1, 256, 0, s>>>(a);
  if (hipGetLastError() != hipSuccess) return SDE_ERR_HIP;
  // A cooperative launch: every block resident at once, which the grid
  // barrier needs.
  void* args[] = {&a};
  const hipError_t e =
      hipLaunchCooperativeKernel(kernel, dim3(cache->n_cus), dim3(kThreads), args, 0, s);
  if (e != hipSuccess) return SDE_ERR_HIP;
  cache->seq_len_on_device = true;
  if (two) c.draft_cache->seq_len_on_device = true;
  return SDE_OK;
}

sde_spec_loop_config self_config(int k, int n_draft, int max_new) {
  sde_spec_loop_config c{};
  c.k = k;
  c.n_draft = n_draft;
  c.max_new = max_new;
  c.eos_token = -1;
  return c;
}

}  // namespace

extern "C" {

size_t sde_spec_loop_config_workspace_size(const sde_kv_cache* cache, const sde_loop_model* model,
                                           const sde_spec_loop_config* cfg) {
  if (!cfg || cfg->k < 0 || cfg->k + 1 > sde::loop::kMaxWindow) return 0;
  if (check_model(cache, model) != SDE_OK) return 0;
  if (cfg->draft_cache || cfg->draft_model) {
    if (!cfg->draft_cache || !cfg->draft_model ||
        check_model(cfg->draft_cache, cfg->draft_model) != SDE_OK ||
        cfg->draft_model->vocab != model->vocab)
      return 0;
  }
  return config_layout(cache, model, *cfg).total;
}

size_t sde_spec_loop_workspace_size(const sde_kv_cache* cache, const sde_loop_model* model,
                                    int k) {
  if (!cache || !model || k < 0 || k + 1 > sde::loop::kMaxWindow) return 0;
  if (model->n_heads < 1 || model->n_kv_heads < 1 || model->head_dim < 1 || model->vocab < 1)
    return 0;
  return sde::loop::layout(shape_of(cache, model), nullptr, model->vocab, k).total;
}

int sde_spec_loop(sde_kv_cache* cache, const sde_loop_model* model, const sde_spec_loop_config* cfg,
                  const sde_loop_sampling* sampling, uint64_t* d_rng_offset, int32_t* d_state,
                  int32_t* d_emitted, int32_t* d_accepted, void* d_workspace,
                  size_t workspace_bytes, sde_stream_t stream) {
  return launch_loop(cache, model, cfg, d_state, d_emitted, d_accepted, d_workspace,
                     workspace_bytes, stream, sampling, d_rng_offset);
}

int sde_spec_loop_greedy(sde_kv_cache* cache, const sde_loop_model* model, int k, int n_draft,
                         int max_new, int32_t* d_state, int32_t* d_emitted,
                         int32_t* d_accepted, void* d_workspace, size_t workspace_bytes,
                         sde_stream_t stream) {
  const sde_spec_loop_config c = self_config(k, n_draft, max_new);
  return launch_loop(cache, model, &c, d_state, d_emitted, d_accepted, d_workspace,
                     workspace_bytes, stream, nullptr, nullptr);
}

int sde_spec_loop_stochastic(sde_kv_cache* cache, const sde_loop_model* model, int k,
                             int n_draft, int max_new, const sde_loop_sampling* sampling,
                             uint64_t* d_rng_offset, int32_t* d_state, int32_t* d_emitted,
                             int32_t* d_accepted, void* d_workspace, size_t workspace_bytes,
                             sde_stream_t stream) {
  if (!sampling) return SDE_ERR_INVALID_ARGUMENT;
  const sde_spec_loop_config c = self_config(k, n_draft, max_new);
  return launch_loop(cache, model, &c, d_state, d_emitted, d_accepted, d_workspace,
                     workspace_bytes, stream, sampling, d_rng_offset);
}

}  // extern "C"
