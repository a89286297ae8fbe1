// C ABI (include/funasr_hip.h) over the gfx950 kernels.
//
// Ownership follows the reference's seam: host pointers are used only during
// a call; weights are copied to the device once and immutable afterwards; a
// context owns one stream and serialises its calls with a mutex.
#include "../../include/funasr_hip.h"
#include "fah_internal.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& message) {
  g_error = message;
  return code;
}

struct DeviceError {
  std::string what;
};

void check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw DeviceError{std::string(what) + ": " + hipGetErrorString(e)};
}

struct ArgumentError {
  std::string what;
};

// A call in the wrong state (FAH_ERROR_STATE), e.g. greedy without logits.
struct StateError {
  std::string what;
};

void require(bool ok, const std::string& what) {
  if (!ok) throw ArgumentError{what};
}

template <typename F>
int guarded(F&& f) {
  try {
    return f();
  } catch (const ArgumentError& e) {
    return fail(FAH_ERROR_ARGUMENT, e.what);
  } catch (const StateError& e) {
    return fail(FAH_ERROR_STATE, e.what);
  } catch (const DeviceError& e) {
    return fail(FAH_ERROR_DEVICE, e.what);
  } catch (const std::bad_alloc&) {
    return fail(FAH_ERROR_DEVICE, "host allocation failed");
  }
}

// Device allocation owned by one object; freed on destruction.
struct DeviceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept : ptr(o.ptr), bytes(o.bytes) {
    o.ptr = nullptr;
    o.bytes = 0;
  }
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
      release();
      ptr = o.ptr;
      bytes = o.bytes;
      o.ptr = nullptr;
      o.bytes = 0;
    }
    return *this;
  }
  ~DeviceBuffer() { release(); }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  void allocate(size_t n) {
    release();
    if (n == 0) n = 16;
    check(hipMalloc(&ptr, n), "hipMalloc");
    bytes = n;
  }
  void ensure(size_t n) {
    if (n > bytes) allocate(n);
  }
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

uint16_t float_to_half_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t a = x & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (a >= 0x38800000u) return (uint16_t)(sign | ((a + 0xfffu + ((a >> 13) & 1u) - 0x38000000u) >> 13));
  uint32_t e = a >> 23;
  if (e < 102) return sign;
  uint32_t m = (a & 0x7fffffu) | 0x800000u, shift = 126u - e;
  uint32_t r = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (r & 1u))) r++;
  return (uint16_t)(sign | r);
}

float half_bits_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, u;
  if (e == 0) {
    float mag = (float)m * (1.0f / 16777216.0f);
    std::memcpy(&u, &mag, 4);
    u |= sign;
  } else if (e == 31) {
    u = m == 0 ? (sign | 0x7f800000u) : (sign | 0x7fc00000u | (m << 13));
  } else {
    u = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// True when every scale survives fp32 -> fp16 -> fp32 bit for bit.
bool scales_fit_half(const float* s, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    float back = half_bits_to_float(float_to_half_bits(s[i]));
    if (std::memcmp(&back, &s[i], 4) != 0) return false;
  }
  return true;
}

// Rows per workgroup for a Q8 GEMV: at most 4 (row, block) pairs per lane,
// then shrink until the grid has >= 512 workgroups (floor `min_rows`).
int pick_group_rows(int rows, int K, int min_rows, bool even) {
  int B = K / 32;
  int group = 64;
  while (group > 1 && group * B > 1024) group /= 2;
  while (group > min_rows && rows / group < 512) group /= 2;
  if (even && group < 2) group = 2;
  return group;
}

// Row buffers and the captured step of one lock-step batch of sessions. The
// context keeps the last one while its sessions live, so repeated calls on
// the same sessions replay the same graph.
struct SessionBatch {
  std::vector<fah_decoder*> members;
  int max_positions = 0;
  DeviceBuffer table, x, a, qkv, q, h, xq, xs, logits, keys;
  DeviceBuffer tokens;  // the step batcher's gathered tokens, one per session
  std::vector<fah::SessionRef> host_table;  // source of the last table upload (alive until the next)
  hipGraphExec_t graph = nullptr;
  // One-launch layers (fah_sessions.hip): its layer table, exchange words,
  // epoch and error word, and the launch arguments.
  bool fused = false;
  DeviceBuffer layer_table, exchange, epoch, error;
  fah::SessionStepArgs sargs{};
  // Pinned read-back of a batcher step: the tokens, then the error word and
  // the epoch (asynchronous copies, one synchronisation).
  int32_t* readback = nullptr;
  SessionBatch() = default;
  SessionBatch(const SessionBatch&) = delete;
  SessionBatch& operator=(const SessionBatch&) = delete;
  ~SessionBatch() {
    if (graph) (void)hipGraphExecDestroy(graph);
    if (readback) (void)hipHostFree(readback);
  }
};

// State of one context: device, stream, working buffers. The handle the
// caller holds (fah_context) and every weight and decoder made from it share
// it, so it outlives fah_context_destroy until the last of them is released;
// after destroy it only reports "disposed".
struct Ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t mark = nullptr;  // recorded by a persistent section on another context of the device
  std::mutex gate;
  bool disposed = false;
  int64_t minimum_operations = 250000;
  DeviceBuffer in, out, q, s;
  std::string name;
  std::unique_ptr<SessionBatch> batch;  // last lock-step batch (its sessions alive)
  // Seam-call statistics (fah_context_statistics) and the call observer;
  // t0/t1 bracket a call's kernels on the stream.
  std::mutex stats_m;
  fah_call_stats stats[FAH_CALL_KINDS] = {};
  fah_call_observer observer = nullptr;
  void* observer_user = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  Ctx() = default;
  Ctx(const Ctx&) = delete;
  Ctx& operator=(const Ctx&) = delete;
  ~Ctx();
};

// Work of every context on one device is enqueued under this lock. The
// persistent decode step needs every CU of the device to itself (one
// workgroup per CU, all co-resident, dealt to the XCDs in turn), so a
// persistent section holds the lock from before its launches until its
// stream has drained, after making its stream wait for the work already
// enqueued on the other contexts' streams: no other context's kernel can
// then run beside it.
struct DeviceGate {
  std::mutex m;
  std::vector<Ctx*> members;
};
constexpr int kMaxDevices = 64;
DeviceGate& device_gate(int device) {
  static DeviceGate gates[kMaxDevices];
  return gates[device];
}

Ctx::~Ctx() {
  if (!stream) return;
  (void)hipSetDevice(device);
  (void)hipStreamSynchronize(stream);
  batch.reset();
  {
    DeviceGate& g = device_gate(device);
    std::lock_guard<std::mutex> lock(g.m);
    g.members.erase(std::remove(g.members.begin(), g.members.end(), this), g.members.end());
  }
  in.release();
  out.release();
  q.release();
  s.release();
  if (mark) (void)hipEventDestroy(mark);
  if (t0) (void)hipEventDestroy(t0);
  if (t1) (void)hipEventDestroy(t1);
  (void)hipStreamDestroy(stream);
}

// Enqueue section for ordinary work: holds the device lock while the caller
// enqueues. Calls that then wait for their stream release it first, so the
// wait and the copy back do not hold up other contexts of the device.
struct DeviceWork {
  std::unique_lock<std::mutex> lock;
  explicit DeviceWork(const Ctx& c) : lock(device_gate(c.device).m) {}
  void release() {
    if (lock.owns_lock()) lock.unlock();
  }
};

// Persistent section: the device lock, the other streams' pending work
// ahead of this stream, and this stream drained before the lock is let go.
struct PersistentSection {
  Ctx& c;
  std::unique_lock<std::mutex> lock;
  explicit PersistentSection(Ctx& ctx) : c(ctx), lock(device_gate(ctx.device).m) {
    for (Ctx* o : device_gate(c.device).members) {
      if (o == &c) continue;
      check(hipEventRecord(o->mark, o->stream), "hipEventRecord");
      check(hipStreamWaitEvent(c.stream, o->mark, 0), "hipStreamWaitEvent");
    }
  }
  ~PersistentSection() { (void)hipStreamSynchronize(c.stream); }
};

// Accounting of one seam call that runs on the device: its kernels between
// the context's two events, its wall time from construction to done(), and
// the bytes it copies. done() runs after the stream has drained.
struct CallMeter {
  Ctx& c;
  int kind;
  int64_t up = 0, down = 0;
  std::chrono::steady_clock::time_point start = std::chrono::steady_clock::now();
  CallMeter(Ctx& ctx, int k) : c(ctx), kind(k) {}
  void kernels_begin() { check(hipEventRecord(c.t0, c.stream), "hipEventRecord"); }
  void kernels_end() { check(hipEventRecord(c.t1, c.stream), "hipEventRecord"); }
  void done(int frames, int cols, int rows, int64_t operations) {
    float device_ms = 0.0f;
    (void)hipEventElapsedTime(&device_ms, c.t0, c.t1);
    const double total_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
    fah_call_observer observer;
    void* user;
    {
      std::lock_guard<std::mutex> lock(c.stats_m);
      fah_call_stats& s = c.stats[kind];
      ++s.calls;
      s.operations += operations;
      s.uploaded_bytes += up;
      s.downloaded_bytes += down;
      s.device_ms += device_ms;
      s.total_ms += total_ms;
      observer = c.observer;
      user = c.observer_user;
    }
    if (observer) observer(user, kind, frames, cols, rows, device_ms, total_ms);
  }
};

int declined(Ctx* c, int kind) {
  std::lock_guard<std::mutex> lock(c->stats_m);
  ++c->stats[kind].declined;
  return FAH_DECLINED;
}

// Workspace of fah_quantized_linear_noalloc: the staged input, bias and
// output and the quantised activations, in one fixed device array per GPU
// (no hipMalloc on that path). Host code never passes `scratch` itself (its
// host-side name is not a device address): it uses the address that
// hipGetSymbolAddress returned for the device, kept in scratch_ptr.
constexpr size_t kScratchBytes = 8u << 20;
}  // namespace
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
namespace {
std::mutex g_scratch_gate;
void* g_scratch_ptr[kMaxDevices] = {};

// Once per device, with that device current (called by fah_context_create).
void init_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_gate);
  if (g_scratch_ptr[device]) return;
  void* ptr = nullptr;
  check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  g_scratch_ptr[device] = ptr;
}

void* scratch_ptr(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_gate);
  return g_scratch_ptr[device];
}

}  // namespace

struct fah_context {
  std::shared_ptr<Ctx> st;
};

struct fah_weight {
  std::shared_ptr<Ctx> ctx;
  int rows = 0, cols = 0;
  bool half_scales = true;
  DeviceBuffer q, s;
  int group_rows = 1;
  // FP32 weight (Weight.Values): `f` holds [rows][cols] floats, q/s unused.
  bool f32 = false;
  DeviceBuffer f;
};

struct DeviceMatrix {
  DeviceBuffer q, s;
  int rows = 0, cols = 0, group_rows = 1;
};

// Device weights of one decoder, shared by every session created from it.
struct DecoderWeights {
  bool half_scales = true;
  std::vector<DeviceMatrix> qkv, wo, gateup, down;
  std::vector<DeviceBuffer> attn_norm, q_norm, k_norm, ffn_norm;
  DeviceMatrix embed, lm_head;  // lm_head aliases embed when tied
  bool tied = true;
  DeviceBuffer output_norm;
  int64_t weight_bytes = 0;
  // Persistent kernel's per-layer pointer table (when the layout is the
  // persistent one) and the gate/up storage tiles: base rows, the first
  // `extra` tiles one more, or (persistent layout) the storage row of every
  // gate and up row in gu_map.
  bool persistent_layout = false;
  DeviceBuffer layer_table;
  int gu_base = 1, gu_extra = 0;
  DeviceBuffer gu_map;
};

struct fah_decoder {
  std::shared_ptr<Ctx> ctx;
  fah_decoder_config cfg{};
  int q_width = 0, kv_width = 0;
  std::shared_ptr<DecoderWeights> wt;
  DeviceBuffer rope_cos, rope_sin, kcache, vcache;
  DeviceBuffer x, qkv_out, qh, scores, block_max, block_sum, exp_t, attn, a, h, logits, keys, token, position, history, history_count, staging;
  DeviceBuffer row_q, row_s;  // one quantised row (multi-kernel path over persistent-layout weights)
  int lm_groups = 0;
  int host_position = 0;
  bool have_logits = false;
  bool fail_sessions = false;  // fah_decoder_fail_next_step: the next one-launch lock-step step fails too
  hipGraphExec_t graph_row = nullptr, graph_logits = nullptr, graph_step = nullptr;
  // Persistent single-launch step (one workgroup per CU), when the shape has
  // an instantiation and the device has the CUs for it.
  bool persistent = false;
  int blocks = 0;
  int persistent_positions = 0;  // positions below which steps take the persistent kernel
  DeviceBuffer tx, tqkv, tatt, ta, th, tkeys, tattq, thq, tscore, tready, epoch, error, timeline;
  fah::PersistentArgs pargs{};
  // Prefill (decode of many rows at once): row buffers grown on demand.
  DeviceBuffer pf_x, pf_a, pf_qkv, pf_q, pf_h, pf_xq, pf_xs, pf_hq, pf_hs;
  // Attention timing of the multi-kernel step (FAH_ATTENTION_TIMES=1 at
  // creation): events around every layer's attention kernels, the steps
  // launched one by one and their attention time summed.
  bool attention_times = false;
  std::vector<hipEvent_t> attn_events;
  double attn_ms = 0.0;
  int attn_steps = 0;
  ~fah_decoder() {
    for (hipEvent_t e : attn_events) (void)hipEventDestroy(e);
  }
};

// One blocking step request of a session in a step batcher.
struct BatchRequest {
  fah_decoder* session = nullptr;
  int32_t token = 0;
  int status = FAH_OK;
  std::string error;
  // Set by the leader after every other field, as its last access: the
  // requester may then read them without the batcher's lock and return.
  std::atomic<bool> done{false};
};

// Cross-context step batcher: greedy steps of sessions of one weight set,
// requested from different threads, run together as one lock-step batch.
struct fah_batcher {
  std::shared_ptr<Ctx> ctx;
  std::shared_ptr<DecoderWeights> wt;
  int max_positions = 0;
  std::chrono::microseconds window{0};
  std::mutex m;
  std::condition_variable cv;
  std::vector<BatchRequest*> pending;
  std::vector<fah_decoder*> joined;
  // Joined sessions that had no step in the last batch (busy elsewhere:
  // encoding, prefilling, idle between requests). The collector stops
  // waiting for them until they request a step again.
  std::vector<fah_decoder*> idle;
  std::atomic<bool> running{false};  // a leader is collecting or running a batch (written under m)
  std::atomic<int64_t> arrivals{0};  // steps requested so far (incremented under m)
  int64_t batches_run = 0, rows_run = 0;
  // The captured step of each batch size (the session table is rewritten
  // before each launch).
  std::unique_ptr<SessionBatch> by_size[fah::kFewFrames + 1];
};

namespace {

void upload(DeviceBuffer& dst, const void* src, size_t bytes, hipStream_t s) {
  dst.allocate(bytes);
  check(hipMemcpyAsync(dst.ptr, src, bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync H2D");
  check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

// Upload rows in the given order (row_index[i] = source row of storage row i).
// GGUF Q8_0 blocks on the host -> int8 plane + fp16 scale plane on the
// device (the split runs on the device; `raw` may be freed on return).
void upload_blocks(DeviceBuffer& q, DeviceBuffer& sc, const uint8_t* raw, size_t blocks, hipStream_t s) {
  DeviceBuffer staging;
  upload(staging, raw, blocks * 34, s);
  q.allocate(blocks * 32);
  sc.allocate(blocks * 2);
  check(fah::launch_unpack_q8_blocks(staging.as<uint8_t>(), (int64_t)blocks, q.as<int8_t>(), sc.as<uint16_t>(), s),
        "unpack Q8_0 blocks");
  check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

// Scale of block b of row r of a part, widened exactly to fp32.
float part_scale(const fah_q8_host* p, size_t r, int b, int B) {
  if (p->scales) return p->scales[r * B + b];
  const uint8_t* blk = p->blocks + (r * B + b) * 34;
  return half_bits_to_float((uint16_t)(blk[0] | (blk[1] << 8)));
}

// Upload rows in the given order (order[i] = (part, source row) of storage
// row i). With fp16 scales every row goes through the GGUF block layout and
// the device split (parts given as GGUF blocks are copied as they are);
// otherwise the int8 and fp32 planes are assembled on the host.
void upload_matrix(DeviceMatrix& m, const std::vector<const fah_q8_host*>& parts,
                   const std::vector<std::pair<int, int>>& order, int cols, bool half, hipStream_t s) {
  const int B = cols / 32;
  const size_t rows = order.size(), row_bytes = (size_t)B * 34;
  if (half) {
    std::vector<uint8_t> raw(rows * row_bytes);
    for (size_t i = 0; i < rows; ++i) {
      const fah_q8_host* p = parts[order[i].first];
      const size_t r = (size_t)order[i].second;
      uint8_t* dst = &raw[i * row_bytes];
      if (!p->quantized) {
        std::memcpy(dst, p->blocks + r * row_bytes, row_bytes);
        continue;
      }
      for (int b = 0; b < B; ++b) {
        const uint16_t h = float_to_half_bits(p->scales[r * B + b]);
        dst[34 * b] = (uint8_t)(h & 0xff);
        dst[34 * b + 1] = (uint8_t)(h >> 8);
        std::memcpy(dst + 34 * b + 2, p->quantized + r * cols + 32 * b, 32);
      }
    }
    upload_blocks(m.q, m.s, raw.data(), rows * B, s);
  } else {
    std::vector<int8_t> q(rows * cols);
    std::vector<float> fs(rows * B);
    for (size_t i = 0; i < rows; ++i) {
      const fah_q8_host* p = parts[order[i].first];
      const size_t r = (size_t)order[i].second;
      for (int b = 0; b < B; ++b) {
        fs[i * B + b] = part_scale(p, r, b, B);
        const int8_t* src = p->quantized ? p->quantized + r * cols + 32 * b
                                         : reinterpret_cast<const int8_t*>(p->blocks + (r * B + b) * 34 + 2);
        std::memcpy(&q[i * cols + 32 * b], src, 32);
      }
    }
    upload(m.q, q.data(), q.size(), s);
    upload(m.s, fs.data(), fs.size() * 4, s);
  }
  m.rows = (int)rows;
  m.cols = cols;
}

void validate_q8(const fah_q8_host* w, int rows, int cols, const char* name) {
  require(w && ((w->quantized && w->scales) || (!w->quantized && !w->scales && w->blocks)),
          std::string(name) + ": missing Q8 weight (int8 + scales, or GGUF blocks)");
  require(w->rows == rows && w->cols == cols,
          std::string(name) + ": shape " + std::to_string(w->rows) + "x" + std::to_string(w->cols) + " != " +
              std::to_string(rows) + "x" + std::to_string(cols));
}

int64_t matrix_bytes(const DeviceMatrix& m) { return (int64_t)m.q.bytes + (int64_t)m.s.bytes; }

fah::GemvArgs gemv_args(const DeviceMatrix& m) {
  fah::GemvArgs a{};
  a.w = m.q.as<int8_t>();
  a.ws = m.s.ptr;
  a.rows = m.rows;
  a.K = m.cols;
  a.group_rows = m.group_rows;
  return a;
}

// One decoder row through every layer (x -> x), then optionally the final
// norm, lm_head and greedy. Records onto the context stream (captured).
void enqueue_layers(fah_decoder* d, hipStream_t s) {
  const fah_decoder_config& c = d->cfg;
  int* pos = d->position.as<int>();
  for (int l = 0; l < c.layers; ++l) {
    fah::GemvArgs g = gemv_args(d->wt->qkv[l]);
    g.x = d->x.as<float>();
    g.norm_w = d->wt->attn_norm[l].as<float>();
    g.eps = c.eps;
    g.out = d->qkv_out.as<float>();
    g.out_rows = d->wt->qkv[l].rows;
    check(fah::launch_gemv(g, d->wt->half_scales, fah::kInputNorm, fah::kOutPlain, 1, s), "qkv gemv");

    size_t kv_layer = (size_t)c.kv_heads * c.capacity * c.head_size;
    fah::QkArgs qa{};
    qa.qkv = d->qkv_out.as<float>();
    qa.q_norm = d->wt->q_norm[l].as<float>();
    qa.k_norm = d->wt->k_norm[l].as<float>();
    qa.rope_cos = d->rope_cos.as<float>();
    qa.rope_sin = d->rope_sin.as<float>();
    qa.position = pos;
    qa.q_out = d->qh.as<float>();
    qa.kcache = d->kcache.as<_Float16>() + kv_layer * l;
    qa.vcache = d->vcache.as<_Float16>() + kv_layer * l;
    qa.heads = c.heads;
    qa.kv_heads = c.kv_heads;
    qa.head_size = c.head_size;
    qa.q_width = d->q_width;
    qa.kv_width = d->kv_width;
    qa.capacity = c.capacity;
    qa.eps = c.eps;
    check(fah::launch_qk_prepare(qa, s), "qk prepare");

    fah::AttnArgs at{};
    at.q = d->qh.as<float>();
    at.kcache = qa.kcache;
    at.vcache = qa.vcache;
    at.position = pos;
    at.scores = d->scores.as<float>();
    at.block_max = d->block_max.as<float>();
    at.exp_t = d->exp_t.as<double>();
    at.block_sum = d->block_sum.as<double>();
    at.exp_stride = fah::attention_exp_stride(c.capacity);
    at.out = d->attn.as<float>();
    at.heads = c.heads;
    at.kv_heads = c.kv_heads;
    at.head_size = c.head_size;
    at.capacity = c.capacity;
    at.divisor = std::sqrt((float)c.head_size);
    if (d->attention_times) check(hipEventRecord(d->attn_events[2 * l], s), "hipEventRecord");
    check(fah::launch_attention(at, 16, s), "attention");
    if (d->attention_times) check(hipEventRecord(d->attn_events[2 * l + 1], s), "hipEventRecord");

    fah::GemvArgs o = gemv_args(d->wt->wo[l]);
    o.x = d->attn.as<float>();
    o.out = d->a.as<float>();
    o.out_rows = c.width;
    o.resid = d->x.as<float>();
    check(fah::launch_gemv(o, d->wt->half_scales, fah::kInputFloat, fah::kOutResidual, 1, s), "o gemv");

    if (d->wt->persistent_layout) {
      // Gate/up stored in the persistent kernel's tiles: the few-frame GEMM
      // reads any tiling (norm + quantise first).
      int8_t* xq = d->row_q.as<int8_t>();
      float* xs = d->row_s.as<float>();
      check(fah::launch_norm_quantize_rows(d->a.as<float>(), 1, c.width, d->wt->ffn_norm[l].as<float>(), c.eps, xq, xs,
                                           s),
            "ffn_norm");
      fah::GemmArgs g{};
      g.w = d->wt->gateup[l].q.as<int8_t>();
      g.ws = d->wt->gateup[l].s.ptr;
      g.rows = c.ffn;
      g.K = c.width;
      g.xq = xq;
      g.xs = xs;
      g.frames = 1;
      g.out = d->h.as<float>();
      g.out_stride = c.ffn;
      g.split_base = d->wt->gu_base;
      g.split_extra = d->wt->gu_extra;
      g.gu_map = d->wt->gu_map.as<int>();
      check(fah::launch_gemm_few(g, d->wt->half_scales, fah::kGemmSwiGLU, s), "gate/up gemm");
    } else {
      fah::GemvArgs gu = gemv_args(d->wt->gateup[l]);
      gu.x = d->a.as<float>();
      gu.norm_w = d->wt->ffn_norm[l].as<float>();
      gu.eps = c.eps;
      gu.out = d->h.as<float>();
      gu.out_rows = c.ffn;
      check(fah::launch_gemv(gu, d->wt->half_scales, fah::kInputNorm, fah::kOutSwiGLU, 1, s), "gate/up gemv");
    }

    fah::GemvArgs dn = gemv_args(d->wt->down[l]);
    dn.x = d->h.as<float>();
    dn.out = d->x.as<float>();
    dn.out_rows = c.width;
    dn.resid = d->a.as<float>();
    check(fah::launch_gemv(dn, d->wt->half_scales, fah::kInputFloat, fah::kOutResidual, 1, s), "down gemv");
  }
}

const DeviceMatrix& head_matrix(const fah_decoder* d) { return d->wt->tied ? d->wt->embed : d->wt->lm_head; }

void enqueue_head(fah_decoder* d, hipStream_t s) {
  fah::GemvArgs g = gemv_args(head_matrix(d));
  g.x = d->x.as<float>();
  g.norm_w = d->wt->output_norm.as<float>();
  g.eps = d->cfg.eps;
  g.out = d->logits.as<float>();
  g.out_rows = d->cfg.vocab;
  g.partial_keys = d->keys.as<unsigned long long>();
  check(fah::launch_gemv(g, d->wt->half_scales, fah::kInputNorm, fah::kOutGreedy, 1, s), "lm_head gemv");
  check(fah::launch_greedy_reduce(d->keys.as<unsigned long long>(), d->lm_groups, d->logits.as<float>(),
                                  d->token.as<int>(), s),
        "greedy");
}

// Per-decoder state over shared weights: RoPE tables for this capacity, the
// F16 KV cache, row buffers, token/position/history words and, on the
// persistent path, the tagged exchange buffers and the kernel's arguments.
void init_state(fah_decoder* d, hipStream_t s) {
  const fah_decoder_config& k = d->cfg;
  const int q_width = d->q_width, kv_width = d->kv_width, qkv_rows = q_width + 2 * kv_width;
  const int nb = 256;
  d->blocks = nb;
  const DeviceMatrix& head = head_matrix(d);
  // RoPE table with the C runtime's powf/cosf/sinf (QwenDecoder.cs:78-95).
  int half_hs = k.head_size / 2;
  std::vector<float> freq(half_hs), cs((size_t)k.capacity * half_hs), sn((size_t)k.capacity * half_hs);
  for (int i = 0; i < half_hs; ++i) freq[i] = powf(k.rope_base, (-2.0f * (float)i) / (float)k.head_size);
  for (int t = 0; t < k.capacity; ++t)
    for (int i = 0; i < half_hs; ++i) {
      float angle = (float)t * freq[i];
      cs[(size_t)t * half_hs + i] = cosf(angle);
      sn[(size_t)t * half_hs + i] = sinf(angle);
    }
  upload(d->rope_cos, cs.data(), cs.size() * 4, s);
  upload(d->rope_sin, sn.data(), sn.size() * 4, s);

  const char* at_env = std::getenv("FAH_ATTENTION_TIMES");
  if (at_env && at_env[0] == '1') {
    d->attention_times = true;
    d->attn_events.assign(2 * (size_t)k.layers, nullptr);
    for (hipEvent_t& e : d->attn_events) check(hipEventCreate(&e), "hipEventCreate");
  }
  size_t kv_elems = (size_t)k.layers * k.kv_heads * k.capacity * k.head_size;
  d->kcache.allocate(kv_elems * 2);
  d->vcache.allocate(kv_elems * 2);
  check(hipMemsetAsync(d->kcache.ptr, 0, kv_elems * 2, s), "memset kv");
  check(hipMemsetAsync(d->vcache.ptr, 0, kv_elems * 2, s), "memset kv");
  d->x.allocate((size_t)k.width * 4);
  d->qkv_out.allocate((size_t)qkv_rows * 4);
  d->qh.allocate((size_t)q_width * 4);
  // Scores, then probabilities, [heads][capacity]; the values kernel copies
  // each head's row in 16-byte pieces, up to 3 floats past the capacity.
  d->scores.allocate(((size_t)k.heads * k.capacity + 4) * 4);
  d->block_max.allocate((size_t)k.heads * ((k.capacity + 255) / 256) * 4);
  d->block_sum.allocate((size_t)k.heads * ((k.capacity + 255) / 256) * 8);
  d->exp_t.allocate((size_t)k.heads * 8 * fah::attention_exp_stride(k.capacity) * 8);
  d->attn.allocate((size_t)q_width * 4);
  d->a.allocate((size_t)k.width * 4);
  d->h.allocate((size_t)k.ffn * 4);
  d->row_q.allocate((size_t)std::max(std::max(k.width, q_width), k.ffn));
  d->row_s.allocate((size_t)std::max(std::max(k.width, q_width), k.ffn) / 32 * 4);
  d->logits.allocate((size_t)k.vocab * 4);
  d->lm_groups = (k.vocab + head.group_rows - 1) / head.group_rows;
  d->keys.allocate((size_t)d->lm_groups * 8);
  d->token.allocate(16);
  d->position.allocate(16);
  d->history.allocate((size_t)k.capacity * 4 + 16);
  d->history_count.allocate(16);
  check(hipMemsetAsync(d->token.ptr, 0, 16, s), "memset");
  check(hipMemsetAsync(d->position.ptr, 0, 16, s), "memset");
  check(hipMemsetAsync(d->history_count.ptr, 0, 16, s), "memset");
  if (d->persistent) {
    auto tagged = [&](DeviceBuffer& b, size_t words) {
      b.allocate(words * 8);
      check(hipMemsetAsync(b.ptr, 0, words * 8, s), "memset tagged");
    };
    tagged(d->tx, k.width);
    tagged(d->tqkv, qkv_rows);
    tagged(d->tatt, q_width);
    tagged(d->ta, k.width);
    tagged(d->th, k.ffn);
    tagged(d->tkeys, 2 * nb);
    tagged(d->tattq, (size_t)fah::qblock_words(q_width));
    tagged(d->thq, (size_t)fah::qblock_words(k.ffn));
    const int score_stride = (k.capacity + 127) & ~127;
    tagged(d->tscore, (size_t)k.heads * score_stride);
    tagged(d->tready, 2 * (size_t)k.heads);
    d->epoch.allocate(16);
    d->error.allocate(16);
    unsigned one = 1;
    check(hipMemcpyAsync(d->epoch.ptr, &one, 4, hipMemcpyHostToDevice, s), "epoch");
    check(hipMemsetAsync(d->error.ptr, 0, 16, s), "memset error");
    fah::PersistentArgs& a = d->pargs;
    a.layer_table = d->wt->layer_table.as<fah::PersistentLayer>();
    a.layers = k.layers;
    a.embed_q = d->wt->embed.q.as<int8_t>();
    a.embed_s = d->wt->embed.s.as<_Float16>();
    a.head_q = head.q.as<int8_t>();
    a.head_s = head.s.as<_Float16>();
    a.output_norm = d->wt->output_norm.as<float>();
    a.rope_cos = d->rope_cos.as<float>();
    a.rope_sin = d->rope_sin.as<float>();
    a.kcache = d->kcache.as<_Float16>();
    a.vcache = d->vcache.as<_Float16>();
    a.width = k.width;
    a.heads = k.heads;
    a.kv_heads = k.kv_heads;
    a.head_size = k.head_size;
    a.ffn = k.ffn;
    a.vocab = k.vocab;
    a.capacity = k.capacity;
    a.q_width = q_width;
    a.kv_width = kv_width;
    a.eps = k.eps;
    a.divisor = std::sqrt((float)k.head_size);
    const char* l2 = std::getenv("FAH_LOCAL_L2");
    a.local_l2 = (l2 && l2[0] == '0') ? 0 : (fah::persistent_xcd_round_robin(s) ? 1 : 0);
    a.rq = qkv_rows / nb;
    a.ro = k.width / nb;
    a.rgu = k.ffn / nb;
    a.rd = k.width / nb;
    a.head_chunks = (k.vocab + 31) / 32;
    a.tx = d->tx.as<unsigned long long>();
    a.tqkv = d->tqkv.as<unsigned long long>();
    a.tatt = d->tatt.as<unsigned long long>();
    a.ta = d->ta.as<unsigned long long>();
    a.th = d->th.as<unsigned long long>();
    a.tkeys = d->tkeys.as<unsigned long long>();
    a.tattq = d->tattq.as<unsigned long long>();
    a.thq = d->thq.as<unsigned long long>();
    a.tscore = d->tscore.as<unsigned long long>();
    a.tready = d->tready.as<unsigned long long>();
    a.score_stride = score_stride;
    // FAH_LONG_FROM: the long-cache attention from this position on (at
    // most, and by default, the positions the attention workgroups hold).
    a.long_from = fah::persistent_exact_positions();
    if (const char* lf = std::getenv("FAH_LONG_FROM")) a.long_from = std::max(0, std::min(a.long_from, std::atoi(lf)));
    // Every position the persistent kernel holds runs on it: with the value
    // sums spread over the projection workgroups it is the faster step at
    // every length it takes (measured, a token, persistent against the
    // multi-kernel step over these weights: 1.34 / 1.79 ms at 4,096 cached
    // positions). Past that the multi-kernel step runs.
    // FAH_PERSISTENT_POSITIONS moves the switch.
    d->persistent_positions = fah::persistent_max_positions();
    if (const char* pp = std::getenv("FAH_PERSISTENT_POSITIONS"))
      d->persistent_positions = std::max(0, std::min(fah::persistent_max_positions(), std::atoi(pp)));
    a.x_in = d->x.as<float>();
    a.position = d->position.as<int>();
    a.token = d->token.as<int>();
    a.history = d->history.as<int>();
    a.history_count = d->history_count.as<int>();
    a.epoch = d->epoch.as<unsigned>();
    a.error = d->error.as<unsigned>();
    a.logits = d->logits.as<float>();
    const char* tl = std::getenv("FAH_TIMELINE");
    if (tl && tl[0] == '1') {
      d->timeline.allocate((size_t)nb * fah::kTimelineEvents * 8);
      check(hipMemsetAsync(d->timeline.ptr, 0, (size_t)nb * fah::kTimelineEvents * 8, s), "memset timeline");
      a.timeline = d->timeline.as<unsigned long long>();
    }
  }
}

void enqueue_kind(fah_decoder* d, int kind, hipStream_t s);

// Rows per prefill pass: the GEMMs see all of them at once.
constexpr int kPrefillChunk = 1024;

// QwenDecoder.Decode for frames > 1 (QwenDecoder.cs:161-271): every layer
// runs over all rows of a chunk -- norm + quantise per row, MFMA Q8_0 GEMMs
// with the per-row block order, QK-norm/RoPE/KV write per row, causal
// attention per (head, row) -- then the last row's final norm, lm_head and
// greedy when logits are wanted. `x` is the device copy of the rows.
void prefill(fah_decoder* d, const float* x, int frames, bool logits, hipStream_t s) {
  const fah_decoder_config& c = d->cfg;
  const int qkv_rows = d->q_width + 2 * d->kv_width;
  const int widest = std::max(std::max(c.width, d->q_width), c.ffn);
  const size_t kv_layer = (size_t)c.kv_heads * c.capacity * c.head_size;
  for (int done = 0; done < frames; done += kPrefillChunk) {
    const int T = std::min(kPrefillChunk, frames - done);
    d->pf_x.ensure((size_t)T * c.width * 4);
    d->pf_a.ensure((size_t)T * c.width * 4);
    d->pf_qkv.ensure((size_t)T * qkv_rows * 4);
    d->pf_q.ensure((size_t)T * d->q_width * 4);
    d->pf_h.ensure((size_t)T * c.ffn * 4);
    d->pf_xq.ensure((size_t)T * widest);
    d->pf_xs.ensure((size_t)T * widest / 32 * 4);
    check(hipMemcpyAsync(d->pf_x.ptr, x + (size_t)done * c.width, (size_t)T * c.width * 4, hipMemcpyDeviceToDevice, s),
          "D2D prefill rows");
    int8_t* xq = d->pf_xq.as<int8_t>();
    float* xs = d->pf_xs.as<float>();
    // More rows than the few-frame kernel takes: the SwiGLU GEMM writes the
    // Q8_0 blocks of its output itself (into pf_hq / pf_hs, which the down
    // projection reads), with no separate quantisation pass.
    const bool fused_h = !fah::few_frame_groups(c.ffn, c.width, T, fah::kGemmSwiGLU) && c.ffn % 32 == 0;
    if (fused_h) {
      d->pf_hq.ensure((size_t)T * c.ffn);
      d->pf_hs.ensure((size_t)T * c.ffn / 32 * 4);
    }
    auto gemm = [&](const DeviceMatrix& m, int rows, float* out, int stride, const float* resid, int mode,
                    const int8_t* in_q = nullptr, const float* in_s = nullptr, int8_t* out_q = nullptr,
                    float* out_s = nullptr) {
      fah::GemmArgs g{};
      g.w = m.q.as<int8_t>();
      g.ws = m.s.ptr;
      g.rows = rows;
      g.K = m.cols;
      g.xq = in_q ? in_q : xq;
      g.xs = in_s ? in_s : xs;
      g.out_q = out_q;
      g.out_s = out_s;
      g.frames = T;
      g.out = out;
      g.out_stride = stride;
      g.resid = resid;
      g.split_base = d->wt->gu_base;
      g.split_extra = d->wt->gu_extra;
      g.gu_map = d->wt->gu_map.as<int>();
      if (fah::few_frame_groups(rows, m.cols, T, mode)) check(fah::launch_gemm_few(g, d->wt->half_scales, mode, s), "prefill gemm");
      else check(fah::launch_gemm(g, d->wt->half_scales, mode, s), "prefill gemm");
    };
    for (int l = 0; l < c.layers; ++l) {
      check(fah::launch_norm_quantize_rows(d->pf_x.as<float>(), T, c.width, d->wt->attn_norm[l].as<float>(), c.eps, xq, xs,
                                           s),
            "prefill attn_norm");
      gemm(d->wt->qkv[l], qkv_rows, d->pf_qkv.as<float>(), qkv_rows, nullptr, fah::kGemmPlain);
      fah::QkArgs qa{};
      qa.qkv = d->pf_qkv.as<float>();
      qa.q_norm = d->wt->q_norm[l].as<float>();
      qa.k_norm = d->wt->k_norm[l].as<float>();
      qa.rope_cos = d->rope_cos.as<float>();
      qa.rope_sin = d->rope_sin.as<float>();
      qa.position = d->position.as<int>();
      qa.q_out = d->pf_q.as<float>();
      qa.kcache = d->kcache.as<_Float16>() + kv_layer * l;
      qa.vcache = d->vcache.as<_Float16>() + kv_layer * l;
      qa.heads = c.heads;
      qa.kv_heads = c.kv_heads;
      qa.head_size = c.head_size;
      qa.q_width = d->q_width;
      qa.kv_width = d->kv_width;
      qa.capacity = c.capacity;
      qa.eps = c.eps;
      qa.frames = T;
      check(fah::launch_qk_prepare(qa, s), "prefill qk prepare");
      fah::PrefillAttnArgs pa{};
      pa.q = d->pf_q.as<float>();
      pa.kcache = qa.kcache;
      pa.vcache = qa.vcache;
      pa.xq = xq;  // quantised for the o projection inside the kernel
      pa.xs = xs;
      pa.frames = T;
      pa.position = d->host_position + done;
      pa.heads = c.heads;
      pa.kv_heads = c.kv_heads;
      pa.head_size = c.head_size;
      pa.capacity = c.capacity;
      pa.divisor = std::sqrt((float)c.head_size);
      check(fah::launch_attn_prefill(pa, s), "prefill attention");
      gemm(d->wt->wo[l], c.width, d->pf_a.as<float>(), c.width, d->pf_x.as<float>(), fah::kGemmResidual);
      check(fah::launch_norm_quantize_rows(d->pf_a.as<float>(), T, c.width, d->wt->ffn_norm[l].as<float>(), c.eps, xq, xs,
                                           s),
            "prefill ffn_norm");
      if (fused_h) {
        gemm(d->wt->gateup[l], c.ffn, d->pf_h.as<float>(), c.ffn, nullptr, fah::kGemmSwiGLU, nullptr, nullptr,
             d->pf_hq.as<int8_t>(), d->pf_hs.as<float>());
        gemm(d->wt->down[l], c.width, d->pf_x.as<float>(), c.width, d->pf_a.as<float>(), fah::kGemmResidual,
             d->pf_hq.as<int8_t>(), d->pf_hs.as<float>());
      } else {
        gemm(d->wt->gateup[l], c.ffn, d->pf_h.as<float>(), c.ffn, nullptr, fah::kGemmSwiGLU);
        check(fah::launch_norm_quantize_rows(d->pf_h.as<float>(), T, c.ffn, nullptr, 0.0f, xq, xs, s),
              "prefill quantise ffn");
        gemm(d->wt->down[l], c.width, d->pf_x.as<float>(), c.width, d->pf_a.as<float>(), fah::kGemmResidual);
      }
    }
    check(fah::launch_advance(d->position.as<int>(), T, s), "advance");
    if (logits && done + T == frames) {
      check(hipMemcpyAsync(d->x.ptr, d->pf_x.as<float>() + (size_t)(T - 1) * c.width, (size_t)c.width * 4,
                           hipMemcpyDeviceToDevice, s),
            "D2D last row");
      enqueue_head(d, s);
    }
  }
}

// Row-by-row decode below this many frames, for widths the GEMMs do not
// take (multiples of 128 up to 3072), and with FAH_PREFILL=0.
bool use_prefill(const fah_decoder* d, int frames) {
  const char* env = std::getenv("FAH_PREFILL");
  const fah_decoder_config& c = d->cfg;
  auto fits = [](int k) { return k % 128 == 0 && k <= 3072; };
  return frames >= 4 && fits(c.width) && fits(c.ffn) && fits(d->q_width) && !(env && env[0] == '0');
}

hipGraphExec_t capture(fah_decoder* d, int kind) {
  hipStream_t s = d->ctx->stream;
  hipGraph_t graph = nullptr;
  check(hipStreamSynchronize(s), "hipStreamSynchronize");
  check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  try {
    enqueue_kind(d, kind, s);
  } catch (...) {
    hipGraph_t dead = nullptr;
    (void)hipStreamEndCapture(s, &dead);
    if (dead) (void)hipGraphDestroy(dead);
    throw;
  }
  check(hipStreamEndCapture(s, &graph), "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  check(e, "hipGraphInstantiate");
  return exec;
}

// Error word values: bit 0 a bounded wait expired (an exchange never came),
// bit 1 preset by the host (fah_decoder_fail_next_step), bit 2 the device
// position lay outside the cache. While the word is set every launch ends at
// its entry check, so the steps enqueued after a failed one do nothing.
constexpr unsigned kErrorTimeout = 1u, kErrorPreset = 2u, kErrorPosition = 4u;

// After a persistent launch: if the error word is set, restore the device
// state from the host's and throw. The epoch moves past every generation the
// failed launch may have published (so none of its words can look current
// to the next launch), the device position returns to the host position, the
// history is emptied and the word cleared; the logits of the failed call are
// not valid, so the caller decodes again before greedy or generate.
void recover_step_error(fah_decoder* d) {
  if (!d->persistent) return;
  hipStream_t s = d->ctx->stream;
  unsigned e = 0, epoch = 0;
  check(hipMemcpyAsync(&e, d->error.ptr, 4, hipMemcpyDeviceToHost, s), "D2H error word");
  check(hipStreamSynchronize(s), "hipStreamSynchronize");
  if (!e) return;
  d->fail_sessions = false;  // the preset, if any, is consumed by this step
  check(hipMemcpyAsync(&epoch, d->epoch.ptr, 4, hipMemcpyDeviceToHost, s), "D2H epoch");
  check(hipStreamSynchronize(s), "hipStreamSynchronize");
  epoch += 2;
  const int position = d->host_position, zero = 0;
  check(hipMemcpyAsync(d->epoch.ptr, &epoch, 4, hipMemcpyHostToDevice, s), "H2D epoch");
  check(hipMemcpyAsync(d->position.ptr, &position, 4, hipMemcpyHostToDevice, s), "H2D position");
  check(hipMemcpyAsync(d->history_count.ptr, &zero, 4, hipMemcpyHostToDevice, s), "H2D history count");
  check(hipMemcpyAsync(d->error.ptr, &zero, 4, hipMemcpyHostToDevice, s), "H2D error word");
  check(hipStreamSynchronize(s), "hipStreamSynchronize");
  d->have_logits = false;
  if (e & kErrorTimeout) {
    // A launch whose workgroups were not dealt to the XCDs in turn leaves a
    // role unfilled and times out: later steps use placement-free roles.
    const bool was_local = d->pargs.local_l2 != 0;
    d->pargs.local_l2 = 0;
    throw DeviceError{was_local ? "persistent decode step: an exchange timed out (XCD-local roles are now off)"
                                : "persistent decode step: an exchange timed out (workgroups not co-resident?)"};
  }
  if (e & kErrorPosition) throw DeviceError{"persistent decode step: device position outside the cache"};
  throw DeviceError{"persistent decode step: stopped by the host (fah_decoder_fail_next_step)"};
}

// Enqueue one decoder row: kind 0 = layers only, 1 = layers + lm_head +
// greedy, 2 = embedding of the device token + layers + lm_head + greedy.
void enqueue_kind(fah_decoder* d, int kind, hipStream_t s) {
  if (kind == 2)
    check(fah::launch_embed(d->wt->embed.q.as<int8_t>(), d->wt->embed.s.ptr, d->wt->half_scales, d->cfg.width, d->cfg.vocab,
                            d->token.as<int>(), d->x.as<float>(), d->history.as<int>(),
                            d->history_count.as<int>(), s),
          "embed");
  enqueue_layers(d, s);
  if (kind >= 1) enqueue_head(d, s);
  check(fah::launch_advance(d->position.as<int>(), 1, s), "advance");
}

// FAH_GRAPHS=0 launches the kernels directly instead of replaying captured
// graphs (profilers that do not follow stream capture).
bool use_graphs() {
  static const bool on = [] {
    const char* v = std::getenv("FAH_GRAPHS");
    return !(v && v[0] == '0');
  }();
  return on;
}

// `position` is the position of the row this step decodes. A
// persistent-layout decoder takes the persistent kernel below
// d->persistent_positions and the multi-kernel step from it on.
void run_kind(fah_decoder* d, int kind, hipStream_t s, int position) {
  if (d->persistent && position < d->persistent_positions) {
    fah::PersistentArgs a = d->pargs;
    a.mode = kind;
    check(fah::launch_decode_step(a, d->blocks, s, position >= a.long_from), "persistent decode step");
    return;
  }
  if (d->attention_times) {
    enqueue_kind(d, kind, s);
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    for (int l = 0; l < d->cfg.layers; ++l) {
      float ms = 0.0f;
      check(hipEventElapsedTime(&ms, d->attn_events[2 * l], d->attn_events[2 * l + 1]), "hipEventElapsedTime");
      d->attn_ms += ms;
    }
    ++d->attn_steps;
    return;
  }
  if (!use_graphs()) {
    enqueue_kind(d, kind, s);
    return;
  }
  hipGraphExec_t* slot = kind == 0 ? &d->graph_row : kind == 1 ? &d->graph_logits : &d->graph_step;
  if (!*slot) *slot = capture(d, kind);
  check(hipGraphLaunch(*slot, s), "hipGraphLaunch");
}

// ---- lock-step sessions ---------------------------------------------------

// Upper bound on the positions of lock-step sessions (the batched attention
// keeps a row's probabilities in 60 KiB of LDS).
constexpr int kSessionPositions = 15360;

// One greedy step of every session at once: the embeddings of their tokens,
// the layers over all rows (MFMA Q8_0 GEMMs with the per-row block order;
// per-session QK-norm, RoPE, KV write and attention), the final norm,
// lm_head and a greedy pick per row. Each row's arithmetic is the
// single-session step's, so each session's tokens are its own.
void enqueue_sessions_step(const fah_decoder* d, SessionBatch& b, hipStream_t s) {
  const fah_decoder_config& c = d->cfg;
  const DecoderWeights& w = *d->wt;
  const int S = (int)b.members.size();
  const int qkv_rows = d->q_width + 2 * d->kv_width;
  const fah::SessionRef* table = b.table.as<fah::SessionRef>();
  int8_t* xq = b.xq.as<int8_t>();
  float* xs = b.xs.as<float>();
  auto norm_quantize = [&](const float* x, int K, const DeviceBuffer* norm) {
    check(fah::launch_norm_quantize_rows(x, S, K, norm ? norm->as<float>() : nullptr, norm ? c.eps : 0.0f, xq, xs, s),
          "session norm/quantise");
  };
  auto gemm = [&](const DeviceMatrix& m, int rows, float* out, const float* resid, int mode) {
    fah::GemmArgs g{};
    g.w = m.q.as<int8_t>();
    g.ws = m.s.ptr;
    g.rows = rows;
    g.K = m.cols;
    g.xq = xq;
    g.xs = xs;
    g.frames = S;
    g.out = out;
    g.out_stride = rows;
    g.resid = resid;
    g.split_base = w.gu_base;
    g.split_extra = w.gu_extra;
    g.gu_map = w.gu_map.as<int>();
    g.keys = b.keys.as<unsigned long long>();
    if (fah::few_frame_groups(rows, m.cols, S, mode)) check(fah::launch_gemm_few(g, w.half_scales, mode, s), "session gemm");
    else check(fah::launch_gemm(g, w.half_scales, mode == fah::kGemmGreedy ? fah::kGemmPlain : mode, s), "session gemm");
  };
  check(fah::launch_session_embed(w.embed.q.as<int8_t>(), w.embed.s.ptr, w.half_scales, c.width, c.vocab, table, S,
                                  b.x.as<float>(), s),
        "session embed");
  // One launch for every layer and the output norm (its rows land in xq/xs).
  if (b.fused) check(fah::launch_session_step(b.sargs, s), "session step");
  for (int l = 0; l < c.layers && !b.fused; ++l) {
    norm_quantize(b.x.as<float>(), c.width, &w.attn_norm[l]);
    gemm(w.qkv[l], qkv_rows, b.qkv.as<float>(), nullptr, fah::kGemmPlain);
    // Attention with the QK-norm, RoPE and K/V row write of each session's
    // new position done in the same kernel.
    fah::PrefillAttnArgs pa{};
    pa.qkv = b.qkv.as<float>();
    pa.q_norm = w.q_norm[l].as<float>();
    pa.k_norm = w.k_norm[l].as<float>();
    pa.eps = c.eps;
    pa.q_width = d->q_width;
    pa.kv_width = d->kv_width;
    pa.xq = xq;
    pa.xs = xs;
    pa.frames = S;
    pa.heads = c.heads;
    pa.kv_heads = c.kv_heads;
    pa.head_size = c.head_size;
    pa.divisor = std::sqrt((float)c.head_size);
    pa.sessions = table;
    pa.layer = l;
    pa.max_positions = b.max_positions;
    check(fah::launch_attn_prefill(pa, s), "session attention");
    gemm(w.wo[l], c.width, b.a.as<float>(), b.x.as<float>(), fah::kGemmResidual);
    norm_quantize(b.a.as<float>(), c.width, &w.ffn_norm[l]);
    gemm(w.gateup[l], c.ffn, b.h.as<float>(), nullptr, fah::kGemmSwiGLU);
    norm_quantize(b.h.as<float>(), c.ffn, nullptr);
    gemm(w.down[l], c.width, b.x.as<float>(), b.a.as<float>(), fah::kGemmResidual);
  }
  if (!b.fused) norm_quantize(b.x.as<float>(), c.width, &w.output_norm);
  const int head_groups = fah::few_frame_groups(c.vocab, c.width, S, fah::kGemmGreedy);
  require(head_groups > 0, "lock-step sessions: the lm_head shape does not fit the few-frame kernel");
  gemm(head_matrix(d), c.vocab, b.logits.as<float>(), nullptr, fah::kGemmGreedy);
  check(fah::launch_greedy_keys(b.keys.as<unsigned long long>(), head_groups, b.logits.as<float>(), c.vocab, table,
                                S, s),
        "session greedy");
}

// Session references of `sessions` into b.table, ordered on the stream; the
// captured step reads the table when it runs, so a batch's graph serves any
// sessions of its size.
// The device table of the sessions' buffers, uploaded only when it differs
// from the last upload (a recurring batch keeps its table).
void upload_session_table(SessionBatch& b, fah_decoder* const* sessions, int count, hipStream_t s) {
  std::vector<fah::SessionRef> table(count, fah::SessionRef{});
  for (int i = 0; i < count; ++i) {
    const fah_decoder* d = sessions[i];
    fah::SessionRef& r = table[i];
    r.kcache = d->kcache.as<_Float16>();
    r.vcache = d->vcache.as<_Float16>();
    r.rope_cos = d->rope_cos.as<float>();
    r.rope_sin = d->rope_sin.as<float>();
    r.position = d->position.as<int>();
    r.token = d->token.as<int>();
    r.history = d->history.as<int>();
    r.history_count = d->history_count.as<int>();
    r.capacity = d->cfg.capacity;
  }
  if (b.host_table.size() == table.size() &&
      std::memcmp(b.host_table.data(), table.data(), table.size() * sizeof(fah::SessionRef)) == 0)
    return;
  b.host_table = std::move(table);
  check(hipMemcpyAsync(b.table.ptr, b.host_table.data(), (size_t)count * sizeof(fah::SessionRef),
                       hipMemcpyHostToDevice, s),
        "H2D session table");
}

// Whether `count` sessions of d0's weights with positions below `bound` step
// on the one-launch layers (fah_sessions.hip): a shape it is built for, fp16
// block scales, every position within what an attention workgroup stages,
// and a device whose CUs hold all of its workgroups at once.
// FAH_SESSION_STEP=0 keeps the kernel-per-projection step.
bool session_step_fits(const fah_decoder* d0, int count, int bound) {
  static const bool on = [] {
    const char* v = std::getenv("FAH_SESSION_STEP");
    return !(v && v[0] == '0');
  }();
  const fah_decoder_config& k = d0->cfg;
  if (!on || !d0->wt->half_scales || bound > fah::session_step_positions() || count * k.heads > fah::session_step_groups())
    return false;
  if (!fah::session_step_supported(k.width, k.heads, k.kv_heads, k.head_size, k.ffn)) return false;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, d0->ctx->device) != hipSuccess) return false;
  static const int fit1024 = fah::session_step_blocks_per_cu(1024), fit512 = fah::session_step_blocks_per_cu(512);
  return cus >= fah::session_step_groups() && (k.width == 1024 ? fit1024 : fit512) >= 1;
}

// The one-launch step's buffers and arguments for batch b (zeroed exchange
// words, so that no word carries a generation before it is written).
void prepare_session_step(const fah_decoder* d0, SessionBatch& b, int count, hipStream_t s) {
  const fah_decoder_config& k = d0->cfg;
  const DecoderWeights& w = *d0->wt;
  std::vector<fah::PersistentLayer> layers(k.layers);
  for (int l = 0; l < k.layers; ++l) {
    fah::PersistentLayer& e = layers[l];
    e.wqkv = w.qkv[l].q.as<int8_t>();
    e.sqkv = w.qkv[l].s.as<_Float16>();
    e.wo = w.wo[l].q.as<int8_t>();
    e.so = w.wo[l].s.as<_Float16>();
    e.wgu = w.gateup[l].q.as<int8_t>();
    e.sgu = w.gateup[l].s.as<_Float16>();
    e.wd = w.down[l].q.as<int8_t>();
    e.sd = w.down[l].s.as<_Float16>();
    e.attn_norm = w.attn_norm[l].as<float>();
    e.q_norm = w.q_norm[l].as<float>();
    e.k_norm = w.k_norm[l].as<float>();
    e.ffn_norm = w.ffn_norm[l].as<float>();
  }
  upload(b.layer_table, layers.data(), layers.size() * sizeof(fah::PersistentLayer), s);
  const size_t qkv_rows = (size_t)d0->q_width + 2 * (size_t)d0->kv_width;
  // Every layer has its own exchange words (the gate/up maxima excepted).
  const size_t L = (size_t)k.layers;
  const size_t words[8] = {L * count * k.width,       L * count * k.width / 4, L * count * qkv_rows,
                           L * count * d0->q_width / 4, L * count * k.width,     L * count * k.width / 4,
                           (size_t)fah::session_step_groups() * 16, L * count * k.ffn / 4};
  size_t total = 0;
  for (size_t n : words) total += n;
  b.exchange.allocate(total * 8);
  b.epoch.allocate(16);
  b.error.allocate(16);
  check(hipMemsetAsync(b.exchange.ptr, 0, total * 8, s), "clear exchange words");
  check(hipMemsetAsync(b.epoch.ptr, 0, 16, s), "clear epoch");
  check(hipMemsetAsync(b.error.ptr, 0, 16, s), "clear error word");
  check(hipStreamSynchronize(s), "hipStreamSynchronize");
  unsigned long long* at[8];
  unsigned long long* p = b.exchange.as<unsigned long long>();
  for (int i = 0; i < 8; ++i) {
    at[i] = p;
    p += words[i];
  }
  fah::SessionStepArgs& a = b.sargs;
  a.layer_table = b.layer_table.as<fah::PersistentLayer>();
  a.layers = k.layers;
  a.width = k.width;
  a.heads = k.heads;
  a.kv_heads = k.kv_heads;
  a.head_size = k.head_size;
  a.ffn = k.ffn;
  a.output_norm = w.output_norm.as<float>();
  a.sessions = b.table.as<fah::SessionRef>();
  a.S = count;
  a.max_positions = b.max_positions;
  a.gu_map = w.gu_map.as<int>();
  a.gu_base = w.gu_base;
  a.gu_extra = w.gu_extra;
  a.eps = k.eps;
  a.divisor = std::sqrt((float)k.head_size);
  a.x_in = b.x.as<float>();
  a.xq_out = b.xq.as<int8_t>();
  a.xs_out = b.xs.as<float>();
  a.tx = at[0];
  a.txq = at[1];
  a.tqkv = at[2];
  a.tattq = at[3];
  a.ta = at[4];
  a.taq = at[5];
  a.tmax = at[6];
  a.thq = at[7];
  a.epoch = b.epoch.as<unsigned>();
  a.error = b.error.as<unsigned>();
  b.fused = true;
}

// After the steps of a one-launch batch: if a bounded wait expired, move
// the epoch past every generation the failed launches may have published,
// clear the error word, return every session's device position to its
// host position with an empty history, and throw. The sessions' logits are
// not valid afterwards (decode again before the next greedy step).
void recover_session_step_read(SessionBatch& b, fah_decoder* const* sessions, int count, unsigned e, unsigned epoch,
                               hipStream_t s);

void recover_session_step(SessionBatch& b, fah_decoder* const* sessions, int count, hipStream_t s) {
  if (!b.fused) return;
  unsigned e = 0, epoch = 0;
  check(hipMemcpyAsync(&e, b.error.ptr, 4, hipMemcpyDeviceToHost, s), "D2H error word");
  check(hipMemcpyAsync(&epoch, b.epoch.ptr, 4, hipMemcpyDeviceToHost, s), "D2H epoch");
  check(hipStreamSynchronize(s), "hipStreamSynchronize");
  recover_session_step_read(b, sessions, count, e, epoch, s);
}

// The same with the error word and epoch already read back (e, epoch).
void recover_session_step_read(SessionBatch& b, fah_decoder* const* sessions, int count, unsigned e, unsigned epoch,
                               hipStream_t s) {
  if (!b.fused || !e) return;
  epoch += 2;
  const unsigned zero = 0;
  check(hipMemcpyAsync(b.epoch.ptr, &epoch, 4, hipMemcpyHostToDevice, s), "H2D epoch");
  check(hipMemcpyAsync(b.error.ptr, &zero, 4, hipMemcpyHostToDevice, s), "H2D error word");
  std::vector<int> positions(count);
  for (int i = 0; i < count; ++i) {
    positions[i] = sessions[i]->host_position;
    check(hipMemcpyAsync(sessions[i]->position.ptr, &positions[i], 4, hipMemcpyHostToDevice, s), "H2D position");
    check(hipMemcpyAsync(sessions[i]->history_count.ptr, &zero, 4, hipMemcpyHostToDevice, s), "H2D history count");
    sessions[i]->have_logits = false;
  }
  check(hipStreamSynchronize(s), "hipStreamSynchronize");
  if (e & kErrorPreset) throw DeviceError{"lock-step sessions step: stopped by the host (fah_decoder_fail_next_step)"};
  throw DeviceError{"lock-step sessions step: an exchange timed out (workgroups not co-resident?)"};
}

// Before the steps of a one-launch batch: a session marked by
// fah_decoder_fail_next_step makes the batch's next launch end at its entry
// check (the word is set before the step is enqueued, never inside it); the
// mark and the session's own preset are consumed.
void preset_session_failure(SessionBatch& b, fah_decoder* const* sessions, int count, hipStream_t s) {
  if (!b.fused) return;
  bool any = false;
  const unsigned preset = kErrorPreset, zero = 0;
  for (int i = 0; i < count; ++i) {
    fah_decoder* d = sessions[i];
    if (!d->fail_sessions) continue;
    any = true;
    d->fail_sessions = false;
    if (d->persistent) check(hipMemcpyAsync(d->error.ptr, &zero, 4, hipMemcpyHostToDevice, s), "H2D error word");
  }
  if (!any) return;
  check(hipMemcpyAsync(b.error.ptr, &preset, 4, hipMemcpyHostToDevice, s), "H2D error word");
  check(hipStreamSynchronize(s), "hipStreamSynchronize");  // (the copies read these locals)
}

// Row buffers and the captured lock-step step of `count` sessions of d0's
// weights whose positions stay below `bound` (on the one-launch layers when
// `fused`).
std::unique_ptr<SessionBatch> make_session_batch(const fah_decoder* d0, int count, int bound, hipStream_t s,
                                                 bool fused) {
  auto b = std::make_unique<SessionBatch>();
  b->members.assign(count, nullptr);
  b->max_positions = bound;
  const fah_decoder_config& k = d0->cfg;
  const int widest = std::max(std::max(k.width, d0->q_width), k.ffn);
  b->table.allocate((size_t)count * sizeof(fah::SessionRef));
  b->x.allocate((size_t)count * k.width * 4);
  b->a.allocate((size_t)count * k.width * 4);
  b->qkv.allocate((size_t)count * (d0->q_width + 2 * d0->kv_width) * 4);
  b->q.allocate((size_t)count * d0->q_width * 4);
  b->h.allocate((size_t)count * k.ffn * 4);
  b->xq.allocate((size_t)count * widest);
  b->xs.allocate((size_t)count * (widest / 32) * 4);
  b->logits.allocate((size_t)count * k.vocab * 4);
  b->keys.allocate((size_t)count * std::max(1, fah::few_frame_groups(k.vocab, k.width, count, fah::kGemmGreedy)) * 8);
  if (fused) prepare_session_step(d0, *b, count, s);
  if (use_graphs()) {
    hipGraph_t graph = nullptr;
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
      enqueue_sessions_step(d0, *b, s);
    } catch (...) {
      hipGraph_t dead = nullptr;
      (void)hipStreamEndCapture(s, &dead);
      if (dead) (void)hipGraphDestroy(dead);
      throw;
    }
    check(hipStreamEndCapture(s, &graph), "hipStreamEndCapture");
    hipError_t e = hipGraphInstantiate(&b->graph, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    check(e, "hipGraphInstantiate");
  }
  return b;
}

// Checks shared by the lock-step entry points: sessions of one weight set,
// distinct, holding logits, with room for `steps` more positions; returns
// the position bound the batch's step is sized for.
int check_sessions(fah_decoder* const* sessions, int count, int steps) {
  require(count >= 1 && count <= fah::kFewFrames, "at most " + std::to_string(fah::kFewFrames) + " sessions per batch");
  const fah_decoder* d0 = sessions[0];
  require(d0 != nullptr, "session is NULL");
  require(d0->cfg.width % 128 == 0 && d0->cfg.ffn % 128 == 0 && d0->q_width % 128 == 0 && d0->cfg.ffn <= 3072,
          "lock-step sessions need projection widths that are multiples of 128, at most 3072");
  int bound = 0;
  for (int i = 0; i < count; ++i) {
    const fah_decoder* d = sessions[i];
    require(d != nullptr, "session is NULL");
    require(d->wt == d0->wt && d->ctx == d0->ctx, "sessions must share one decoder's weights");
    for (int j = 0; j < i; ++j) require(sessions[j] != d, "a session appears twice");
    if (!d->have_logits) throw StateError{"session " + std::to_string(i) + " has no logits: decode with logits first"};
    require(d->host_position + steps <= d->cfg.capacity, "Decoder context exhausted");
    require(d->host_position + steps <= kSessionPositions,
            "lock-step sessions are limited to " + std::to_string(kSessionPositions) + " positions");
    bound = std::max(bound, std::min(d->cfg.capacity, kSessionPositions));
  }
  return bound;
}

}  // namespace

extern "C" {

int fah_abi_version(void) { return FAH_ABI_VERSION; }

const char* fah_last_error(void) { return g_error.c_str(); }

int fah_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int fah_context_create(int device, fah_context** out) {
  if (!out) return fail(FAH_ERROR_ARGUMENT, "out is NULL");
  return guarded([&] {
    int n = fah_device_count();
    require(device >= 0 && device < n && device < kMaxDevices, "no HIP device " + std::to_string(device));
    check(hipSetDevice(device), "hipSetDevice");
    auto st = std::make_shared<Ctx>();
    st->device = device;
    init_scratch(device);
    hipStream_t stream = nullptr;
    check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
    st->stream = stream;
    check(hipEventCreateWithFlags(&st->mark, hipEventDisableTiming), "hipEventCreate");
    check(hipEventCreate(&st->t0), "hipEventCreate");
    check(hipEventCreate(&st->t1), "hipEventCreate");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) st->name = std::string("HIP ") + prop.gcnArchName;
    else st->name = "HIP";
    {
      DeviceGate& g = device_gate(device);
      std::lock_guard<std::mutex> lock(g.m);
      g.members.push_back(st.get());
    }
    auto* h = new fah_context();
    h->st = std::move(st);
    *out = h;
    return FAH_OK;
  });
}

// The handle goes; the state stays while weights or decoders made from it
// exist (their later calls report FAH_ERROR_DISPOSED, their release works).
int fah_context_destroy(fah_context* h) {
  if (!h) return FAH_OK;
  std::shared_ptr<Ctx> st = std::move(h->st);
  delete h;
  if (st) {
    std::lock_guard<std::mutex> lock(st->gate);
    (void)hipSetDevice(st->device);
    (void)hipStreamSynchronize(st->stream);
    st->batch.reset();
    st->disposed = true;
  }
  return FAH_OK;
}

int fah_context_synchronize(fah_context* h) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  return guarded([&] {
    std::lock_guard<std::mutex> lock(c->gate);
    check(hipSetDevice(c->device), "hipSetDevice");
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return FAH_OK;
  });
}

const char* fah_context_name(const fah_context* h) { return h ? h->st->name.c_str() : ""; }

int fah_context_set_minimum_operations(fah_context* h, int64_t operations) {
  if (!h || operations < 0) return fail(FAH_ERROR_ARGUMENT, "invalid minimum operations");
  h->st->minimum_operations = operations;
  return FAH_OK;
}

void* fah_context_stream(fah_context* h) { return h ? (void*)h->st->stream : nullptr; }

int fah_context_statistics(fah_context* h, fah_call_stats* out, int kinds) {
  if (!h || (kinds > 0 && !out) || kinds < 0) return fail(FAH_ERROR_ARGUMENT, "invalid statistics request");
  Ctx* c = h->st.get();
  std::lock_guard<std::mutex> lock(c->stats_m);
  for (int i = 0; i < std::min(kinds, (int)FAH_CALL_KINDS); ++i) out[i] = c->stats[i];
  return FAH_OK;
}

int fah_context_reset_statistics(fah_context* h) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  std::lock_guard<std::mutex> lock(c->stats_m);
  for (fah_call_stats& s : c->stats) s = fah_call_stats{};
  return FAH_OK;
}

int fah_context_set_call_observer(fah_context* h, fah_call_observer observer, void* user) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  std::lock_guard<std::mutex> lock(c->stats_m);
  c->observer = observer;
  c->observer_user = user;
  return FAH_OK;
}

int fah_weight_q8_upload(fah_context* h, const int8_t* quantized, const float* scales, int rows, int cols,
                         fah_weight** out) {
  if (!h || !out) return fail(FAH_ERROR_ARGUMENT, "context/out is NULL");
  Ctx* c = h->st.get();
  return guarded([&] {
    require(quantized && scales, "Q8 weight needs quantized bytes and scales");
    require(rows > 0 && cols > 0 && cols % 32 == 0, "Invalid row-major Q8 dimensions");
    std::lock_guard<std::mutex> lock(c->gate);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    auto w = std::make_unique<fah_weight>();
    w->ctx = h->st;
    w->rows = rows;
    w->cols = cols;
    size_t nb = (size_t)rows * (cols / 32);
    w->half_scales = scales_fit_half(scales, nb);
    upload(w->q, quantized, (size_t)rows * cols, c->stream);
    if (w->half_scales) {
      std::vector<uint16_t> hs(nb);
      for (size_t i = 0; i < nb; ++i) hs[i] = float_to_half_bits(scales[i]);
      upload(w->s, hs.data(), nb * 2, c->stream);
    } else {
      upload(w->s, scales, nb * 4, c->stream);
    }
    w->group_rows = pick_group_rows(rows, cols, 4, false);
    *out = w.release();
    return FAH_OK;
  });
}

int fah_weight_q8_upload_blocks(fah_context* h, const uint8_t* blocks, int rows, int cols, fah_weight** out) {
  if (!h || !out) return fail(FAH_ERROR_ARGUMENT, "context/out is NULL");
  Ctx* c = h->st.get();
  return guarded([&] {
    require(blocks != nullptr, "Q8 weight needs its GGUF blocks");
    require(rows > 0 && cols > 0 && cols % 32 == 0, "Invalid row-major Q8 dimensions");
    std::lock_guard<std::mutex> lock(c->gate);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    auto w = std::make_unique<fah_weight>();
    w->ctx = h->st;
    w->rows = rows;
    w->cols = cols;
    w->half_scales = true;
    upload_blocks(w->q, w->s, blocks, (size_t)rows * (cols / 32), c->stream);
    w->group_rows = pick_group_rows(rows, cols, 4, false);
    *out = w.release();
    return FAH_OK;
  });
}

// Drains the context's stream first (device-pointer calls may still read the
// weight), then frees it; valid before or after fah_context_destroy.
int fah_weight_release(fah_weight* w) {
  if (!w) return FAH_OK;
  std::shared_ptr<Ctx> st = w->ctx;
  {
    std::lock_guard<std::mutex> lock(st->gate);
    (void)hipSetDevice(st->device);
    (void)hipStreamSynchronize(st->stream);
    delete w;
  }
  return FAH_OK;
}

int64_t fah_weight_device_bytes(const fah_weight* w) {
  return w ? (int64_t)(w->q.bytes + w->s.bytes + w->f.bytes) : 0;
}

int fah_weight_f32_upload(fah_context* h, const float* values, int rows, int cols, fah_weight** out) {
  if (!h || !out) return fail(FAH_ERROR_ARGUMENT, "context/out is NULL");
  Ctx* c = h->st.get();
  return guarded([&] {
    require(values != nullptr, "FP32 weight needs its values");
    require(rows > 0 && cols > 0, "Invalid row-major FP32 dimensions");
    std::lock_guard<std::mutex> lock(c->gate);
    if (c->disposed) return fail(FAH_ERROR_DISPOSED, "context disposed");
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    auto w = std::make_unique<fah_weight>();
    w->ctx = h->st;
    w->rows = rows;
    w->cols = cols;
    w->f32 = true;
    upload(w->f, values, (size_t)rows * cols * 4, c->stream);
    *out = w.release();
    return FAH_OK;
  });
}

// Many rows at once go through the MFMA GEMM (same per-row block order).
constexpr int kGemmMinFrames = 4;
bool gemm_fits(const fah_weight* w, int frames) {
  return frames >= kGemmMinFrames && w->cols <= 3072 && w->cols % 128 == 0;
}

void launch_weight_gemm(const fah_weight* w, const int8_t* xq, const float* xs, int frames, float* out,
                        const float* bias, hipStream_t s) {
  fah::GemmArgs g{};
  g.w = w->q.as<int8_t>();
  g.ws = w->s.ptr;
  g.rows = w->rows;
  g.K = w->cols;
  g.xq = xq;
  g.xs = xs;
  g.frames = frames;
  g.out = out;
  g.out_stride = w->rows;
  g.bias = bias;
  check(fah::launch_gemm(g, w->half_scales, fah::kGemmPlain, s), "gemm");
}

static fah::GemvArgs weight_args(const fah_weight* w) {
  fah::GemvArgs a{};
  a.w = w->q.as<int8_t>();
  a.ws = w->s.ptr;
  a.rows = w->rows;
  a.K = w->cols;
  a.group_rows = w->group_rows;
  return a;
}

int fah_quantized_linear(fah_context* h, const float* input, int frames, const fah_weight* w, const float* bias,
                         float* output) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  if (!w || w->f32 || frames <= 0 || w->cols > fah::gemv_max_k()) return declined(c, FAH_CALL_QUANTIZED_LINEAR);
  if ((int64_t)frames * w->cols * w->rows < c->minimum_operations) return declined(c, FAH_CALL_QUANTIZED_LINEAR);
  return guarded([&] {
    require(input && output, "Q8 GPU projection needs input and output");
    require(w->ctx.get() == c, "weight belongs to another context");
    std::lock_guard<std::mutex> lock(c->gate);
    if (c->disposed) return fail(FAH_ERROR_DISPOSED, "context disposed");
    CallMeter meter(*c, FAH_CALL_QUANTIZED_LINEAR);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    size_t in_bytes = (size_t)frames * w->cols * 4, out_bytes = (size_t)frames * w->rows * 4;
    meter.up = (int64_t)in_bytes + (bias ? (int64_t)w->rows * 4 : 0);
    meter.down = (int64_t)out_bytes;
    c->in.ensure(in_bytes + (bias ? (size_t)w->rows * 4 : 0));
    c->out.ensure(out_bytes);
    check(hipMemcpyAsync(c->in.ptr, input, in_bytes, hipMemcpyHostToDevice, c->stream), "H2D input");
    float* dbias = nullptr;
    if (bias) {
      dbias = reinterpret_cast<float*>(c->in.as<char>() + in_bytes);
      check(hipMemcpyAsync(dbias, bias, (size_t)w->rows * 4, hipMemcpyHostToDevice, c->stream), "H2D bias");
    }
    if (gemm_fits(w, frames)) {
      size_t n = (size_t)frames * w->cols;
      c->q.ensure(n);
      c->s.ensure(n / 32 * 4);
      meter.kernels_begin();
      check(fah::launch_quantize(c->in.as<float>(), (int64_t)n, c->q.as<int8_t>(), c->s.as<float>(), c->stream),
            "quantize");
      launch_weight_gemm(w, c->q.as<int8_t>(), c->s.as<float>(), frames, c->out.as<float>(), dbias, c->stream);
    } else {
      fah::GemvArgs a = weight_args(w);
      a.x = c->in.as<float>();
      a.out = c->out.as<float>();
      a.out_rows = w->rows;
      a.bias = dbias;
      meter.kernels_begin();
      check(fah::launch_gemv(a, w->half_scales, fah::kInputFloat, fah::kOutPlain, frames, c->stream), "gemv");
    }
    meter.kernels_end();
    check(hipMemcpyAsync(output, c->out.ptr, out_bytes, hipMemcpyDeviceToHost, c->stream), "D2H output");
    work.release();  // enqueued: other contexts may enqueue while this stream drains
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    meter.done(frames, w->cols, w->rows, (int64_t)frames * w->cols * w->rows);
    return FAH_OK;
  });
}

int fah_quantized_linear_noalloc(fah_context* h, const float* input, int frames, const fah_weight* w,
                                 const float* bias, float* output) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  if (!w || w->f32 || frames <= 0 || w->cols > fah::gemv_max_k())
    return declined(c, FAH_CALL_QUANTIZED_LINEAR_NOALLOC);
  if ((int64_t)frames * w->cols * w->rows < c->minimum_operations) return declined(c, FAH_CALL_QUANTIZED_LINEAR_NOALLOC);
  return guarded([&] {
    require(input && output, "Q8 GPU projection needs input and output");
    require(w->ctx.get() == c, "weight belongs to another context");
    auto aligned = [](size_t n) { return (n + 255) & ~(size_t)255; };
    const size_t in_bytes = (size_t)frames * w->cols * 4, out_bytes = (size_t)frames * w->rows * 4;
    const size_t n = (size_t)frames * w->cols;
    const size_t at_bias = aligned(in_bytes), at_out = at_bias + aligned(bias ? (size_t)w->rows * 4 : 0);
    const size_t at_q = at_out + aligned(out_bytes), at_s = at_q + aligned(n), end = at_s + aligned(n / 32 * 4);
    require(end <= kScratchBytes, "projection needs " + std::to_string(end) +
                                      " bytes of workspace; the allocation-free path holds " +
                                      std::to_string(kScratchBytes));
    std::lock_guard<std::mutex> lock(c->gate);
    if (c->disposed) return fail(FAH_ERROR_DISPOSED, "context disposed");
    CallMeter meter(*c, FAH_CALL_QUANTIZED_LINEAR_NOALLOC);
    meter.up = (int64_t)in_bytes + (bias ? (int64_t)w->rows * 4 : 0);
    meter.down = (int64_t)out_bytes;
    check(hipSetDevice(c->device), "hipSetDevice");
    char* base = static_cast<char*>(scratch_ptr(c->device));
    require(base != nullptr, "no workspace for this device");
    // Held until the work has finished: no other call of this library can
    // use the device's workspace meanwhile.
    std::lock_guard<std::mutex> device(device_gate(c->device).m);
    // On every exit, error paths included, the stream drains before the
    // device lock is let go (destroyed first): nothing this call enqueued
    // still writes the workspace when another call may take it.
    struct Drain {
      hipStream_t s;
      ~Drain() { (void)hipStreamSynchronize(s); }
    } drain{c->stream};
    float* din = reinterpret_cast<float*>(base);
    float* dbias = bias ? reinterpret_cast<float*>(base + at_bias) : nullptr;
    float* dout = reinterpret_cast<float*>(base + at_out);
    check(hipMemcpyAsync(din, input, in_bytes, hipMemcpyHostToDevice, c->stream), "H2D input");
    if (bias) check(hipMemcpyAsync(dbias, bias, (size_t)w->rows * 4, hipMemcpyHostToDevice, c->stream), "H2D bias");
    meter.kernels_begin();
    if (gemm_fits(w, frames)) {
      int8_t* q = reinterpret_cast<int8_t*>(base + at_q);
      float* sc = reinterpret_cast<float*>(base + at_s);
      check(fah::launch_quantize(din, (int64_t)n, q, sc, c->stream), "quantize");
      launch_weight_gemm(w, q, sc, frames, dout, dbias, c->stream);
    } else {
      fah::GemvArgs a = weight_args(w);
      a.x = din;
      a.out = dout;
      a.out_rows = w->rows;
      a.bias = dbias;
      check(fah::launch_gemv(a, w->half_scales, fah::kInputFloat, fah::kOutPlain, frames, c->stream), "gemv");
    }
    meter.kernels_end();
    check(hipMemcpyAsync(output, dout, out_bytes, hipMemcpyDeviceToHost, c->stream), "D2H output");
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    meter.done(frames, w->cols, w->rows, (int64_t)frames * w->cols * w->rows);
    return FAH_OK;
  });
}

int fah_linear_many(fah_context* h, const float* input, int frames, const fah_weight* const* weights, int count,
                    float* const* outputs) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  if (count == 0) return FAH_OK;
  if (!weights || count < 0 || frames <= 0) return declined(c, FAH_CALL_LINEAR_MANY);
  int cols = weights[0] ? weights[0]->cols : 0;
  int64_t total_rows = 0;
  const bool f32 = weights[0] && weights[0]->f32;
  for (int i = 0; i < count; ++i) {
    if (!weights[i] || weights[i]->f32 != f32 || (!f32 && weights[i]->cols > fah::gemv_max_k()))
      return declined(c, FAH_CALL_LINEAR_MANY);
    total_rows += weights[i]->rows;
  }
  if ((int64_t)frames * cols * total_rows < c->minimum_operations) return declined(c, FAH_CALL_LINEAR_MANY);
  return guarded([&] {
    require(input && outputs, "grouped projection needs input and outputs");
    for (int i = 0; i < count; ++i) {
      require(weights[i]->cols == cols, "Grouped projection dimensions differ");
      require(weights[i]->ctx.get() == c, "weight belongs to another context");
      require(outputs[i] != nullptr, "grouped projection output is NULL");
    }
    std::lock_guard<std::mutex> lock(c->gate);
    if (c->disposed) return fail(FAH_ERROR_DISPOSED, "context disposed");
    CallMeter meter(*c, FAH_CALL_LINEAR_MANY);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    size_t n = (size_t)frames * cols;
    meter.up = (int64_t)n * 4;
    meter.down = (int64_t)frames * total_rows * 4;
    c->in.ensure(n * 4);
    c->q.ensure(n);
    c->s.ensure(n / 32 * 4);
    size_t out_total = 0;
    for (int i = 0; i < count; ++i) out_total += (size_t)frames * weights[i]->rows;
    c->out.ensure(out_total * 4);
    check(hipMemcpyAsync(c->in.ptr, input, n * 4, hipMemcpyHostToDevice, c->stream), "H2D input");
    meter.kernels_begin();
    if (f32) {
      // FP32 group (IGroupedComputeBackend over Weight.Values): each weight
      // through the same kernel as fah_linear, so the bits equal separate calls.
      size_t at = 0;
      for (int i = 0; i < count; ++i) {
        check(fah::launch_f32_linear(c->in.as<float>(), weights[i]->f.as<float>(), nullptr, c->out.as<float>() + at,
                                     frames, weights[i]->rows, cols, false, c->stream),
              "f32 linear");
        at += (size_t)frames * weights[i]->rows;
      }
    } else {
      check(fah::launch_quantize(c->in.as<float>(), (int64_t)n, c->q.as<int8_t>(), c->s.as<float>(), c->stream),
            "quantize");
      size_t at = 0;
      for (int i = 0; i < count; ++i) {
        if (gemm_fits(weights[i], frames)) {
          launch_weight_gemm(weights[i], c->q.as<int8_t>(), c->s.as<float>(), frames, c->out.as<float>() + at, nullptr,
                             c->stream);
        } else {
          fah::GemvArgs a = weight_args(weights[i]);
          a.xq = c->q.as<int8_t>();
          a.xs = c->s.as<float>();
          a.out = c->out.as<float>() + at;
          a.out_rows = weights[i]->rows;
          check(fah::launch_gemv(a, weights[i]->half_scales, fah::kInputQuantized, fah::kOutPlain, frames, c->stream),
                "gemv");
        }
        at += (size_t)frames * weights[i]->rows;
      }
    }
    meter.kernels_end();
    size_t at = 0;
    for (int i = 0; i < count; ++i) {
      size_t bytes = (size_t)frames * weights[i]->rows * 4;
      check(hipMemcpyAsync(outputs[i], c->out.as<float>() + at, bytes, hipMemcpyDeviceToHost, c->stream), "D2H");
      at += (size_t)frames * weights[i]->rows;
    }
    work.release();  // enqueued: other contexts may enqueue while this stream drains
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    meter.done(frames, cols, (int)total_rows, (int64_t)frames * cols * total_rows);
    return FAH_OK;
  });
}

int fah_linear(fah_context* h, const float* input, int frames, const fah_weight* w, const float* bias, float* output) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  if (!w || !w->f32 || frames <= 0) return declined(c, FAH_CALL_LINEAR);
  if ((int64_t)frames * w->cols * w->rows < c->minimum_operations) return declined(c, FAH_CALL_LINEAR);
  return guarded([&] {
    require(input && output, "FP32 GPU projection needs input and output");
    require(w->ctx.get() == c, "weight belongs to another context");
    std::lock_guard<std::mutex> lock(c->gate);
    if (c->disposed) return fail(FAH_ERROR_DISPOSED, "context disposed");
    CallMeter meter(*c, FAH_CALL_LINEAR);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    const size_t in_bytes = (size_t)frames * w->cols * 4, out_bytes = (size_t)frames * w->rows * 4;
    meter.up = (int64_t)in_bytes + (bias ? (int64_t)w->rows * 4 : 0);
    meter.down = (int64_t)out_bytes;
    c->in.ensure(in_bytes + (bias ? (size_t)w->rows * 4 : 0));
    c->out.ensure(out_bytes);
    check(hipMemcpyAsync(c->in.ptr, input, in_bytes, hipMemcpyHostToDevice, c->stream), "H2D input");
    float* dbias = nullptr;
    if (bias) {
      dbias = reinterpret_cast<float*>(c->in.as<char>() + in_bytes);
      check(hipMemcpyAsync(dbias, bias, (size_t)w->rows * 4, hipMemcpyHostToDevice, c->stream), "H2D bias");
    }
    meter.kernels_begin();
    check(fah::launch_f32_linear(c->in.as<float>(), w->f.as<float>(), dbias, c->out.as<float>(), frames, w->rows,
                                 w->cols, false, c->stream),
          "f32 linear");
    meter.kernels_end();
    check(hipMemcpyAsync(output, c->out.ptr, out_bytes, hipMemcpyDeviceToHost, c->stream), "D2H output");
    work.release();  // enqueued: other contexts may enqueue while this stream drains
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    meter.done(frames, w->cols, w->rows, (int64_t)frames * w->cols * w->rows);
    return FAH_OK;
  });
}

int fah_linear_device(fah_context* h, const float* x, int frames, const fah_weight* w, const float* bias, float* out) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  if (!w || !w->f32) return FAH_DECLINED;
  return guarded([&] {
    require(frames > 0 && x && out, "invalid FP32 projection arguments");
    require(w->ctx.get() == c, "weight belongs to another context");
    std::lock_guard<std::mutex> lock(c->gate);
    if (c->disposed) return fail(FAH_ERROR_DISPOSED, "context disposed");
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    check(fah::launch_f32_linear(x, w->f.as<float>(), bias, out, frames, w->rows, w->cols, false, c->stream),
          "f32 linear");
    return FAH_OK;
  });
}

int fah_relu_projection(fah_context* h, const float* input, int frames, const fah_weight* first,
                        const float* first_bias, const fah_weight* second, const float* second_bias, float* output) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  if (!first || !second || !first->f32 || !second->f32 || frames <= 0 || first->rows != second->cols ||
      first->rows % 4 != 0)
    return declined(c, FAH_CALL_RELU_PROJECTION);
  if ((int64_t)frames * first->rows * first->cols < c->minimum_operations ||
      (int64_t)frames * second->rows * second->cols < c->minimum_operations)
    return declined(c, FAH_CALL_RELU_PROJECTION);
  return guarded([&] {
    require(input && output, "ReLU projection needs input and output");
    require(first->ctx.get() == c && second->ctx.get() == c, "weight belongs to another context");
    std::lock_guard<std::mutex> lock(c->gate);
    if (c->disposed) return fail(FAH_ERROR_DISPOSED, "context disposed");
    CallMeter meter(*c, FAH_CALL_RELU_PROJECTION);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    const int H = first->rows, N = second->rows, K = first->cols;
    const size_t in_bytes = (size_t)frames * K * 4, mid_bytes = (size_t)frames * H * 4, out_bytes = (size_t)frames * N * 4;
    const size_t b1 = first_bias ? (size_t)H * 4 : 0, b2 = second_bias ? (size_t)N * 4 : 0;
    meter.up = (int64_t)(in_bytes + b1 + b2);
    meter.down = (int64_t)out_bytes;
    c->in.ensure(in_bytes + b1 + b2);
    c->out.ensure(mid_bytes + out_bytes);
    check(hipMemcpyAsync(c->in.ptr, input, in_bytes, hipMemcpyHostToDevice, c->stream), "H2D input");
    float* d1 = first_bias ? reinterpret_cast<float*>(c->in.as<char>() + in_bytes) : nullptr;
    float* d2 = second_bias ? reinterpret_cast<float*>(c->in.as<char>() + in_bytes + b1) : nullptr;
    if (d1) check(hipMemcpyAsync(d1, first_bias, b1, hipMemcpyHostToDevice, c->stream), "H2D bias");
    if (d2) check(hipMemcpyAsync(d2, second_bias, b2, hipMemcpyHostToDevice, c->stream), "H2D bias");
    float* mid = c->out.as<float>();
    float* dout = reinterpret_cast<float*>(c->out.as<char>() + mid_bytes);
    // The intermediate stays on the device (IReluProjectionBackend.cs:4-16).
    meter.kernels_begin();
    check(fah::launch_f32_linear(c->in.as<float>(), first->f.as<float>(), d1, mid, frames, H, K, true, c->stream),
          "f32 linear + ReLU");
    check(fah::launch_f32_linear(mid, second->f.as<float>(), d2, dout, frames, N, H, false, c->stream), "f32 linear");
    meter.kernels_end();
    check(hipMemcpyAsync(output, dout, out_bytes, hipMemcpyDeviceToHost, c->stream), "D2H output");
    work.release();  // enqueued: other contexts may enqueue while this stream drains
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    meter.done(frames, K, N, (int64_t)frames * H * (K + N));
    return FAH_OK;
  });
}

int fah_attention(fah_context* h, const float* query, const float* key, const float* value, int frames, int width,
                  int heads, float* output) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  if (!fah::f32_attention_supported(frames, width, heads)) return declined(c, FAH_CALL_ATTENTION);
  if (c->minimum_operations > 0 && (frames < 160 || (int64_t)frames * frames * width < c->minimum_operations))
    return declined(c, FAH_CALL_ATTENTION);
  return guarded([&] {
    require(query && key && value && output, "GPU attention needs query, key, value and output");
    std::lock_guard<std::mutex> lock(c->gate);
    if (c->disposed) return fail(FAH_ERROR_DISPOSED, "context disposed");
    CallMeter meter(*c, FAH_CALL_ATTENTION);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    const size_t bytes = (size_t)frames * width * 4;
    meter.up = 3 * (int64_t)bytes;
    meter.down = (int64_t)bytes;
    c->in.ensure(3 * bytes);
    c->out.ensure(bytes);
    float* dq = c->in.as<float>();
    float* dk = reinterpret_cast<float*>(c->in.as<char>() + bytes);
    float* dv = reinterpret_cast<float*>(c->in.as<char>() + 2 * bytes);
    check(hipMemcpyAsync(dq, query, bytes, hipMemcpyHostToDevice, c->stream), "H2D query");
    check(hipMemcpyAsync(dk, key, bytes, hipMemcpyHostToDevice, c->stream), "H2D key");
    check(hipMemcpyAsync(dv, value, bytes, hipMemcpyHostToDevice, c->stream), "H2D value");
    meter.kernels_begin();
    check(fah::launch_f32_attention(dq, dk, dv, c->out.as<float>(), frames, width, heads, c->stream), "attention");
    meter.kernels_end();
    check(hipMemcpyAsync(output, c->out.ptr, bytes, hipMemcpyDeviceToHost, c->stream), "D2H output");
    work.release();  // enqueued: other contexts may enqueue while this stream drains
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    meter.done(frames, width, width, 2 * (int64_t)frames * frames * width);
    return FAH_OK;
  });
}

int fah_attention_device(fah_context* h, const float* query, const float* key, const float* value, int frames,
                         int width, int heads, float* output) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  if (!fah::f32_attention_supported(frames, width, heads)) return FAH_DECLINED;
  return guarded([&] {
    require(query && key && value && output, "GPU attention needs query, key, value and output");
    std::lock_guard<std::mutex> lock(c->gate);
    if (c->disposed) return fail(FAH_ERROR_DISPOSED, "context disposed");
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    check(fah::launch_f32_attention(query, key, value, output, frames, width, heads, c->stream), "attention");
    return FAH_OK;
  });
}

int fah_quantize_device(fah_context* h, const float* x, int64_t n, int8_t* q, float* scales) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  return guarded([&] {
    require(n >= 0 && n % 32 == 0, "Quantization needs matching complete blocks");
    require(n == 0 || (x && q && scales), "NULL buffer");
    std::lock_guard<std::mutex> lock(c->gate);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    check(fah::launch_quantize(x, n, q, scales, c->stream), "quantize");
    return FAH_OK;
  });
}

int fah_rms_norm_device(fah_context* h, const float* x, int rows, int width, const float* scale, float eps,
                        float* y) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  return guarded([&] {
    require(rows >= 0 && (width == 128 || (width > 0 && width % 4 == 0 && width <= 4096)),
            "Invalid normalization dimensions");
    require(rows == 0 || (x && scale && y), "NULL buffer");
    std::lock_guard<std::mutex> lock(c->gate);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    check(fah::launch_rms_norm_rows(x, rows, width, scale, eps, y, c->stream), "rms norm");
    return FAH_OK;
  });
}

int fah_q8_gemv_device(fah_context* h, const int8_t* q, const float* scales, int frames, const fah_weight* w,
                       float* out) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  if (!w || w->f32 || w->cols > fah::gemv_max_k()) return FAH_DECLINED;
  return guarded([&] {
    require(frames > 0 && q && scales && out, "invalid GEMV arguments");
    require(w->ctx.get() == c, "weight belongs to another context");
    std::lock_guard<std::mutex> lock(c->gate);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    if (gemm_fits(w, frames)) {
      launch_weight_gemm(w, q, scales, frames, out, nullptr, c->stream);
    } else {
      fah::GemvArgs a = weight_args(w);
      a.xq = q;
      a.xs = scales;
      a.out = out;
      a.out_rows = w->rows;
      check(fah::launch_gemv(a, w->half_scales, fah::kInputQuantized, fah::kOutPlain, frames, c->stream), "gemv");
    }
    return FAH_OK;
  });
}

int fah_q8_block_dots_device(fah_context* h, const int8_t* q, const fah_weight* w, int32_t* dots) {
  if (!h) return fail(FAH_ERROR_ARGUMENT, "context is NULL");
  Ctx* c = h->st.get();
  return guarded([&] {
    require(w && q && dots, "invalid block-dot arguments");
    require(!w->f32, "block dots need a Q8_0 weight");
    require(w->ctx.get() == c, "weight belongs to another context");
    std::lock_guard<std::mutex> lock(c->gate);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    check(fah::launch_block_dots(q, w->q.as<int8_t>(), w->rows, w->cols, dots, c->stream), "block dots");
    return FAH_OK;
  });
}

int fah_decoder_create(fah_context* h, const fah_decoder_config* cfg, const fah_layer_host* layers,
                       const fah_q8_host* token_embd, const fah_q8_host* output, const float* output_norm,
                       fah_decoder** out) {
  if (!h || !out) return fail(FAH_ERROR_ARGUMENT, "context/out is NULL");
  Ctx* c = h->st.get();
  return guarded([&] {
    require(cfg && layers && token_embd && output_norm, "decoder needs config, layers, embeddings and norm");
    const fah_decoder_config& k = *cfg;
    require(k.layers > 0 && k.width > 0 && k.heads > 0 && k.kv_heads > 0 && k.vocab > 0 && k.ffn > 0,
            "invalid decoder dimensions");
    require(k.heads % k.kv_heads == 0, "Invalid GQA head counts");
    require(k.head_size == 128, "head_size must be 128");
    require(k.heads == 2 * k.kv_heads || k.heads == 4 * k.kv_heads, "GQA groups of 2 or 4 query heads per KV head");
    require(k.width % 32 == 0 && k.ffn % 32 == 0, "widths must be multiples of 32");
    int q_width = k.heads * k.head_size, kv_width = k.kv_heads * k.head_size;
    // The ffn width (the down projection's K) up to the GEMV's limit; the
    // model width and q width up to 4096 (the norm, embedding and attention
    // kernels hold rows of that width).
    require(k.width <= 4096 && q_width <= 4096 && k.ffn <= fah::gemv_max_k(), "projection width exceeds kernel limit");
    require(k.capacity >= 1 && fah::attention_slices(k.capacity, k.head_size, k.heads / k.kv_heads) != 0,
            "capacity exceeds the attention kernel's LDS budget");
    for (int l = 0; l < k.layers; ++l) {
      const fah_layer_host& L = layers[l];
      std::string p = "blk." + std::to_string(l) + ".";
      validate_q8(&L.wq, q_width, k.width, (p + "attn_q").c_str());
      validate_q8(&L.wk, kv_width, k.width, (p + "attn_k").c_str());
      validate_q8(&L.wv, kv_width, k.width, (p + "attn_v").c_str());
      validate_q8(&L.wo, k.width, q_width, (p + "attn_output").c_str());
      validate_q8(&L.gate, k.ffn, k.width, (p + "ffn_gate").c_str());
      validate_q8(&L.up, k.ffn, k.width, (p + "ffn_up").c_str());
      validate_q8(&L.down, k.width, k.ffn, (p + "ffn_down").c_str());
      require(L.attn_norm && L.q_norm && L.k_norm && L.ffn_norm, p + ": missing norm weights");
    }
    validate_q8(token_embd, k.vocab, k.width, "token_embd");
    if (output) validate_q8(output, k.vocab, k.width, "output");

    std::lock_guard<std::mutex> lock(c->gate);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    check(fah::prepare_attention(k.capacity, k.head_size, k.heads / k.kv_heads), "attention LDS budget");
    auto d = std::make_unique<fah_decoder>();
    d->ctx = h->st;
    d->cfg = k;
    d->q_width = q_width;
    d->kv_width = kv_width;
    d->wt = std::make_shared<DecoderWeights>();
    hipStream_t s = c->stream;

    bool half = true;
    auto fits = [&](const fah_q8_host& w) {
      return !w.scales || scales_fit_half(w.scales, (size_t)w.rows * (w.cols / 32));  // GGUF blocks: fp16
    };
    for (int l = 0; l < k.layers && half; ++l) {
      const fah_layer_host& L = layers[l];
      half = fits(L.wq) && fits(L.wk) && fits(L.wv) && fits(L.wo) && fits(L.gate) && fits(L.up) && fits(L.down);
    }
    half = half && fits(*token_embd) && (!output || fits(*output));
    d->wt->half_scales = half;

    d->wt->qkv.resize(k.layers);
    d->wt->wo.resize(k.layers);
    d->wt->gateup.resize(k.layers);
    d->wt->down.resize(k.layers);
    d->wt->attn_norm.resize(k.layers);
    d->wt->q_norm.resize(k.layers);
    d->wt->k_norm.resize(k.layers);
    d->wt->ffn_norm.resize(k.layers);
    int qkv_rows = q_width + 2 * kv_width;
    int qkv_group = pick_group_rows(qkv_rows, k.width, 4, false);
    int o_group = pick_group_rows(k.width, q_width, 4, false);
    // Persistent path: one workgroup per CU, 256 workgroups.
    int cus = 0;
    {
      hipDeviceProp_t prop;
      if (hipGetDeviceProperties(&prop, c->device) == hipSuccess) cus = prop.multiProcessorCount;
    }
    const char* env = std::getenv("FAH_PERSISTENT");
    const int nb = 256;
    d->persistent = !(env && env[0] == '0') && half && cus >= nb &&
                    fah::persistent_shape_supported(k.width, k.heads, k.kv_heads, k.head_size, k.ffn, nb) &&
                    fah::persistent_blocks_per_cu(k.width) >= 1;
    d->wt->persistent_layout = d->persistent;
    // Gate/up storage tiles: R gate rows then the matching R up rows. The
    // persistent kernel gives each projection workgroup (all but the
    // attention ones) an even share of the ffn rows, as one tile each.
    int gu_group = pick_group_rows(2 * k.ffn, k.width, 4, true);
    while (gu_group > 2 && (k.ffn % (gu_group / 2) != 0)) gu_group /= 2;
    const int ng = nb - k.heads;
    d->wt->gu_base = d->persistent ? k.ffn / ng : gu_group / 2;
    d->wt->gu_extra = d->persistent ? k.ffn % ng : 0;
    int down_group = pick_group_rows(k.width, k.ffn, 4, false);
    for (int l = 0; l < k.layers; ++l) {
      const fah_layer_host& L = layers[l];
      std::vector<std::pair<int, int>> order;
      for (int r = 0; r < q_width; ++r) order.emplace_back(0, r);
      for (int r = 0; r < kv_width; ++r) order.emplace_back(1, r);
      for (int r = 0; r < kv_width; ++r) order.emplace_back(2, r);
      upload_matrix(d->wt->qkv[l], {&L.wq, &L.wk, &L.wv}, order, k.width, half, s);
      d->wt->qkv[l].group_rows = qkv_group;
      order.clear();
      for (int r = 0; r < k.width; ++r) order.emplace_back(0, r);
      upload_matrix(d->wt->wo[l], {&L.wo}, order, q_width, half, s);
      d->wt->wo[l].group_rows = o_group;
      order.clear();
      if (d->persistent) {
        const int group = k.heads / k.kv_heads;
        for (int x = 0; x < 8; ++x)
          for (int j = 0; j < fah::persistent_xcd_roles(x, k.kv_heads, group, nb); ++j) {
            const fah::XcdEntries f = fah::persistent_xcd_entries(x, j, k.ffn, k.kv_heads, group, nb);
            for (int kind = 0; kind < 2; ++kind)
              for (int e = f.r0; e < f.r0 + f.count; ++e) order.emplace_back(kind, fah::persistent_xcd_row(x, e, 64));
          }
        if (l == 0) {
          std::vector<int> map(2 * (size_t)k.ffn, -1);
          for (size_t i = 0; i < order.size(); ++i) map[2 * (size_t)order[i].second + order[i].first] = (int)i;
          for (int v : map) require(v >= 0, "gate/up layout covers every row");
          upload(d->wt->gu_map, map.data(), map.size() * 4, s);
        }
      } else {
        int R = gu_group / 2;
        for (int t = 0; t < k.ffn / R; ++t) {
          for (int r = 0; r < R; ++r) order.emplace_back(0, t * R + r);
          for (int r = 0; r < R; ++r) order.emplace_back(1, t * R + r);
        }
      }
      upload_matrix(d->wt->gateup[l], {&L.gate, &L.up}, order, k.width, half, s);
      d->wt->gateup[l].group_rows = gu_group;
      order.clear();
      for (int r = 0; r < k.width; ++r) order.emplace_back(0, r);
      upload_matrix(d->wt->down[l], {&L.down}, order, k.ffn, half, s);
      d->wt->down[l].group_rows = down_group;
      upload(d->wt->attn_norm[l], L.attn_norm, (size_t)k.width * 4, s);
      upload(d->wt->q_norm[l], L.q_norm, (size_t)k.head_size * 4, s);
      upload(d->wt->k_norm[l], L.k_norm, (size_t)k.head_size * 4, s);
      upload(d->wt->ffn_norm[l], L.ffn_norm, (size_t)k.width * 4, s);
      d->wt->weight_bytes += matrix_bytes(d->wt->qkv[l]) + matrix_bytes(d->wt->wo[l]) + matrix_bytes(d->wt->gateup[l]) +
                         matrix_bytes(d->wt->down[l]);
    }
    {
      std::vector<std::pair<int, int>> order;
      for (int r = 0; r < k.vocab; ++r) order.emplace_back(0, r);
      upload_matrix(d->wt->embed, {token_embd}, order, k.width, half, s);
      d->wt->embed.group_rows = pick_group_rows(k.vocab, k.width, 4, false);
      d->wt->tied = output == nullptr;
      if (!d->wt->tied) {
        upload_matrix(d->wt->lm_head, {output}, order, k.width, half, s);
        d->wt->lm_head.group_rows = d->wt->embed.group_rows;
      }
    }
    DeviceMatrix& head = d->wt->tied ? d->wt->embed : d->wt->lm_head;
    d->wt->weight_bytes += matrix_bytes(head);
    upload(d->wt->output_norm, output_norm, (size_t)k.width * 4, s);

    if (d->persistent) {
      std::vector<fah::PersistentLayer> table(k.layers);
      for (int l = 0; l < k.layers; ++l) {
        fah::PersistentLayer& t = table[l];
        t.wqkv = d->wt->qkv[l].q.as<int8_t>();
        t.sqkv = d->wt->qkv[l].s.as<_Float16>();
        t.wo = d->wt->wo[l].q.as<int8_t>();
        t.so = d->wt->wo[l].s.as<_Float16>();
        t.wgu = d->wt->gateup[l].q.as<int8_t>();
        t.sgu = d->wt->gateup[l].s.as<_Float16>();
        t.wd = d->wt->down[l].q.as<int8_t>();
        t.sd = d->wt->down[l].s.as<_Float16>();
        t.attn_norm = d->wt->attn_norm[l].as<float>();
        t.q_norm = d->wt->q_norm[l].as<float>();
        t.k_norm = d->wt->k_norm[l].as<float>();
        t.ffn_norm = d->wt->ffn_norm[l].as<float>();
      }
      upload(d->wt->layer_table, table.data(), table.size() * sizeof(fah::PersistentLayer), s);
    }
    init_state(d.get(), s);
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    *out = d.release();
    return FAH_OK;
  });
}

int fah_decoder_destroy(fah_decoder* d) {
  if (!d) return FAH_OK;
  std::shared_ptr<Ctx> st = d->ctx;
  std::lock_guard<std::mutex> lock(st->gate);
  (void)hipSetDevice(st->device);
  (void)hipStreamSynchronize(st->stream);
  auto& batch = st->batch;
  if (batch && std::find(batch->members.begin(), batch->members.end(), d) != batch->members.end()) batch.reset();
  for (hipGraphExec_t g : {d->graph_row, d->graph_logits, d->graph_step})
    if (g) (void)hipGraphExecDestroy(g);
  delete d;
  return FAH_OK;
}

}  // extern "C"

namespace {

// Decoder calls after fah_context_destroy report FAH_ERROR_DISPOSED (the
// reference's ObjectDisposedException, VulkanQuantizedBackend.cs:54-56).
struct DisposedError {};
void require_live(const fah_decoder* d) {
  if (d->ctx->disposed) throw DisposedError{};
}

template <typename F>
int guarded_decoder(F&& f) {
  return guarded([&] {
    try {
      return f();
    } catch (const DisposedError&) {
      return fail(FAH_ERROR_DISPOSED, "decoder used after its context was destroyed");
    }
  });
}

// Device section of a decoder call: exclusive use of the device around
// persistent launches, the plain enqueue lock otherwise.
struct DecoderSection {
  std::optional<PersistentSection> persistent;
  std::optional<DeviceWork> work;
  DecoderSection(fah_decoder* d, bool exclusive) {
    if (exclusive && d->persistent) persistent.emplace(*d->ctx);
    else work.emplace(*d->ctx);
  }
};

}  // namespace

extern "C" {

int fah_decoder_set_position(fah_decoder* d, int position) {
  if (!d) return fail(FAH_ERROR_ARGUMENT, "decoder is NULL");
  return guarded_decoder([&] {
    require(position >= 0 && position <= d->cfg.capacity, "position out of range");
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    DeviceWork work(*d->ctx);
    check(hipMemcpyAsync(d->position.ptr, &position, 4, hipMemcpyHostToDevice, d->ctx->stream), "H2D");
    check(hipStreamSynchronize(d->ctx->stream), "sync");
    d->host_position = position;
    d->have_logits = false;
    return FAH_OK;
  });
}

int fah_decoder_position(const fah_decoder* d, int* position) {
  if (!d || !position) return fail(FAH_ERROR_ARGUMENT, "decoder/position is NULL");
  *position = d->host_position;
  return FAH_OK;
}

int fah_decoder_decode(fah_decoder* d, const float* embeddings, int frames, float* logits) {
  if (!d) return fail(FAH_ERROR_ARGUMENT, "decoder is NULL");
  return guarded_decoder([&] {
    require(embeddings && frames >= 1 && d->host_position + frames <= d->cfg.capacity,
            "Decoder context exhausted or invalid embeddings");
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    hipStream_t s = d->ctx->stream;
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    const bool batched = use_prefill(d, frames);
    {
      DecoderSection section(d, !batched);
      size_t row = (size_t)d->cfg.width * 4;
      d->staging.ensure(row * frames);
      check(hipMemcpyAsync(d->staging.ptr, embeddings, row * frames, hipMemcpyHostToDevice, s), "H2D embeddings");
      if (batched) {
        prefill(d, d->staging.as<float>(), frames, logits != nullptr, s);
      } else {
        for (int f = 0; f < frames; ++f) {
          check(hipMemcpyAsync(d->x.ptr, d->staging.as<char>() + row * f, row, hipMemcpyDeviceToDevice, s), "D2D row");
          bool last = f == frames - 1;
          run_kind(d, last && logits ? 1 : 0, s, d->host_position + f);
        }
      }
      if (logits)
        check(hipMemcpyAsync(logits, d->logits.ptr, (size_t)d->cfg.vocab * 4, hipMemcpyDeviceToHost, s), "D2H");
      check(hipStreamSynchronize(s), "hipStreamSynchronize");
    }
    recover_step_error(d);
    d->host_position += frames;
    d->have_logits = logits != nullptr;
    return FAH_OK;
  });
}

int fah_decoder_embed(fah_decoder* d, const int32_t* tokens, int count, float* out) {
  if (!d) return fail(FAH_ERROR_ARGUMENT, "decoder is NULL");
  return guarded_decoder([&] {
    require(count >= 0 && (count == 0 || (tokens && out)), "invalid embed arguments");
    for (int i = 0; i < count; ++i) require(tokens[i] >= 0 && tokens[i] < d->cfg.vocab, "token out of range");
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    hipStream_t s = d->ctx->stream;
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    DeviceWork work(*d->ctx);
    d->staging.ensure((size_t)d->cfg.width * 4 + 16);
    int* tok = reinterpret_cast<int*>(d->staging.as<char>() + (size_t)d->cfg.width * 4);
    for (int i = 0; i < count; ++i) {
      check(hipMemcpyAsync(tok, &tokens[i], 4, hipMemcpyHostToDevice, s), "H2D token");
      check(fah::launch_embed(d->wt->embed.q.as<int8_t>(), d->wt->embed.s.ptr, d->wt->half_scales, d->cfg.width, d->cfg.vocab,
                              tok, d->staging.as<float>(), nullptr, nullptr, s),
            "embed");
      check(hipMemcpyAsync(out + (size_t)i * d->cfg.width, d->staging.ptr, (size_t)d->cfg.width * 4,
                           hipMemcpyDeviceToHost, s),
            "D2H");
      check(hipStreamSynchronize(s), "sync");
    }
    return FAH_OK;
  });
}

int fah_decoder_greedy(fah_decoder* d, int32_t* token) {
  if (!d || !token) return fail(FAH_ERROR_ARGUMENT, "decoder/token is NULL");
  return guarded_decoder([&] {
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    if (!d->have_logits) return fail(FAH_ERROR_STATE, "no logits: decode with logits first");
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    DeviceWork work(*d->ctx);
    check(hipMemcpyAsync(token, d->token.ptr, 4, hipMemcpyDeviceToHost, d->ctx->stream), "D2H token");
    check(hipStreamSynchronize(d->ctx->stream), "sync");
    return FAH_OK;
  });
}

int fah_decoder_generate(fah_decoder* d, int steps, int32_t* tokens) {
  if (!d) return fail(FAH_ERROR_ARGUMENT, "decoder is NULL");
  return guarded_decoder([&] {
    require(steps >= 0 && (steps == 0 || tokens), "invalid generate arguments");
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    if (!d->have_logits) return fail(FAH_ERROR_STATE, "no logits: decode with logits first");
    require(d->host_position + steps <= d->cfg.capacity, "Decoder context exhausted");
    hipStream_t s = d->ctx->stream;
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    {
      DecoderSection section(d, true);
      check(hipMemsetAsync(d->history_count.ptr, 0, 4, s), "reset history");
      for (int i = 0; i < steps; ++i) run_kind(d, 2, s, d->host_position + i);
      if (steps > 0)
        check(hipMemcpyAsync(tokens, d->history.ptr, (size_t)steps * 4, hipMemcpyDeviceToHost, s), "D2H tokens");
      check(hipStreamSynchronize(s), "hipStreamSynchronize");
    }
    recover_step_error(d);
    d->host_position += steps;
    return FAH_OK;
  });
}

int fah_decoder_fail_next_step(fah_decoder* d) {
  if (!d) return fail(FAH_ERROR_ARGUMENT, "decoder is NULL");
  return guarded_decoder([&] {
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    if (!d->persistent) return FAH_DECLINED;
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    DeviceWork work(*d->ctx);
    const unsigned preset = kErrorPreset;
    check(hipMemcpyAsync(d->error.ptr, &preset, 4, hipMemcpyHostToDevice, d->ctx->stream), "H2D error word");
    check(hipStreamSynchronize(d->ctx->stream), "sync");
    d->fail_sessions = true;
    return FAH_OK;
  });
}

int fah_decoder_create_session(fah_decoder* parent, int capacity, fah_decoder** out) {
  if (!parent || !out) return fail(FAH_ERROR_ARGUMENT, "parent/session is NULL");
  return guarded_decoder([&] {
    require(capacity >= 1, "capacity must be positive");
    Ctx* c = parent->ctx.get();
    auto d = std::make_unique<fah_decoder>();
    d->ctx = parent->ctx;
    d->cfg = parent->cfg;
    d->cfg.capacity = capacity;
    d->q_width = parent->q_width;
    d->kv_width = parent->kv_width;
    d->wt = parent->wt;
    if (d->wt->persistent_layout) d->persistent = true;
    require(fah::attention_slices(capacity, d->cfg.head_size, d->cfg.heads / d->cfg.kv_heads) != 0,
            "capacity exceeds the attention kernel's LDS budget");
    std::lock_guard<std::mutex> lock(c->gate);
    require_live(parent);
    check(hipSetDevice(c->device), "hipSetDevice");
    DeviceWork work(*c);
    check(fah::prepare_attention(capacity, d->cfg.head_size, d->cfg.heads / d->cfg.kv_heads), "attention LDS budget");
    init_state(d.get(), c->stream);
    work.release();  // enqueued: other contexts may enqueue while this stream drains
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    *out = d.release();
    return FAH_OK;
  });
}

int fah_decoder_generate_sessions(fah_decoder* const* sessions, int count, int steps, int32_t* tokens) {
  if (!sessions || count < 1) return fail(FAH_ERROR_ARGUMENT, "no sessions");
  return guarded_decoder([&] {
    require(steps >= 0 && (steps == 0 || tokens), "invalid generate arguments");
    // The captured step is sized for kSessionPositions (or the largest
    // capacity, if smaller) so it serves every later call on these sessions.
    const int bound = check_sessions(sessions, count, steps);
    if (steps == 0) return FAH_OK;
    const fah_decoder* d0 = sessions[0];
    Ctx* c = d0->ctx.get();
    std::lock_guard<std::mutex> lock(c->gate);
    require_live(d0);
    hipStream_t s = c->stream;
    check(hipSetDevice(c->device), "hipSetDevice");
    // The one-launch step needs every CU: the device to itself until its
    // stream drains (PersistentSection), the plain enqueue lock otherwise.
    const bool fused = session_step_fits(d0, count, bound);
    std::optional<PersistentSection> exclusive;
    std::optional<DeviceWork> work;
    if (fused) exclusive.emplace(*c);
    else work.emplace(*c);
    std::vector<fah_decoder*> members(sessions, sessions + count);
    if (!c->batch || c->batch->members != members || c->batch->max_positions != bound) {
      c->batch.reset();
      auto b = make_session_batch(d0, count, bound, s, fused);
      upload_session_table(*b, sessions, count, s);
      b->members = members;
      c->batch = std::move(b);
    }
    SessionBatch& b = *c->batch;
    for (int i = 0; i < count; ++i)
      check(hipMemsetAsync(sessions[i]->history_count.ptr, 0, 4, s), "reset history");
    preset_session_failure(b, sessions, count, s);
    for (int i = 0; i < steps; ++i) {
      if (b.graph) check(hipGraphLaunch(b.graph, s), "hipGraphLaunch");
      else enqueue_sessions_step(d0, b, s);
    }
    for (int i = 0; i < count; ++i)
      check(hipMemcpyAsync(tokens + (size_t)i * steps, sessions[i]->history.ptr, (size_t)steps * 4,
                           hipMemcpyDeviceToHost, s),
            "D2H tokens");
    if (work) work->release();  // enqueued: other contexts may enqueue while this stream drains
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    recover_session_step(b, sessions, count, s);
    for (int i = 0; i < count; ++i) sessions[i]->host_position += steps;
    return FAH_OK;
  });
}

int fah_batcher_create(fah_decoder* parent, int max_positions, int window_us, fah_batcher** out) {
  if (!parent || !out) return fail(FAH_ERROR_ARGUMENT, "parent/out is NULL");
  return guarded_decoder([&] {
    require(max_positions >= 1 && max_positions <= kSessionPositions,
            "batched sessions are limited to " + std::to_string(kSessionPositions) + " positions");
    require(window_us >= 0 && window_us <= 1000000, "collection window out of range (0..1 s)");
    const fah_decoder_config& k = parent->cfg;
    require(k.width % 128 == 0 && k.ffn % 128 == 0 && parent->q_width % 128 == 0 && k.ffn <= 3072,
            "lock-step sessions need projection widths that are multiples of 128, at most 3072");
    std::lock_guard<std::mutex> lock(parent->ctx->gate);
    require_live(parent);
    auto b = std::make_unique<fah_batcher>();
    b->ctx = parent->ctx;
    b->wt = parent->wt;
    b->max_positions = max_positions;
    b->window = std::chrono::microseconds(window_us);
    *out = b.release();
    return FAH_OK;
  });
}

int fah_batcher_destroy(fah_batcher* b) {
  if (!b) return FAH_OK;
  {
    std::lock_guard<std::mutex> lk(b->m);
    if (b->running || !b->pending.empty()) return fail(FAH_ERROR_STATE, "step batcher busy: a step is in progress");
  }
  std::shared_ptr<Ctx> st = b->ctx;
  {
    std::lock_guard<std::mutex> lock(st->gate);
    (void)hipSetDevice(st->device);
    (void)hipStreamSynchronize(st->stream);
    delete b;
  }
  return FAH_OK;
}

int fah_batcher_join(fah_batcher* b, fah_decoder* session) {
  if (!b || !session) return fail(FAH_ERROR_ARGUMENT, "batcher/session is NULL");
  return guarded_decoder([&] {
    require(session->wt == b->wt && session->ctx == b->ctx, "session does not share the batcher's weights");
    std::lock_guard<std::mutex> lk(b->m);
    if (std::find(b->joined.begin(), b->joined.end(), session) == b->joined.end()) b->joined.push_back(session);
    b->cv.notify_all();
    return FAH_OK;
  });
}

int fah_batcher_leave(fah_batcher* b, fah_decoder* session) {
  if (!b || !session) return fail(FAH_ERROR_ARGUMENT, "batcher/session is NULL");
  std::lock_guard<std::mutex> lk(b->m);
  b->joined.erase(std::remove(b->joined.begin(), b->joined.end(), session), b->joined.end());
  b->idle.erase(std::remove(b->idle.begin(), b->idle.end(), session), b->idle.end());
  b->cv.notify_all();
  return FAH_OK;
}

}  // extern "C"

namespace {

// Checks of one session's own step through a batcher; a failure goes to
// that session's request alone (the reference throws for that decoder only,
// QwenDecoder.cs:163).
void check_batch_session(const fah_batcher* b, const fah_decoder* d) {
  require_live(d);
  if (!d->have_logits) throw StateError{"session has no logits: decode with logits first"};
  require(d->host_position + 1 <= d->cfg.capacity, "Decoder context exhausted");
  require(d->host_position + 1 <= b->max_positions,
          "session at position " + std::to_string(d->host_position) + " is past the batcher's bound of " +
              std::to_string(b->max_positions) + " positions");
}

// One lock-step batch of the requests' sessions (one greedy step each, as
// fah_decoder_generate(session, 1)): the batch size's captured step with
// this batch's session table. A request whose session fails its own checks
// gets that error and is left out; the others run. A device error of the
// batch itself goes to every request that was in it.
void run_batch(fah_batcher* b, const std::vector<BatchRequest*>& reqs) {
  std::vector<BatchRequest*> ok;
  for (BatchRequest* r : reqs) {
    r->status = guarded_decoder([&] {
      check_batch_session(b, r->session);
      return FAH_OK;
    });
    if (r->status != FAH_OK) r->error = fah_last_error();
    else ok.push_back(r);
  }
  if (ok.empty()) return;
  // A stable order (by session) keeps the table of a recurring batch the
  // same, so it is uploaded only when the members change.
  std::sort(ok.begin(), ok.end(), [](const BatchRequest* x, const BatchRequest* y) {
    return std::less<const fah_decoder*>()(x->session, y->session);
  });
  std::vector<fah_decoder*> sessions;
  for (BatchRequest* r : ok) sessions.push_back(r->session);
  const int count = (int)sessions.size();
  std::vector<int32_t> tokens(count, 0);
  const int status = guarded_decoder([&] {
    (void)check_sessions(sessions.data(), count, 1);
    Ctx* c = b->ctx.get();
    std::lock_guard<std::mutex> lock(c->gate);
    require_live(sessions[0]);
    hipStream_t s = c->stream;
    check(hipSetDevice(c->device), "hipSetDevice");
    const bool fused = session_step_fits(sessions[0], count, b->max_positions);
    auto& batch = b->by_size[count];
    {
      // The one-launch step needs the device to itself until its stream
      // drains; the plain enqueue lock otherwise.
      std::optional<PersistentSection> exclusive;
      std::optional<DeviceWork> work;
      if (fused) exclusive.emplace(*c);
      else work.emplace(*c);
      if (!batch) batch = make_session_batch(sessions[0], count, b->max_positions, s, fused);
      upload_session_table(*batch, sessions.data(), count, s);
      preset_session_failure(*batch, sessions.data(), count, s);
      const fah::SessionRef* table = batch->table.as<fah::SessionRef>();
      batch->tokens.ensure((size_t)fah::kFewFrames * 4);
      check(fah::launch_session_batch_io(table, count, nullptr, s), "reset histories");
      if (batch->graph) check(hipGraphLaunch(batch->graph, s), "hipGraphLaunch");
      else enqueue_sessions_step(sessions[0], *batch, s);
      check(fah::launch_session_batch_io(table, count, batch->tokens.as<int>(), s), "gather tokens");
      if (!batch->readback)
        check(hipHostMalloc(reinterpret_cast<void**>(&batch->readback), (fah::kFewFrames + 2) * 4, hipHostMallocDefault),
              "hipHostMalloc read-back");
      int32_t* rb = batch->readback;
      check(hipMemcpyAsync(rb, batch->tokens.ptr, (size_t)count * 4, hipMemcpyDeviceToHost, s), "D2H tokens");
      if (fused) {
        check(hipMemcpyAsync(rb + fah::kFewFrames, batch->error.ptr, 4, hipMemcpyDeviceToHost, s), "D2H error word");
        check(hipMemcpyAsync(rb + fah::kFewFrames + 1, batch->epoch.ptr, 4, hipMemcpyDeviceToHost, s), "D2H epoch");
      }
      check(hipStreamSynchronize(s), "hipStreamSynchronize");
      std::copy(rb, rb + count, tokens.begin());
      if (fused)
        recover_session_step_read(*batch, sessions.data(), count, (unsigned)rb[fah::kFewFrames],
                                  (unsigned)rb[fah::kFewFrames + 1], s);
    }
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    for (fah_decoder* d : sessions) d->host_position += 1;
    return FAH_OK;
  });
  const std::string message = status != FAH_OK ? fah_last_error() : std::string();
  for (int i = 0; i < count; ++i) {
    ok[i]->status = status;
    ok[i]->error = message;
    ok[i]->token = tokens[i];
  }
}

}  // namespace

extern "C" {

int fah_batcher_step(fah_batcher* b, fah_decoder* session, int32_t* token) {
  if (!b || !session || !token) return fail(FAH_ERROR_ARGUMENT, "batcher/session/token is NULL");
  if (session->wt != b->wt || session->ctx != b->ctx)
    return fail(FAH_ERROR_ARGUMENT, "session does not share the batcher's weights");
  // The session's own checks first: a step it cannot take fails here, for
  // this caller alone, and never enters a batch.
  const int checked = guarded_decoder([&] {
    check_batch_session(b, session);
    return FAH_OK;
  });
  if (checked != FAH_OK) return checked;
  BatchRequest req;
  req.session = session;
  std::unique_lock<std::mutex> lk(b->m);
  for (BatchRequest* r : b->pending)
    if (r->session == session) return fail(FAH_ERROR_STATE, "the session already has a step pending");
  b->pending.push_back(&req);
  b->arrivals.fetch_add(1, std::memory_order_release);
  b->idle.erase(std::remove(b->idle.begin(), b->idle.end(), session), b->idle.end());
  b->cv.notify_all();
  while (!req.done) {
    if (!b->running) {
      // Leader: collect the steps of the joined sessions that are stepping
      // (or of whoever arrives within the window), then run them as one
      // batch. A joined session that had no step in the last batch is idle
      // and not waited for until it requests a step again.
      b->running = true;
      const auto deadline = std::chrono::steady_clock::now() + b->window;
      auto is_joined = [&](const fah_decoder* d) {
        return std::find(b->joined.begin(), b->joined.end(), d) != b->joined.end();
      };
      auto want = [&] {
        size_t joined_pending = 0;
        for (BatchRequest* r : b->pending)
          if (is_joined(r->session)) ++joined_pending;
        const size_t expected = b->joined.size() - b->idle.size();
        return b->pending.size() >= (size_t)fah::kFewFrames || (expected > 0 && joined_pending >= expected);
      };
      while (!want()) {
        // Spin a little for the next arrival before blocking (arrivals come
        // microseconds apart when every session is stepping).
        const int64_t seen = b->arrivals.load(std::memory_order_acquire);
        lk.unlock();
        const auto spin_until = std::min(deadline, std::chrono::steady_clock::now() + std::chrono::microseconds(500));
        while (b->arrivals.load(std::memory_order_acquire) == seen && std::chrono::steady_clock::now() < spin_until)
          std::this_thread::yield();
        lk.lock();
        if (want()) break;
        if (b->arrivals.load(std::memory_order_acquire) != seen) continue;
        if (std::chrono::steady_clock::now() >= deadline) break;
        if (b->cv.wait_until(lk, deadline) == std::cv_status::timeout) break;
      }
      const size_t n = std::min<size_t>(fah::kFewFrames, b->pending.size());
      std::vector<BatchRequest*> batch(b->pending.begin(), b->pending.begin() + n);
      b->pending.erase(b->pending.begin(), b->pending.begin() + n);
      for (fah_decoder* d : b->joined) {
        bool stepping = false;
        for (BatchRequest* r : batch) stepping = stepping || r->session == d;
        for (BatchRequest* r : b->pending) stepping = stepping || r->session == d;
        if (!stepping && std::find(b->idle.begin(), b->idle.end(), d) == b->idle.end()) b->idle.push_back(d);
      }
      lk.unlock();
      run_batch(b, batch);
      lk.lock();
      int64_t served = 0;
      for (BatchRequest* r : batch) served += r->status == FAH_OK;
      b->batches_run += served > 0;
      b->rows_run += served;
      for (BatchRequest* r : batch) r->done.store(true, std::memory_order_release);  // (last access)
      b->running = false;
      b->cv.notify_all();
      continue;
    }
    // Another thread leads: spin a little (a batch ends within a step's
    // time; 16 blocked waiters would otherwise wake one after another
    // through the lock), then block.
    lk.unlock();
    const auto spin_until = std::chrono::steady_clock::now() + std::chrono::milliseconds(3);
    while (!req.done.load(std::memory_order_acquire) && b->running.load(std::memory_order_acquire) &&
           std::chrono::steady_clock::now() < spin_until)
      std::this_thread::yield();
    if (req.done.load(std::memory_order_acquire)) break;
    lk.lock();
    if (!req.done.load(std::memory_order_acquire) && b->running) b->cv.wait(lk);
  }
  if (lk.owns_lock()) lk.unlock();
  if (req.status != FAH_OK) return fail(req.status, req.error);
  *token = req.token;
  return FAH_OK;
}

int fah_batcher_stats(fah_batcher* b, int64_t* batches, int64_t* rows) {
  if (!b || !batches || !rows) return fail(FAH_ERROR_ARGUMENT, "batcher/batches/rows is NULL");
  std::lock_guard<std::mutex> lk(b->m);
  *batches = b->batches_run;
  *rows = b->rows_run;
  return FAH_OK;
}

int fah_decoder_kv_write(fah_decoder* d, int layer, const uint16_t* keys, const uint16_t* values, int positions) {
  if (!d) return fail(FAH_ERROR_ARGUMENT, "decoder is NULL");
  return guarded_decoder([&] {
    const fah_decoder_config& k = d->cfg;
    require(layer >= 0 && layer < k.layers && positions >= 0 && positions <= k.capacity && keys && values,
            "invalid KV write");
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    hipStream_t s = d->ctx->stream;
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    DeviceWork work(*d->ctx);
    size_t layer_elems = (size_t)k.kv_heads * k.capacity * k.head_size;
    for (int h = 0; h < k.kv_heads; ++h) {
      // host [t][h][c] -> device [h][t][c]
      check(hipMemcpy2DAsync(d->kcache.as<uint16_t>() + layer_elems * layer + (size_t)h * k.capacity * k.head_size,
                             (size_t)k.head_size * 2, keys + (size_t)h * k.head_size, (size_t)d->kv_width * 2,
                             (size_t)k.head_size * 2, positions, hipMemcpyHostToDevice, s),
            "H2D keys");
      check(hipMemcpy2DAsync(d->vcache.as<uint16_t>() + layer_elems * layer + (size_t)h * k.capacity * k.head_size,
                             (size_t)k.head_size * 2, values + (size_t)h * k.head_size, (size_t)d->kv_width * 2,
                             (size_t)k.head_size * 2, positions, hipMemcpyHostToDevice, s),
            "H2D values");
    }
    check(hipStreamSynchronize(s), "sync");
    return FAH_OK;
  });
}

int fah_decoder_kv_read(fah_decoder* d, int layer, uint16_t* keys, uint16_t* values, int positions) {
  if (!d) return fail(FAH_ERROR_ARGUMENT, "decoder is NULL");
  return guarded_decoder([&] {
    const fah_decoder_config& k = d->cfg;
    require(layer >= 0 && layer < k.layers && positions >= 0 && positions <= k.capacity && keys && values,
            "invalid KV read");
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    hipStream_t s = d->ctx->stream;
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    DeviceWork work(*d->ctx);
    size_t layer_elems = (size_t)k.kv_heads * k.capacity * k.head_size;
    for (int h = 0; h < k.kv_heads; ++h) {
      check(hipMemcpy2DAsync(keys + (size_t)h * k.head_size, (size_t)d->kv_width * 2,
                             d->kcache.as<uint16_t>() + layer_elems * layer + (size_t)h * k.capacity * k.head_size,
                             (size_t)k.head_size * 2, (size_t)k.head_size * 2, positions, hipMemcpyDeviceToHost, s),
            "D2H keys");
      check(hipMemcpy2DAsync(values + (size_t)h * k.head_size, (size_t)d->kv_width * 2,
                             d->vcache.as<uint16_t>() + layer_elems * layer + (size_t)h * k.capacity * k.head_size,
                             (size_t)k.head_size * 2, (size_t)k.head_size * 2, positions, hipMemcpyDeviceToHost, s),
            "D2H values");
    }
    check(hipStreamSynchronize(s), "sync");
    return FAH_OK;
  });
}

int64_t fah_decoder_weight_bytes(const fah_decoder* d) { return d ? d->wt->weight_bytes : 0; }

int fah_decoder_persistent(const fah_decoder* d) { return d && d->persistent ? (d->pargs.local_l2 ? 2 : 1) : 0; }

int fah_decoder_timeline(fah_decoder* d, uint64_t* ticks, int count) {
  if (!d || !ticks) return fail(FAH_ERROR_ARGUMENT, "decoder/ticks is NULL");
  if (!d->timeline.ptr) return FAH_DECLINED;
  return guarded_decoder([&] {
    require(count >= 0 && count <= d->blocks * fah::kTimelineEvents, "invalid timeline size");
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    DeviceWork work(*d->ctx);
    check(hipMemcpyAsync(ticks, d->timeline.ptr, (size_t)count * 8, hipMemcpyDeviceToHost, d->ctx->stream),
          "D2H timeline");
    check(hipStreamSynchronize(d->ctx->stream), "sync");
    return FAH_OK;
  });
}

int fah_decoder_attention_time(fah_decoder* d, double* milliseconds, int* steps) {
  if (!d || !milliseconds || !steps) return fail(FAH_ERROR_ARGUMENT, "decoder/milliseconds/steps is NULL");
  if (!d->attention_times) return FAH_DECLINED;
  return guarded_decoder([&] {
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    *milliseconds = d->attn_ms;
    *steps = d->attn_steps;
    d->attn_ms = 0.0;
    d->attn_steps = 0;
    return FAH_OK;
  });
}

int fah_decoder_trace(fah_decoder* d, int which, float* out, int count) {
  if (!d) return fail(FAH_ERROR_ARGUMENT, "decoder is NULL");
  return guarded_decoder([&] {
    const fah_decoder_config& k = d->cfg;
    const int sizes[5] = {k.width, d->q_width + 2 * d->kv_width, d->q_width, k.width, k.ffn};
    require(which >= 0 && which < 5 && out && count >= 0 && count <= sizes[which], "invalid trace request");
    std::lock_guard<std::mutex> lock(d->ctx->gate);
    require_live(d);
    check(hipSetDevice(d->ctx->device), "hipSetDevice");
    DeviceWork work(*d->ctx);
    hipStream_t s = d->ctx->stream;
    if (d->persistent) {
      DeviceBuffer* tagged[5] = {&d->tx, &d->tqkv, &d->tatt, &d->ta, &d->th};
      std::vector<unsigned long long> words(count);
      check(hipMemcpyAsync(words.data(), tagged[which]->ptr, (size_t)count * 8, hipMemcpyDeviceToHost, s),
            "D2H trace");
      check(hipStreamSynchronize(s), "sync");
      for (int i = 0; i < count; ++i) {
        uint32_t bits = (uint32_t)words[i];
        std::memcpy(&out[i], &bits, 4);
      }
    } else {
      DeviceBuffer* plain[5] = {&d->x, &d->qkv_out, &d->attn, &d->a, &d->h};
      check(hipMemcpyAsync(out, plain[which]->ptr, (size_t)count * 4, hipMemcpyDeviceToHost, s), "D2H trace");
      check(hipStreamSynchronize(s), "sync");
    }
    return FAH_OK;
  });
}

}  // extern "C"
