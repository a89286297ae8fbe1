// Persistent decode step: the whole Qwen3 decoder row (28 layers + lm_head +
// greedy) in one launch of one workgroup per CU.
//
// Every workgroup owns a fixed slice of rows of every projection. A layer is
// five phases -- qkv, attention, o, gate/up, down -- separated by exchanges
// of the activation vector through global memory. Each value is published
// as a 64-bit word (generation << 32 | float bits) with one relaxed store,
// so a consumer sees value and readiness in the same load. The attention
// output and the ffn activations, which the next phase quantises without a
// norm, travel already quantised (Q8_0 blocks with 16-bit tags), each
// 128-byte line written by a single workgroup.
//
// Placement: the hardware deals a launch's workgroups to the eight XCDs in
// turn. The attention workgroups of kv head x and the workgroups that form
// that head's q/k/v rows all sit on XCD x, and the ffn rows of block pair p
// are computed on XCD p % 8, so those hand-overs stay in one L2 (stores
// that are not written through); the other exchanges cross XCDs
// (device-scope stores, device-coherent loads).
//
// Roles inside a projection workgroup (8 waves, two per SIMD):
//  * waves 0-3 are the memory waves: they gather the next phase's input, a
//    part of the chunks each (wave 0 also fetches the small per-layer
//    constants in the same batch), after a short sleep, polling a part of
//    one chunk whole and longer parts through their last 64 bytes, so that
//    the polls of all consumers stay a small part of the traffic. Wave 0
//    also sums the phase's rows in order and publishes them, and the ffn
//    block-pair owners' wave 0 quantises and publishes the pair.
//  * waves 4-7 are the compute waves: while the attention runs they copy
//    the layer's weight slices (and the next layer's q/k/v slice) into LDS,
//    so that no weight stream overlaps an exchange.
//  * all eight quantise the phase input and form the block products from
//    the LDS slices.
// Attention workgroups use all eight waves for the scores, the softmax and
// the K/V staging; two of them run the time-ordered value sums.
// The arithmetic of every phase is the one of the multi-kernel path
// (bit-identical GEMV order, RMSNorm sum tree, exact softmax and
// time-ordered value sums).
//
// Every wait is bounded: a missing generation sets the error word and the
// workgroup leaves, so a broken launch ends instead of hanging.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "fah_device.h"
#include "fah_internal.h"

namespace fah {
namespace {

constexpr int kPT = 512;                 // threads per workgroup (8 waves, two per SIMD)
constexpr int kMem = 256;                // memory threads (waves 0-3): gathers, row sums
constexpr int kComp = kPT - kMem;        // compute threads (waves 4-7): weight slices
constexpr int kSlotPairs = 4;            // (row, block) pairs per compute lane per phase
constexpr int kActFloats = 4096;         // largest phase input (ffn <= 4096)
constexpr int kTagWords = kActFloats * 3 / 4;  // gathered words held in LDS
constexpr int kProdFloats = 1024;        // (row, block) products of one phase
constexpr int kKvBytes = 121 * 1024;     // K/V staging: 512 B per position
constexpr int kProbOffset = 4 * 128;     // attention probabilities after q/k/v in the tag area
constexpr long kSpinLimit = 1L << 21;    // bounded polls per gather (~1-2 s)
// Positions an attention workgroup takes: the V rows of the earlier ones
// fill its K/V area (256 B each), their K rows sit in registers (two passes
// of 256 positions, two lanes each), their probabilities in the gather
// area after the q/k/v words.
constexpr int kExactPositions = kKvBytes / 256;
static_assert(kExactPositions <= 512 && kProbOffset + (kExactPositions + 1) / 2 <= kTagWords, "attention layout");
// Long caches (positions from PersistentArgs::long_from on): the projection
// workgroups of an XCD score the earlier positions of its kv head, the
// attention workgroup gathers those scores (tagged words at the end of its
// K/V area), forms the probabilities of all n = pos + 1 positions in the
// gather area after the q/k/v words and publishes them; the value sums run
// on projection workgroups of the same XCD, one per (query head, 32-channel
// block), each streaming its slice of the V rows and the probabilities
// through a ring of kValSlots blocks of kValPos positions.
constexpr int kLongPositions = 2 * (kTagWords - kProbOffset);
constexpr int kScoreBytes = kLongPositions * 8, kScoreOffset = kKvBytes - kScoreBytes;
static_assert(kExactPositions <= kLongPositions && kLongPositions % 128 == 0, "long attention layout");
constexpr int kValPos = 64;                       // positions per value block
constexpr int kValCh = 32;                        // channels per value workgroup (one quantised block)
constexpr int kValRow = kValPos + 4;              // product row (floats): 4-bank offset per chain
constexpr int kValPSlot = kValCh * kValRow * 4;   // product slot: 32 chains
constexpr int kValVBytes = kValPos * kValCh * 2;  // V slice of a block (fp16)
constexpr int kValSlot = kValVBytes + kValPos * 8;  // V slice, then the block's tagged probabilities
constexpr int kValSlots = 12;                     // V/probability ring depth (blocks)
constexpr int kValRing = kKvBytes - kValSlots * kValSlot;  // the ring sits at the end of the K/V area
static_assert(4 * (kValSlots - 3) <= 63, "ring wait counts");
// A wave polls a sentinel first when its part of a gather has more than this
// many 1 KB chunks; a part of one chunk is polled whole (one round trip
// sooner, and little enough traffic).
constexpr int kSentinelChunks = 1;
// Sentinel polls in flight per gathering wave. Every consumer polls the same
// few words, so deeper pipelines lengthen the queue in front of them:
// measured on the decode step (with the gather delay below), 2 is a little
// faster than 1, and 4 and 8 are slower.
constexpr int kPolls = 2;
// A gather sleeps this long (64-cycle units, about 0.7 us) before its first
// poll: no data can arrive sooner, and polls issued earlier only queue in
// front of the producers' stores. Measured on the decode step: 16 and 32
// are slower, 48 far slower; sleeping after a stale poll is slower too.
constexpr int kGatherDelay = 24;
// s_waitcnt immediate for vmcnt <= kPolls - 1 (expcnt and lgkmcnt not
// waited on): vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
constexpr int kWaitOldestPoll = ((kPolls - 1) & 15) | (((kPolls - 1) >> 4) << 14) | (7 << 4) | (15 << 8);
using u64 = unsigned long long;
using lds_ptr = __attribute__((address_space(3))) void*;

__device__ __forceinline__ void lds_barrier_p() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Workgroup barrier that orders LDS without waiting for this wave's direct
// global->LDS loads still in flight (a release fence on LDS drains them
// all): every wave's own LDS reads and writes are complete first (skipped
// with READS_ONLY by a wave whose reads in flight are of data nobody
// overwrites before its next barrier); direct loads that the other waves
// read are waited for on their issuing wave's counter before it arrives.
// The memory clobber keeps the compiler's LDS accesses on their side.
template <bool READS_ONLY = false>
__device__ __forceinline__ void lds_barrier_nodma() {
  if (READS_ONLY) asm volatile("s_barrier" ::: "memory");
  else asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// 16 bytes of LDS read past the compiler, which would drain every direct
// global->LDS load of this wave first (it cannot tell the addresses apart).
__device__ __forceinline__ uint4 lds_read16_nodma(const __attribute__((address_space(3))) char* p) {
  uint4 v;
  const uint32_t at = (uint32_t)(uintptr_t)p;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(at) : "memory");
  return v;
}

// s_waitcnt for vmcnt <= n with n known only at run time (0 <= n < N;
// expcnt and lgkmcnt not waited on): vmcnt bits [3:0] and [15:14].
template <int... I>
__device__ __forceinline__ void vm_wait_n(int n, std::integer_sequence<int, I...>) {
  ((n == I ? __builtin_amdgcn_s_waitcnt((I & 15) | ((I >> 4) << 14) | (7 << 4) | (15 << 8)) : (void)0), ...);
}
template <int N>
__device__ __forceinline__ void vm_wait(int n) {
  vm_wait_n(n, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ void tag_store(u64* p, uint32_t gen, float v) {
  __hip_atomic_store(p, ((u64)gen << 32) | (u64)f2u(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tag_store_bits(u64* p, uint32_t gen, uint32_t bits) {
  __hip_atomic_store(p, ((u64)gen << 32) | (u64)bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Store that other workgroups of the same XCD read through its L2 (not
// written through to memory).
__device__ __forceinline__ void tag_store_local(u64* p, uint32_t gen, float v) {
  __hip_atomic_store(p, ((u64)gen << 32) | (u64)f2u(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// The XCD this wave runs on (hardware register XCC_ID, bits 3:0).
__device__ __forceinline__ int xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15; }
__device__ __forceinline__ unsigned error_load(const unsigned* e) {
  return __hip_atomic_load(e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Phase timeline (100 MHz s_memrealtime) of every workgroup, when the
// caller asked for one.
__device__ __forceinline__ void stamp(unsigned long long* timeline, int slot, int event) {
  if (timeline && event < kTimelineEvents) timeline[slot * kTimelineEvents + event] = __builtin_amdgcn_s_memrealtime();
}

// Wave-level direct global->LDS copy of `bytes` (a multiple of 16): lane i of
// instruction c moves bytes [1024c + 16i, +16).
__device__ __forceinline__ void dma(const void* src, void* lds, int bytes) {
  const int lane = threadIdx.x & (kWave - 1);
  for (int c = 0; c < bytes; c += 1024)
    if (c + 16 * lane < bytes)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(src) + c + 16 * lane,
                                       (lds_ptr)(reinterpret_cast<char*>(lds) + c), 16, 0, 0);
}

// K/V rows [t0, t1) of one kv head into kv: position t at byte 512(t - t0),
// K 256 B then V 256 B; one instruction moves two positions (lanes: K t,
// V t, K t+1, V t+1). The 16-byte pieces of a K row are stored XOR-swizzled
// by (t & 15), so that 16 lanes reading piece i of 16 consecutive rows hit
// 16 different bank groups; V rows stay in order (read one row at a time).
__device__ __forceinline__ void dma_kv(const _Float16* kb, const _Float16* vb, int t0, int t1, char* kv, int first = 0,
                                       int stride = 1) {
  const int lane = threadIdx.x & (kWave - 1);
  for (int m = first; t0 + 2 * m < t1; m += stride) {
    const int t = t0 + 2 * m + (lane >> 5);
    if (t < t1) {
      const bool v = (lane >> 4) & 1;
      const int piece = v ? (lane & 15) : ((lane & 15) ^ (t & 15));
      const _Float16* src = (v ? vb : kb) + (size_t)t * 128 + piece * 8;
      __builtin_amdgcn_global_load_lds(src, (lds_ptr)(kv + (size_t)m * 1024), 16, 0, 0);
    }
  }
}

struct NoPre {
  __device__ void operator()() const {}
};

// One wave gathers tagged words into the LDS staging area `tag` (one u64
// per value; consumers read the low 32 bits). Ranges are multiples of 128
// words (chunks); each chunk is one direct global->LDS load of 16 bytes per
// lane. The chunks are split into `parts` contiguous parts and this wave
// takes part `part`, so that several waves can share a vector (a wave issues
// its loads one after another). `pre` issues the plain constant copies
// once, before the first poll, so they share its wait. Chunks whose tags do
// not all carry `gen` are issued again until every chunk is current.
// Returns false after a timeout or when another workgroup reported an error.
struct NoChunk {
  __device__ void operator()(int) const {}
};

template <class Pre, class OnChunk = NoChunk>
__device__ __forceinline__ bool gather(const u64* s0, int n0, int o0, const u64* s1, int n1, int o1, const u64* s2, int n2, int o2,
                       uint32_t gen, u64* tag, unsigned* error, Pre pre, int part = 0, int parts = 1,
                       OnChunk on_chunk = OnChunk{}, u64* seen = nullptr, uint32_t tmask = ~0u) {
  const int lane = threadIdx.x & (kWave - 1);
  pre();
  const int c0 = n0 >> 7, c01 = c0 + (n1 >> 7), all = c01 + (n2 >> 7);
  const int first = part * all / parts, total = (part + 1) * all / parts;
  if (total <= first) return true;
  u64 pending = (total >= 64 ? ~0ull : ((1ull << total) - 1ull)) & ~((1ull << first) - 1ull);
  auto locate = [&](int k, const u64*& src, int& off) {
    if (k < c0) {
      src = s0 + (k << 7);
      off = o0 + (k << 7);
    } else if (k < c01) {
      src = s1 + ((k - c0) << 7);
      off = o1 + ((k - c0) << 7);
    } else {
      src = s2 + ((k - c01) << 7);
      off = o2 + ((k - c01) << 7);
    }
  };
  long spin = 0;
  __builtin_amdgcn_s_sleep(kGatherDelay);
  // Poll the end of the last chunk until it is current before reading them
  // all (that chunk too), so that consumers that arrive early cost one small
  // load per round trip instead of the whole vector.
  if (total - first > kSentinelChunks) {
    const u64* src;
    int off;
    locate(total - 1, src, off);
    // kPolls sentinel loads in flight, all into the chunk's own LDS place:
    // returns complete in order, so after waiting for the oldest the LDS copy
    // is at least that new.
    // Only the chunk's last 64 bytes (lanes 0-3) are polled: the polls of
    // every consumer together stay a small part of the memory traffic.
    for (int i = 0; i < kPolls - 1; ++i)
      if (lane < 4) __builtin_amdgcn_global_load_lds(src + 120 + 2 * lane, (lds_ptr)(tag + off + 120), 16, 0, 16);
    for (;; ++spin) {
      if (lane < 4) __builtin_amdgcn_global_load_lds(src + 120 + 2 * lane, (lds_ptr)(tag + off + 120), 16, 0, 16);
      __builtin_amdgcn_s_waitcnt(kWaitOldestPoll);
      const uint4 t = lane < 4 ? *reinterpret_cast<const uint4*>(tag + off + 120 + 2 * lane) : make_uint4(0, gen, 0, gen);
      if (__all((t.y & tmask) == gen && (t.w & tmask) == gen)) {
        if (seen) seen[0] = __builtin_amdgcn_s_memrealtime();
        break;
      }
      if (spin > kSpinLimit || ((spin & 63) == 63 && error_load(error))) {
        if (lane == 0) __hip_atomic_fetch_or(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // Drained here so that no store is pending where the waves rejoin.
        __builtin_amdgcn_s_waitcnt(0);
        return false;
      }
    }
  }
  if (total - first == 1) {
    // One chunk: polled whole with two reads in flight, the newer issued
    // before the older is checked. Both land in the chunk's LDS place and
    // each lane's 16 bytes land whole, so a checked lane holds intact words;
    // a later read returns data at least as new.
    const u64* src;
    int off;
    locate(first, src, off);
    auto poll = [&] { __builtin_amdgcn_global_load_lds(src + 2 * lane, (lds_ptr)(tag + off), 16, 0, 16); };
    // s_waitcnt immediate: vmcnt <= 1 (the newer read), expcnt/lgkmcnt not waited.
    constexpr int kWaitOlderRead = 1 | (7 << 4) | (15 << 8);
    poll();
    for (;; ++spin) {
      poll();
      __builtin_amdgcn_s_waitcnt(kWaitOlderRead);
      const uint4 t = *reinterpret_cast<const uint4*>(tag + off + 2 * lane);
      if (__all((t.y & tmask) == gen && (t.w & tmask) == gen)) {
        // Drained: the newer read writes the same current words.
        __builtin_amdgcn_s_waitcnt(0);
        on_chunk(first);
        if (seen) seen[1] = 1;
        return true;
      }
      if (spin > kSpinLimit || ((spin & 63) == 63 && error_load(error))) {
        if (lane == 0) __hip_atomic_fetch_or(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        return false;
      }
    }
  }
  int rounds = 0;
  for (;; ++spin) {
    if (!pending) {
      if (seen) seen[1] = rounds;
      return true;
    }
    ++rounds;
    for (u64 m = pending; m; m &= m - 1) {
      const u64* src;
      int off;
      locate(__builtin_ctzll(m), src, off);
      // aux 16 = sc1: device-coherent read, as relaxed agent-scope atomic loads use.
      __builtin_amdgcn_global_load_lds(src + 2 * lane, (lds_ptr)(tag + off), 16, 0, 16);
    }
    __builtin_amdgcn_s_waitcnt(0);
    for (u64 m = pending; m; m &= m - 1) {
      const int k = __builtin_ctzll(m);
      const u64* src;
      int off;
      locate(k, src, off);
      const uint4 t = *reinterpret_cast<const uint4*>(tag + off + 2 * lane);
      if (__all((t.y & tmask) == gen && (t.w & tmask) == gen)) {
        pending &= ~(1ull << k);
        on_chunk(k);
      }
    }
    if (!pending) return true;
    if (spin > kSpinLimit || ((spin & 63) == 63 && error_load(error))) {
      if (lane == 0) __hip_atomic_fetch_or(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // Drained here so that no store is pending where the waves rejoin.
      __builtin_amdgcn_s_waitcnt(0);
      return false;
    }
  }
}

// The attention workgroup's q, k and v (three 128-word chunks), polled
// directly: rounds of three loads, two rounds in flight, each round's
// chunks checked when it has returned. Its few consumers make the polling
// traffic negligible, and the data are seen one round trip after they are
// current instead of a sentinel's round trip plus a read's. Each lane's
// 16 bytes land in LDS whole, so every tagged word it checks is intact.
template <class Pre>
__device__ __forceinline__ bool gather_qkv(const u64* q, const u64* k, const u64* v, uint32_t gen, u64* tag, unsigned* error, Pre pre,
                           u64* seen = nullptr) {
  const int lane = threadIdx.x & (kWave - 1);
  pre();
  auto round = [&] {
    __builtin_amdgcn_global_load_lds(q + 2 * lane, (lds_ptr)(tag), 16, 0, 16);
    __builtin_amdgcn_global_load_lds(k + 2 * lane, (lds_ptr)(tag + 128), 16, 0, 16);
    __builtin_amdgcn_global_load_lds(v + 2 * lane, (lds_ptr)(tag + 256), 16, 0, 16);
  };
  // s_waitcnt immediate: vmcnt <= 3 (the newer round), expcnt/lgkmcnt not waited.
  constexpr int kWaitOlderRound = 3 | (7 << 4) | (15 << 8);
  round();
  unsigned done = 0;
  for (long spin = 0;; ++spin) {
    round();
    __builtin_amdgcn_s_waitcnt(kWaitOlderRound);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const uint4 t = *reinterpret_cast<const uint4*>(tag + 128 * c + 2 * lane);
      if (__all(t.y == gen && t.w == gen)) done |= 1u << c;
    }
    if (done == 7u) {
      if (seen) seen[0] = __builtin_amdgcn_s_memrealtime();
      // Drained: the newer round writes the same current words.
      __builtin_amdgcn_s_waitcnt(0);
      return true;
    }
    if (spin > kSpinLimit || ((spin & 63) == 63 && error_load(error))) {
      if (lane == 0) __hip_atomic_fetch_or(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      return false;
    }
  }
}

template <class Pre>
__device__ __forceinline__ bool gather1(const u64* src, int count, uint32_t gen, u64* tag, unsigned* error, Pre pre) {
  return gather(src, count, 0, nullptr, 0, 0, nullptr, 0, 0, gen, tag, error, pre);
}

__device__ __forceinline__ float tag_value(const u64* tag, int i) { return u2f((uint32_t)tag[i]); }


// The whole value sum of channel c = 2 * lane + HI over positions [0, pos]:
// the V rows of positions [0, nlds) staged at 256 B per position in vs, later
// ones read from vglob (this layer and head), this position's value in
// cur[2]. Writes cur[0][c].
template <bool HI>
__device__ __forceinline__ void value_chain(const char* vs, const float* p, int nlds, int pos,
                                            const _Float16* vglob, float (*cur)[128]) {
  const int lane = threadIdx.x & (kWave - 1), c = 2 * lane + (HI ? 1 : 0);
  float acc = 0.0f;
  value_region<HI>(vs, p, 0, nlds, acc);
  int t = nlds;
  const _Float16* vg = vglob + c;
  for (; t + 8 <= pos; t += 8) {
    _Float16 x[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = vg[(size_t)(t + k) * 128];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc = fadd(acc, mulh(p[t + k], x[k]));
  }
  for (; t < pos; ++t) acc = fadd(acc, mulh(p[t], vg[(size_t)t * 128]));
  acc = fadd(acc, fmul(cur[2][c], p[pos]));
  cur[0][c] = acc;
}


// Half a K row piece: four F16 channels 8i + 4h .. 8i + 4h + 3 into the
// four accumulators of lane parity h (q[0..3] the matching q channels).
__device__ __forceinline__ void score4_regs(float* acc, const uint2& kk, const float* q) {
  const uint32_t w[2] = {kk.x, kk.y};
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(w[m] & 0xffffu));
    const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(w[m] >> 16));
    acc[2 * m] = fadd(acc[2 * m], mulh(q[2 * m], lo));
    acc[2 * m + 1] = fadd(acc[2 * m + 1], mulh(q[2 * m + 1], hi));
  }
}

// One position's score by a lane pair (lane parity h, its K row halves in
// k, the matching q channels in q): eight accumulators over channels j,
// j + 8, ..., four in each lane, then the pairwise tree
// ((a0 + a4) + (a1 + a5)) + ((a2 + a6) + (a3 + a7)) formed by both lanes
// from the partner's accumulators, divided by the divisor
// (AttentionAvx.cs:74-160).
__device__ __forceinline__ float pair_score(const uint2* k, const float* q, int h, float divisor) {
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < 16; ++i) score4_regs(acc, k[i], q + 4 * i);
  float o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = u2f(dpp_u32<kDppQuadXor1>(f2u(acc[j])));
  const float* lo = h ? o : acc;
  const float* hi = h ? acc : o;
  const float sc = fadd(fadd(fadd(lo[0], hi[0]), fadd(lo[1], hi[1])), fadd(fadd(lo[2], hi[2]), fadd(lo[3], hi[3])));
  return fdiv(sc, divisor);
}

// A compute lane's share of one weight slice: P (row, block) pairs, each 32
// int8 weights and the block's F16 scale.
template <int P>
struct Slot {
  int4 w[P][2];
  _Float16 s[P];
};

// Load this compute lane's pairs j = ct + kComp*i (i < ceil(NP/kComp)) of a
// slice of `valid` pairs. Lanes past the end re-read the last pair, so every
// lane issues the same, compile-time number of loads per slice.
template <int NP, int P>
__device__ __forceinline__ void load_slot(Slot<P>& sl, const int8_t* w, const _Float16* s, int ct, int valid) {
  constexpr int kI = (NP + kComp - 1) / kComp;
  static_assert(kI <= P, "slot capacity");
#pragma unroll
  for (int i = 0; i < kI; ++i) {
    int j = ct + i * kComp;
    j = j < valid ? j : valid - 1;
    const int4* p = reinterpret_cast<const int4*>(w + (size_t)j * 32);
    sl.w[i][0] = p[0];
    sl.w[i][1] = p[1];
    sl.s[i] = s[j];
  }
}

__device__ __forceinline__ int dot32(const int4& w0, const int4& w1, const int* xq) {
  const int4* xp = reinterpret_cast<const int4*>(xq);
  int4 x0 = xp[0], x1 = xp[1];
  int d = 0;
  d = __builtin_amdgcn_sdot4(w0.x, x0.x, d, false);
  d = __builtin_amdgcn_sdot4(w0.y, x0.y, d, false);
  d = __builtin_amdgcn_sdot4(w0.z, x0.z, d, false);
  d = __builtin_amdgcn_sdot4(w0.w, x0.w, d, false);
  d = __builtin_amdgcn_sdot4(w1.x, x1.x, d, false);
  d = __builtin_amdgcn_sdot4(w1.y, x1.y, d, false);
  d = __builtin_amdgcn_sdot4(w1.z, x1.z, d, false);
  d = __builtin_amdgcn_sdot4(w1.w, x1.w, d, false);
  return d;
}

// Scaled block products of a slot into prod[r * (B + 4) + b] (pairs
// j < valid; pair j is row j / B, block j % B of the slice). Rows are padded
// by four floats so that the lanes summing different rows read different
// LDS banks.
template <int NP, int B, int P>
__device__ __forceinline__ void slot_products(const Slot<P>& sl, int ct, const int* xq, const float* xs, float* prod,
                                              int valid) {
  constexpr int kI = (NP + kComp - 1) / kComp;
#pragma unroll
  for (int i = 0; i < kI; ++i) {
    const int j = ct + i * kComp;
    if (j < valid) {
      const int r = j / B, b = j - r * B;
      const int d = dot32(sl.w[i][0], sl.w[i][1], xq + b * 8);
      prod[r * (B + 4) + b] = fmul(fmul((float)d, (float)sl.s[i]), xs[b]);
    }
  }
}

// Compute lanes: copy a weight slice of `rows` storage rows (K int8 each,
// storage row row(r) for slice row r) and then their K / 32 F16 scales into
// LDS at dst, by direct global->LDS loads of 16-byte pieces, R rounds of
// kComp pieces: piece p of the slice lands at dst + 16 p. Pieces past the
// slice re-read its first one into the unused tail (dst holds R rounds).
template <int K, int R, class RowMap>
__device__ __forceinline__ void stage_slice(char* dst, const int8_t* w, const _Float16* s, int rows, int ct,
                                            RowMap row) {
  static_assert(K % 256 == 0, "whole 16-byte pieces of weights and scales");
  constexpr int PW = K / 16, PS = K / 256;  // pieces per row: weights, scales
  const int nw = rows * PW, n = nw + rows * PS;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int p = kComp * k + ct;
    const char* src;
    if (p < nw) {
      const int r = p / PW;
      src = reinterpret_cast<const char*>(w + (size_t)row(r) * K) + 16 * (p - r * PW);
    } else if (p < n) {
      const int q = p - nw, r = q / PS;
      src = reinterpret_cast<const char*>(s + (size_t)row(r) * (K / 32)) + 16 * (q - r * PS);
    } else {
      src = reinterpret_cast<const char*>(w + (size_t)row(0) * K);
    }
    // aux 2 = nt: the layer weights stream through once a token and would
    // only evict the lm_head's rows (read again every token) from the
    // memory-side cache.
    __builtin_amdgcn_global_load_lds(src, (lds_ptr)(dst + 16 * (kComp * k + (ct & ~(kWave - 1)))), 16, 0, 2);
  }
}

// Rounds of stage_slice for slices of up to `rows` rows of K weights.
__host__ __device__ constexpr int stage_rounds(int rows, int K) { return (rows * (K / 16 + K / 256) + kComp - 1) / kComp; }

// slot_products for a slice staged in LDS by stage_slice (`rows` rows), on
// all the workgroup's threads (the memory waves have nothing to wait for
// while the products form).
template <int NP, int B>
__device__ __forceinline__ void lds_products(const char* sl, int rows, const int* xq, const float* xs, float* prod) {
  constexpr int K = 32 * B, kI = (NP + kPT - 1) / kPT;
  const int valid = rows * B;
  const _Float16* sc = reinterpret_cast<const _Float16*>(sl + (size_t)rows * K);
#pragma unroll
  for (int i = 0; i < kI; ++i) {
    const int j = (int)threadIdx.x + i * kPT;
    if (j < valid) {
      const int r = j / B, b = j - r * B;
      const int4* wp = reinterpret_cast<const int4*>(sl + (size_t)r * K + 32 * b);
      const int d = dot32(wp[0], wp[1], xq + b * 8);
      prod[r * (B + 4) + b] = fmul(fmul((float)d, (float)sc[j]), xs[b]);
    }
  }
}

// Rows [r0, r0 + count) of R rows split as evenly as possible over NG
// workgroups (the first R % NG take one more).
struct Rows {
  int r0, count;
};
template <int R, int NG>
__device__ __forceinline__ Rows split_rows(int g) {
  constexpr int base = R / NG, extra = R % NG;
  return {g * base + (g < extra ? g : extra), base + (g < extra ? 1 : 0)};
}

// Ordered block sum from 0f of one row of products (row r of the layout
// above, 16-byte aligned) (TensorMath.QuantizedRowsAvx.cs:27-58).
template <int B>
__device__ __forceinline__ float ordered_sum(const float* prod, int r) {
  static_assert(B % 16 == 0, "whole float4 batches");
  const float* row = prod + r * (B + 4);
  float sum = 0.0f;
  // Batches of 16 products, the next batch's reads issued before the
  // current batch is added (one LDS round trip in all, not one a batch).
  float4 q[2][4];
  auto load = [&](float4* d, int b) {
#pragma unroll
    for (int k = 0; k < 4; ++k) d[k] = *reinterpret_cast<const float4*>(row + b + 4 * k);
  };
  auto add = [&](const float4* d) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      sum = fadd(sum, d[k].x);
      sum = fadd(sum, d[k].y);
      sum = fadd(sum, d[k].z);
      sum = fadd(sum, d[k].w);
    }
  };
  load(q[0], 0);
#pragma unroll
  for (int b = 0; b < B; b += 16) {
    if (b + 16 < B) load(q[((b >> 4) + 1) & 1], b + 16);
    __builtin_amdgcn_sched_barrier(0);
    add(q[(b >> 4) & 1]);
    __builtin_amdgcn_sched_barrier(0);
  }
  return sum;
}

__device__ __forceinline__ float4 tag_float4(const u64* tag, int e) {
  const uint4 a = *reinterpret_cast<const uint4*>(tag + e);
  const uint4 b = *reinterpret_cast<const uint4*>(tag + e + 2);
  return make_float4(u2f(a.x), u2f(a.z), u2f(b.x), u2f(b.z));
}

// Maximum over each aligned group of 8 lanes, in all 8 lanes.
__device__ __forceinline__ uint32_t max8_u32(uint32_t m) {
  uint32_t o = dpp_u32<kDppQuadXor1>(m);
  m = o > m ? o : m;
  o = dpp_u32<kDppQuadXor2>(m);
  m = o > m ? o : m;
  o = dpp_u32<kDppHalfMirror>(m);
  return o > m ? o : m;
}

// Q8_0 quantisation (TensorMath.QuantizeAvx.cs:15-72) of four consecutive
// values of a 32-value block whose eight lanes form an aligned group of 8
// (all 64 lanes active): the block's absolute maximum over DPP, its scale
// into *scale (every lane of the group) and the four int8 values packed
// little-endian. The per-value arithmetic is quantize_value/block_scale's.
__device__ __forceinline__ uint32_t quantize_lane4(float4 v, float* scale) {
  const uint32_t a0 = f2u(v.x) & 0x7fffffffu, a1 = f2u(v.y) & 0x7fffffffu;
  const uint32_t a2 = f2u(v.z) & 0x7fffffffu, a3 = f2u(v.w) & 0x7fffffffu;
  const uint32_t m01 = a1 > a0 ? a1 : a0, m23 = a3 > a2 ? a3 : a2;
  const uint32_t m = max8_u32(m23 > m01 ? m23 : m01);
  float inv;
  *scale = block_scale(m, &inv);
  return (uint32_t)(uint8_t)quantize_value(v.x, inv) | ((uint32_t)(uint8_t)quantize_value(v.y, inv) << 8) |
         ((uint32_t)(uint8_t)quantize_value(v.z, inv) << 16) | ((uint32_t)(uint8_t)quantize_value(v.w, inv) << 24);
}

// Q8_0 quantisation of act[0, K) into xq/xs, optionally RMS-scaled first
// (x * inverse * w, RmsNorm's order), four values per thread.
template <int K, bool NORM>
__device__ __forceinline__ void quantize4(const u64* act, const float* norm_w, float inverse, int* xq, float* xs) {
  static_assert(K % 256 == 0, "whole waves");
  for (int i = threadIdx.x; i < K / 4; i += kPT) {  // wave-uniform
    const int e = 4 * i;
    float4 v = tag_float4(act, e);
    if constexpr (NORM) {
      const float4 w = *reinterpret_cast<const float4*>(norm_w + e);
      v.x = fmul(fmul(v.x, inverse), w.x);
      v.y = fmul(fmul(v.y, inverse), w.y);
      v.z = fmul(fmul(v.z, inverse), w.z);
      v.w = fmul(fmul(v.w, inverse), w.w);
    }
    float d;
    xq[i] = (int)quantize_lane4(v, &d);
    if ((i & 7) == 0) xs[e >> 5] = d;
  }
}

// Quantised-exchange words (qblock_words layout): 16-bit tag and 16 side
// bits above the 32-bit payload; tags are compared under kQTagMask.
constexpr uint32_t kQTagMask = 0xFFFF0000u;
__device__ __forceinline__ uint32_t qtag(uint32_t gen) { return gen << 16; }
__device__ __forceinline__ void qword_store(u64* p, uint32_t gen, uint32_t side, uint32_t payload) {
  __hip_atomic_store(p, ((u64)(qtag(gen) | (side & 0xFFFFu)) << 32) | (u64)payload, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
// The side bits of word k of a block whose scale is d: the scale's low half
// in word 0, its high half in word 1.
__device__ __forceinline__ uint32_t qside(int k, float d) {
  return k == 0 ? (f2u(d) & 0xFFFFu) : (k == 1 ? f2u(d) >> 16 : 0u);
}

// A gathered quantised vector into the products' xq/xs layout.
template <int K>
__device__ __forceinline__ void unpack_qblocks(const u64* tag, int* xq, float* xs) {
  for (int i = threadIdx.x; i < K / 4; i += kPT) {
    xq[i] = (int)(uint32_t)tag[i];
    if ((i & 7) == 0) xs[i >> 3] = u2f(((uint32_t)(tag[i] >> 32) & 0xFFFFu) | ((uint32_t)(tag[i + 1] >> 32) << 16));
  }
}

// One wave: poll the NW tagged words at[0, NW) (written through this XCD's
// L2 or to memory) into blk until all carry `gen`, two polls in flight as
// gather_qkv. False after a timeout or another workgroup's error.
template <int NW>
__device__ __forceinline__ bool poll_words(const u64* at, uint32_t gen, u64* blk, unsigned* error, u64* seen, uint32_t tmask = ~0u) {
  const int lane = threadIdx.x & (kWave - 1);
  static_assert(NW % 2 == 0 && NW <= 2 * kWave, "16 bytes per lane");
  auto poll = [&] {
    if (lane < NW / 2) __builtin_amdgcn_global_load_lds(at + 2 * lane, (lds_ptr)blk, 16, 0, 16);
  };
  // s_waitcnt immediate: vmcnt <= 1 (the newer poll), expcnt/lgkmcnt not waited.
  constexpr int kWaitOlderPoll = 1 | (7 << 4) | (15 << 8);
  poll();
  for (long spin = 0;; ++spin) {
    poll();
    __builtin_amdgcn_s_waitcnt(kWaitOlderPoll);
    const uint4 t = lane < NW / 2 ? *reinterpret_cast<const uint4*>(blk + 2 * lane) : make_uint4(0, gen, 0, gen);
    if (__all((t.y & tmask) == gen && (t.w & tmask) == gen)) break;
    if (spin > kSpinLimit || ((spin & 63) == 63 && error_load(error))) {
      if (lane == 0) __hip_atomic_fetch_or(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      return false;
    }
  }
  if (seen) seen[0] = __builtin_amdgcn_s_memrealtime();
  // Drained: the newer poll writes the same current words.
  __builtin_amdgcn_s_waitcnt(0);
  return true;
}

// One wave: wait for the 64 activations of blocks 2n and 2n + 1 of a
// vector (tagged words src[64n, +64), staged in blk), quantise them and
// publish both blocks (one whole line) in exchange form at dst.
__device__ __forceinline__ bool publish_pair(const u64* src, u64* dst, int n, uint32_t gen, u64* blk, unsigned* error,
                             u64* seen = nullptr) {
  const int lane = threadIdx.x & (kWave - 1);
  if (!poll_words<64>(src + 64 * n, gen, blk, error, seen)) return false;
  float d;
  const uint32_t q = quantize_lane4(tag_float4(blk, 4 * (lane & 15)), &d);
  if (lane < 16) qword_store(dst + 16 * n + lane, gen, qside(lane & 7, d), q);
  return true;
}

// RMSNorm (optional, weights in LDS) + activation quantisation of act[0, K)
// into xq/xs, all threads. The square sum is the multi-kernel GEMV
// prologue's: threads t < 256 hold values 4t + 1024g, each sums its squares
// pairwise in order, then the wave trees and the four wave sums in order, so
// the norm is bit-identical to that path. The scaling and quantisation are
// quantize4's.
template <int K, bool NORM>
__device__ __forceinline__ void quantize_input(const u64* act, const float* norm_w, float eps, int* xq, float* xs,
                                               double* red) {
  const int tid = threadIdx.x;
  float inverse = 1.0f;
  bool unsettled = false;
  if constexpr (NORM) {
    static_assert(K <= 4 * kMem, "one norm group");
    if (tid < kMem) {
      const int e = 4 * tid;
      const float4 v = e < K ? tag_float4(act, e) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      double sq = 0.0;
      sq += (double)v.x * (double)v.x + (double)v.y * (double)v.y;
      sq += (double)v.z * (double)v.z + (double)v.w * (double)v.w;
      sq = wave_sum_double(sq);
      if ((tid & (kWave - 1)) == 0) red[tid / kWave] = sq;
    }
    lds_barrier_p();
    double total = 0.0;
#pragma unroll
    for (int i = 0; i < kMem / kWave; ++i) total += red[i];
    const RmsGuess g = rms_inverse_guess(total, K, eps);
    inverse = g.inverse;
    unsettled = g.unsettled;
  }
  quantize4<K, NORM>(act, norm_w, inverse, xq, xs);
  // (Rare) the reference's own square sum decides the inverse: the same
  // threads quantise the same values again with it.
  if constexpr (NORM)
    if (__builtin_expect(wave_any(unsettled), 0))
      quantize4<K, true>(act, norm_w, rms_inverse_reference(K, eps, [&](int k) { return tag_value(act, k); }), xq, xs);
}

}  // namespace

// Chunk c's part of the RMSNorm square sum of a K-value vector (K <= 1024):
// values 128c .. 128c + 127, i.e. threads 32c .. 32c + 31 of the GEMV
// prologue's tree (four values each), which hold one half (lanes 0-31 or
// 32-63) of one of its waves. The DPP steps of wave_sum_double stay inside
// rows of 16 lanes, so lanes 0 and 16 here hold exactly that wave's row sums
// of this half, and red[c] = row0 + row1 is the half the wave's tree adds
// last: the full tree is (red[2m] + red[2m + 1]) per wave m.
template <int K>
__device__ __forceinline__ void norm_chunk_partial(const u64* act, int c, double* red) {
  const int lane = threadIdx.x & (kWave - 1);
  const int e = 128 * c + 4 * lane;
  const float4 v = (lane < 32 && e < K) ? tag_float4(act, e) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  double sq = 0.0;
  sq += (double)v.x * (double)v.x + (double)v.y * (double)v.y;
  sq += (double)v.z * (double)v.z + (double)v.w * (double)v.w;
  sq += dpp_double<kDppQuadXor1>(sq);
  sq += dpp_double<kDppQuadXor2>(sq);
  sq += dpp_double<kDppHalfMirror>(sq);
  sq += dpp_double<kDppMirror>(sq);
  const double half = readlane_double(sq, 0) + readlane_double(sq, 16);
  if (lane == 0) red[c] = half;
}

// After the barrier that follows norm_chunk_partial: the inverse RMS from the
// four wave sums (each the sum of its two halves) in order, then the scaled vector quantised.
template <int K>
__device__ __forceinline__ void quantize_norm_chunks(const u64* act, const float* norm_w, float eps, const double* red,
                                                     int* xq, float* xs) {
  // The eight halves read at once (one LDS round trip), then added in order.
  double2 h[kMem / kWave];
#pragma unroll
  for (int i = 0; i < kMem / kWave; ++i) h[i] = *reinterpret_cast<const double2*>(red + 2 * i);
  __builtin_amdgcn_sched_barrier(0);
  double total = 0.0;
#pragma unroll
  for (int i = 0; i < kMem / kWave; ++i) total += h[i].x + h[i].y;
  const RmsGuess g = rms_inverse_guess(total, K, eps);
  quantize4<K, true>(act, norm_w, g.inverse, xq, xs);
  // (Rare) the reference's own square sum decides: the same threads
  // quantise the same values again.
  if (__builtin_expect(wave_any(g.unsettled), 0))
    quantize4<K, true>(act, norm_w, rms_inverse_reference(K, eps, [&](int k) { return tag_value(act, k); }), xq, xs);
}

// Shape-specialised: W hidden width, HQ/HKV query/kv heads (head size 128),
// FF feed-forward width, NBK workgroups. Workgroups [0, HQ) run attention,
// one query head each; the other NBK - HQ run the projections, each on an
// even share of the rows of every matrix. All of them run the lm_head.
template <int W, int HQ, int HKV, int FF, int NBK, bool LONG>
__global__ __launch_bounds__(kPT) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_step_kernel(PersistentArgs a) {
  constexpr int HS = 128, QW = HQ * HS, KVW = HKV * HS, QKVR = QW + 2 * KVW;
  constexpr int B1 = W / 32, Bq = QW / 32, Bf = FF / 32;
  constexpr int NB = NBK, NG = NBK - HQ;
  // Attention workgroups: w = x + 8s for kv head x < HKV and s < G, query head
  // G x + s, so that kv head x's attention runs on XCD x (workgroups are
  // dealt to the eight XCDs in turn). The q/k/v rows of kv head x (QL rows)
  // are computed by the NX other workgroups of XCD x.
  constexpr int G = HQ / HKV, QL = (G + 2) * HS, NX = NB / 8 - G;
  static_assert(NB % 8 == 0 && HKV <= 8 && G >= 1 && HQ == G * HKV, "attention placement");
  // Largest per-workgroup slices (rows) and their (row, block) pairs.
  constexpr int RQ = (QL + NX - 1) / NX, RO = (W + NG - 1) / NG, RGU = (FF / 8 + NX - 1) / NX;
  // Quantised exchanges: attention output and ffn activations.
  constexpr int QWA = qblock_words(QW), QWH = qblock_words(FF);
  static_assert(FF % 512 == 0 && RGU < 64 && QWA % 128 == 0 && QWH % 128 == 0 && QWA <= kTagWords &&
                    QWH <= kTagWords,
                "ffn block pairs per XCD, one pair per owner, whole gather chunks");
  constexpr int NPQ = RQ * B1, NPO = RO * Bq, NPG = 2 * RGU * B1, NPD = RO * Bf;
  // Projection workgroups stage their weight slices in the K/V area: q/k/v,
  // o, gate/up and down at these byte offsets, each a whole number of rounds.
  constexpr int SQ = stage_rounds(RQ, W), SO = stage_rounds(RO, QW), SG = stage_rounds(2 * RGU, W),
                SD = stage_rounds(RO, FF);
  constexpr int OQ = 0, OO = OQ + SQ * kComp * 16, OG = OO + SO * kComp * 16, OD = OG + SG * kComp * 16;
  static_assert(OD + SD * kComp * 16 <= kKvBytes, "staged slices fit the K/V area");
  constexpr int NPH = kSlotPairs * kComp, HR = NPH / B1;  // lm_head: pairs and rows per chunk
  static_assert(RQ <= 64 && 2 * RGU <= 64 && RO <= 64 && HR <= 64 && HR * B1 == NPH, "row lanes");
  static_assert(FF <= kActFloats && QW <= kActFloats && W <= 1024 && RQ * (B1 + 4) <= kProdFloats &&
                    2 * RGU * (B1 + 4) <= kProdFloats && RO * (Bq + 4) <= kProdFloats && RO * (Bf + 4) <= kProdFloats,
                "LDS sizing");
  static_assert(W % kPT == 0 && 2 * NPH * 4 <= kKvBytes, "layer-0 input and lm_head product buffers");
  static_assert(HQ < NB && QKVR == HKV * QL, "one attention workgroup per query head");
  __shared__ __attribute__((aligned(16))) u64 tag_s[kTagWords];  // gathered inputs (low 32 bits)
  __shared__ __attribute__((aligned(16))) float norm_s[1024];   // norm weights; attention: q/k norm, cos, sin
  __shared__ __attribute__((aligned(16))) int xq_s[kActFloats / 4];
  __shared__ float xs_s[kActFloats / 32];
  __shared__ float prod_s[kProdFloats];
  __shared__ float row_s[2][64];  // residual rows: [0] x, [1] a
  __shared__ __attribute__((aligned(16))) double red_s[kPT / kWave];
  __shared__ int flag_s;
  __shared__ int okw_s[kPT / kWave];  // per wave: its part of the last gather completed
  __shared__ __attribute__((aligned(16))) float cur_s[3][128];  // attention: q, k, v of the current position
  __shared__ __attribute__((aligned(16))) float tmax_s[kPT / kWave];
  __shared__ float inv_s;
  __shared__ __attribute__((aligned(16))) char kv_s[kKvBytes];  // [t][K 128 | V 128] fp16; lm_head products

  // Role index: with local_l2 the role follows the XCD the workgroup runs
  // on (the hardware deals a launch's workgroups to the eight XCDs in turn,
  // starting wherever the previous launch stopped), so that role w always
  // sits on XCD w % 8. Any other dealing leaves some role unfilled; its
  // exchanges then time out and the launch reports an error.
  const int w = a.local_l2 ? 8 * ((int)blockIdx.x >> 3) + xcc_id() % 8 : (int)blockIdx.x;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const bool is_attn = (w & 7) < HKV && (w >> 3) < G;
  const int ct = tid - kMem;  // compute-lane index (negative in the memory waves)
  const int L = a.layers;
  const int pos = *a.position;
  // A set error word (an earlier launch failed, or the host stopped the
  // step) ends every launch here until the host has restored the state; a
  // position outside the cache ends it before anything is written.
  if (error_load(a.error) != 0) return;
  // LONG: the long-cache attention (scores spread over the projection
  // workgroups, V rows streamed), for positions from long_from on; below it
  // every earlier row is held by the attention workgroups. A separate
  // instantiation, so that neither step carries the other's registers.
  constexpr bool lng = LONG;
  if (pos < 0 || pos >= a.capacity ||
      (LONG ? (pos < a.long_from || pos >= kLongPositions) : (pos >= a.long_from || pos >= kExactPositions))) {
    if (tid == 0) __hip_atomic_fetch_or(a.error, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const uint32_t gen0 = *a.epoch * (uint32_t)(5 * L + 2) + 1u;
  const int chunks = (a.vocab + HR - 1) / HR;
  auto gen = [&](int l, int p) { return gen0 + (uint32_t)(5 * l + p); };
  // The layer table is written before the launch and only read here: the
  // constant address space turns its reads into scalar loads, which do not
  // queue behind the vector loads of the weight slices.
  const __attribute__((address_space(4))) PersistentLayer* LT =
      (const __attribute__((address_space(4))) PersistentLayer*)a.layer_table;

  // Phase timeline of every workgroup: wave 0 keeps the time its last gather
  // completed and writes it, with the time the phase output was stored, just
  // before its next gather (whose wait drains both stores).
  unsigned long long* tl = a.timeline ? a.timeline + (size_t)w * kTimelineEvents : nullptr;
  u64 t_in = __builtin_amdgcn_s_memrealtime();
  u64 t_sub[3] = {0, 0, 0};  // sub-phase times, written with the next stamps
  auto sub = [&](int i) { t_sub[i] = __builtin_amdgcn_s_memrealtime(); };
  auto stamps = [&](int in_event, int out_event, int sub_event = -1, int nsub = 0) {
    if (tl && lane == 0) {
      tl[in_event] = t_in;
      tl[out_event] = __builtin_amdgcn_s_memrealtime();
      for (int i = 0; i < nsub; ++i) tl[sub_event + i] = t_sub[i];
    }
  };

  if (is_attn) {
    // ======================= attention workgroup ================================
    const int kh = w & 7, hq = G * kh + (w >> 3);
    const int n = pos + 1;
    const int nlds = pos;  // every earlier position's V row fits the K/V area (pos < kExactPositions)
    float* p_s = reinterpret_cast<float*>(tag_s + kProbOffset);  // attention probabilities after q/k/v
    const size_t kv_layer = (size_t)HKV * a.capacity * HS;
    const size_t kv_head = (size_t)kh * a.capacity * HS;
    auto kbase = [&](int l) { return a.kcache + kv_layer * l + kv_head; };
    auto vbase = [&](int l) { return a.vcache + kv_layer * l + kv_head; };
    // Layer l's rows of the earlier positions: every wave stages its share
    // of the V rows (1 KB pieces round-robin) in the K/V area, and each lane
    // pair loads the two halves of the K rows of positions (tid >> 1) and
    // (tid >> 1) + 256 into registers (lane parity h: channels 8i + 4h ..
    // 8i + 4h + 3 of every 16-byte piece i), all waited for here; readers
    // are behind the next barrier.
    const int hh = tid & 1;
    uint2 kr[2][16];
    auto stage_kv = [&](int l) {
      const char* src = reinterpret_cast<const char*>(vbase(l));
      const int bytes = nlds * 256;
      for (int c = wave * 1024; c < bytes; c += kPT / kWave * 1024)
        if (c + 16 * lane < bytes) __builtin_amdgcn_global_load_lds(src + c + 16 * lane, (lds_ptr)(kv_s + c), 16, 0, 0);
      if (pos > 0) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          if (g == 0 || pos > kPT / 2) {
            const uint2* kp = reinterpret_cast<const uint2*>(kbase(l) + (size_t)min((tid >> 1) + g * (kPT / 2), pos - 1) * HS + 4 * hh);
#pragma unroll
            for (int i = 0; i < 16; ++i) kr[g][i] = kp[2 * i];
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0);
    };
    if (a.mode == 2 && w == 0 && tid == 0) {
      int token = *a.token;
      if (token < 0 || token >= a.vocab) token = 0;
      const int hcount = *a.history_count;
      a.history[hcount] = token;
      *a.history_count = hcount + 1;
    }
    if (!lng) stage_kv(0);

    for (int l = 0; l < L; ++l) {
      const auto& Ly = LT[l];
      const int e = 16 * l + 1;  // timeline events of this layer
      u64 seen_s[2] = {0, 0};
      const u64 t_start = __builtin_amdgcn_s_memrealtime();
      if (wave == 0) {
        const int qo = hq * HS, ko = QW + kh * HS, vo = QW + KVW + kh * HS;
        const bool ok = gather_qkv(a.tqkv + qo, a.tqkv + ko, a.tqkv + vo, gen(l, 1), tag_s, a.error, [&] {
              dma(Ly.q_norm, norm_s, HS * 4);
              dma(Ly.k_norm, norm_s + HS, HS * 4);
              dma(a.rope_cos + (size_t)pos * (HS / 2), norm_s + 2 * HS, HS * 2);
              dma(a.rope_sin + (size_t)pos * (HS / 2), norm_s + 2 * HS + HS / 2, HS * 2);
            }, seen_s);
        t_in = __builtin_amdgcn_s_memrealtime();
        flag_s = ok ? 1 : 0;
        if (tl && lane == 0) {
          tl[e + 0] = seen_s[0];
          tl[e + 1] = seen_s[1];
          tl[e + 2] = t_start;
        }
      }
      lds_barrier_p();
      if (!flag_s) return;
      auto mark = [&](int event) {  // attention sub-phase stamps (events the projections use)
        if (tl && tid == 0) tl[event] = __builtin_amdgcn_s_memrealtime();
      };

      // QK-norm + RoPE, one wave per vector and channels (c, c + 64) in lane
      // c, so that the rotation partners sit in one lane: wave 0 q, wave 1 k
      // (F16-rounded, also as this position's swizzled K row), wave 2 v
      // rounded to F16. The norm's square sum is the two 64-channel wave
      // sums added low half first.
      char* kcur = reinterpret_cast<char*>(norm_s + 512);
      if (wave < 2) {
        const int c = lane, half = HS / 2;
        const float2 r = head_norm_rope<true>(tag_value(tag_s, wave * HS + c), tag_value(tag_s, wave * HS + half + c),
                                        norm_s + wave * HS, norm_s + 2 * HS, a.eps);
        const float rlo = r.x, rhi = r.y;
        if (wave == 0) {
          cur_s[0][c] = rlo;
          cur_s[0][half + c] = rhi;
        } else {
          const _Float16 klo = to_half(rlo), khi = to_half(rhi);
          cur_s[1][c] = from_half(klo);
          cur_s[1][half + c] = from_half(khi);
          const int cc = half + c;
          reinterpret_cast<_Float16*>(kcur + (((c >> 3) ^ (pos & 15)) << 4))[c & 7] = klo;
          reinterpret_cast<_Float16*>(kcur + (((cc >> 3) ^ (pos & 15)) << 4))[cc & 7] = khi;
        }
      } else if (wave == 2) {
        cur_s[2][lane] = from_half(to_half(tag_value(tag_s, 2 * HS + lane)));
        cur_s[2][kWave + lane] = from_half(to_half(tag_value(tag_s, 2 * HS + kWave + lane)));
      }
      lds_barrier_p();
      sub(0);

      // Scores, one position per lane pair: eight accumulators over channels
      // j, j+8, ..., then the pairwise tree (AttentionAvx.cs:74-160). The
      // products q*k are formed by one mixed-precision fma with a +0 addend
      // (the F16 key widened inside the instruction): round(q*k) + 0 equals
      // round(q*k) except that a -0 product becomes +0, and no accumulator
      // here is ever -0 (they start at +0 and x + y is -0 only for -0 + -0),
      // so every sum is the reference's. The even lane of a pair keeps
      // accumulators 0-3 and the odd lane 4-7, i.e. channels 8i + 4h ..
      // 8i + 4h + 3 (h = lane parity) of every 16-byte piece i, each
      // accumulator still summed over i = 0..15 in order; q's matching
      // channels sit in registers, the K row halves of earlier positions too
      // (staged with the V rows), this position's row in LDS. Each lane keeps
      // the maximum of its scores for the softmax shift.
      float m = -__builtin_inff();
      float qr[64];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float4 v = *reinterpret_cast<const float4*>(&cur_s[0][8 * i + 4 * hh]);
        qr[4 * i] = v.x;
        qr[4 * i + 1] = v.y;
        qr[4 * i + 2] = v.z;
        qr[4 * i + 3] = v.w;
      }
      // This position's row (LDS, swizzled pieces) into the registers of the
      // lane pair that scores it, so that every pair runs the same code.
      if (lng || pos < kPT / 2) {
        if (lng ? tid < 2 : (tid >> 1) == pos) {
#pragma unroll
          for (int i = 0; i < 16; ++i) kr[0][i] = *reinterpret_cast<const uint2*>(kcur + 8 * hh + ((i ^ (pos & 15)) << 4));
        }
      } else if ((tid >> 1) + kPT / 2 == pos) {
#pragma unroll
        for (int i = 0; i < 16; ++i) kr[1][i] = *reinterpret_cast<const uint2*>(kcur + 8 * hh + ((i ^ (pos & 15)) << 4));
      }
      auto score_pair = [&](const uint2* k, int t) {  // both lanes of a pair
        const float sd = pair_score(k, qr, hh, a.divisor);
        if (hh == 0) p_s[t] = sd;
        m = nan_max_p(m, sd);
      };
      if (lng) {
        // This position by lanes 0-1; the earlier ones scored by the
        // projection workgroups of this XCD, gathered by all eight waves
        // (padded to whole chunks).
        if (tid < 2) score_pair(kr[0], pos);
        u64* sc = reinterpret_cast<u64*>(kv_s + kScoreOffset);
        const bool ok = gather(a.tscore + (size_t)hq * a.score_stride, (pos + 127) & ~127, 0, nullptr, 0, 0, nullptr, 0,
                               0, gen(l, 1), sc, a.error, NoPre{}, wave, kPT / kWave);
        if (lane == 0) okw_s[wave] = ok ? 1 : 0;
        lds_barrier_p();
        int all = 1;
#pragma unroll
        for (int i = 0; i < kPT / kWave; ++i) all &= okw_s[i];
        if (!all) return;
        for (int t = tid; t < pos; t += kPT) {
          const float sd = tag_value(sc, t);
          p_s[t] = sd;
          m = nan_max_p(m, sd);
        }
      } else {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const int t = (tid >> 1) + g * (kPT / 2);
          if (t < n) score_pair(kr[g], t);
        }
      }
      // Softmax (TensorMath.SoftmaxAvx.cs:11-58).
      m = wave_max_nan(m);
      if (lane == 0) tmax_s[wave] = m;
      mark(e + 8);
      lds_barrier_p();
      sub(1);
      // The eight wave maxima in two reads, combined in order in registers.
      float mx;
      {
        const float4 m0 = *reinterpret_cast<const float4*>(&tmax_s[0]);
        const float4 m1 = *reinterpret_cast<const float4*>(&tmax_s[4]);
        mx = nan_max_p(nan_max_p(nan_max_p(m0.x, m0.y), m0.z), m0.w);
        mx = nan_max_p(nan_max_p(nan_max_p(nan_max_p(mx, m1.x), m1.y), m1.z), m1.w);
      }
      // The numerators e = exp(s - max). When every one is 0 or at least
      // 2^-17 (and at most 1), each is a multiple of 2^-40 and every partial
      // sum of them stays below 2^13: all of them are exact doubles, so any
      // order of the double additions gives the reference's sum bit for bit,
      // and the sum is formed as wave trees here. Otherwise wave 0 adds them
      // in the reference's order below.
      double dpart = 0.0;
      bool dexact = true;
      for (int t = tid; t < n; t += kPT) {
        const float ev = exp_ref(fadd(p_s[t], -mx));
        p_s[t] = ev;
        dpart += (double)ev;
        dexact = dexact && (ev == 0.0f || (ev >= 0x1p-17f && ev <= 1.0f));
      }
      static_assert(kLongPositions <= 8191, "exact double sums below 2^13");
      dpart = wave_sum_double(dpart);
      const bool wexact = __all(dexact);
      if (lane == 0) {
        red_s[wave] = dpart;
        okw_s[wave] = wexact ? 1 : 0;
      }
      lds_barrier_p();
      mark(e + 9);
      int exact = 1;
#pragma unroll
      for (int i = 0; i < kPT / kWave; ++i) exact &= okw_s[i];
      float inverse;
      if (exact) {
        // Exact in any order: a tree of the eight wave sums.
        static_assert(kPT / kWave == 8, "eight wave sums");
        const double2 r0 = *reinterpret_cast<const double2*>(red_s), r1 = *reinterpret_cast<const double2*>(red_s + 2);
        const double2 r2 = *reinterpret_cast<const double2*>(red_s + 4), r3 = *reinterpret_cast<const double2*>(red_s + 6);
        inverse = (float)(1.0 / (((r0.x + r0.y) + (r1.x + r1.y)) + ((r2.x + r2.y) + (r3.x + r3.y))));
      } else {
        const int full = n & ~7;
        if (wave == 0) {
          // Lane j < 8: p[j] + p[j+8] + ... in order, in double; the eight
          // sums' pairwise tree and the tail in order, read across the wave.
          double acc = 0.0;
          if (lane < 8) {
            int t = lane;
            for (; t + 56 < full; t += 64) {
              float v[8];
#pragma unroll
              for (int k = 0; k < 8; ++k) v[k] = p_s[t + 8 * k];
#pragma unroll
              for (int k = 0; k < 8; ++k) acc = acc + (double)v[k];
            }
            for (; t < full; t += 8) acc = acc + (double)p_s[t];
          }
          double L[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) L[j] = readlane_double(acc, j);
          double sum = ((L[0] + L[4]) + (L[1] + L[5])) + ((L[2] + L[6]) + (L[3] + L[7]));
          for (int t = full; t < n; ++t) sum = sum + (double)p_s[t];
          if (lane == 0) inv_s = (float)(1.0 / sum);
        }
        lds_barrier_p();
        inverse = inv_s;
      }
      if (lng) {
        // For the value workgroups of this XCD: the probabilities of the
        // earlier positions as tagged words over this head's scores, then,
        // once every wave's stores are written, a ready pair carrying p[pos].
        u64* pd = a.tscore + (size_t)hq * a.score_stride;
        for (int t = tid; t < n; t += kPT) {
          const float pv = fmul(p_s[t], inverse);
          p_s[t] = pv;
          if (t < pos) {
            if (a.local_l2) tag_store_local(pd + t, gen(l, 2), pv);
            else tag_store(pd + t, gen(l, 2), pv);
          }
        }
        __builtin_amdgcn_s_waitcnt(0);
      } else {
        for (int t = tid; t < n; t += kPT) p_s[t] = fmul(p_s[t], inverse);
      }
      lds_barrier_p();
      sub(2);
      if (lng) {
        if (tid < 2) {
          const float v = tid == 0 ? p_s[pos] : 0.0f;
          if (a.local_l2) tag_store_local(a.tready + 2 * hq + tid, gen(l, 2), v);
          else tag_store(a.tready + 2 * hq + tid, gen(l, 2), v);
        }
      } else if (wave < 2) {
        // Time-ordered value sums, one lane per channel (AttentionAvx.cs:173-224),
        // with the same exact mixed-precision products as the scores.
        if (wave == 0) value_chain<false>(kv_s, p_s, nlds, pos, vbase(l), cur_s);
        else value_chain<true>(kv_s, p_s, nlds, pos, vbase(l), cur_s);
      }
      mark(e + 10);
      lds_barrier_p();
      if (wave == 0) {
        static_assert(HS == 128, "four blocks per head");
        if (!lng) {
          // The head's four 32-value blocks quantised for the o projection:
          // lanes 0-31 write them (block lane / 8), two whole lines.
          float d;
          const uint32_t q = quantize_lane4(*reinterpret_cast<const float4*>(&cur_s[0][4 * (lane & 31)]), &d);
          if (lane < 32) qword_store(a.tattq + 32 * hq + lane, gen(l, 2), qside(lane & 7, d), q);
          // The output values themselves, for tracing.
          tag_store(a.tatt + hq * HS + lane, gen(l, 2), cur_s[0][lane]);
          tag_store(a.tatt + hq * HS + kWave + lane, gen(l, 2), cur_s[0][kWave + lane]);
        }
        if ((w >> 3) == 0) {
          // The first query head of the pair writes this position's K/V row
          // (four channels per lane).
          const int c = 4 * (lane & 31);
          const float* src = lane < 32 ? cur_s[1] : cur_s[2];
          _Float16* dst = (lane < 32 ? kbase(l) : vbase(l)) + (size_t)pos * HS + c;
          typedef _Float16 half4 __attribute__((ext_vector_type(4)));
          half4 h = {to_half(src[c]), to_half(src[c + 1]), to_half(src[c + 2]), to_half(src[c + 3])};
          *reinterpret_cast<half4*>(dst) = h;
        }
        if (!lng) {
          stamps(e + 3, e + 7, e + 4, 3);
        } else if (tl && lane == 0) {
          // The output's publication time (e + 7) comes from the value
          // workgroups.
          tl[e + 3] = t_in;
          for (int i = 0; i < 3; ++i) tl[e + 4 + i] = t_sub[i];
        }
      }
      // Stage the next layer's K/V while the projections run.
      // The next layer's K/V staging starts ~0.9 us later, after the
      // attention-output exchange has left (measured slightly faster).
      if (!lng && l + 1 < L) {
        __builtin_amdgcn_s_sleep(32);
        stage_kv(l + 1);
      }
    }
    // lm_head input: the last layer's output with output_norm.
    if (wave == 0) {
      const bool ok = gather1(a.tx, W, gen(L - 1, 5), tag_s, a.error, [&] { dma(a.output_norm, norm_s, W * 4); });
      flag_s = ok ? 1 : 0;
    }
    lds_barrier_p();
    if (!flag_s) return;
  } else {
    // ======================= projection workgroup ===============================
    // g: rank among the projection workgroups (attention ones below w skipped).
    int g = w;
#pragma unroll
    for (int s8 = 0; s8 < G; ++s8) g -= min(max(w - 8 * s8, 0), HKV);
    const Rows ro = split_rows<W, NG>(g);
    auto row_at = [&](int r) { return ro.r0 + r; };  // o and down rows
    // ffn rows: entries of this XCD's list (persistent_xcd_entries, 64-row
    // block pairs), the gate/up tile's storage row, and the block pair this
    // role quantises and publishes (the one whose entry 32 it computes), if
    // any.
    const int fx = w & 7;
    const XcdEntries rf = persistent_xcd_entries(fx, (w >> 3) - (fx < HKV ? G : 0), FF, HKV, G, NB);
    const size_t rf_store = 2 * (size_t)(fx * (FF / 8) + rf.r0);
    int own = -1;
    {
      const int k = (rf.r0 + rf.count - 33) >> 6;
      if (rf.count > 0 && k >= 0 && 64 * k + 32 >= rf.r0) own = fx + 8 * k;
    }
    // q/k/v: this XCD's kv head; none on XCDs past the kv heads, whose
    // (unused, clamped) slice loads then read kv head 0's rows.
    const int xk = (w & 7) < HKV ? (w & 7) : 0;
    const Rows rq = (w & 7) < HKV ? split_rows<QL, NX>((w >> 3) - G) : Rows{0, 0};
    auto qkv_row = [&](int r) {  // row r of kv head xk's list -> q/k/v row
      return r < G * HS ? G * HS * xk + r
                        : (r < (G + 1) * HS ? QW + HS * xk + (r - G * HS) : QW + KVW + HS * xk + (r - (G + 1) * HS));
    };
    auto qkv_at = [&](int r) { return qkv_row(rq.r0 + r); };
    auto gu_at = [&](int r) { return (int)rf_store + r; };
    // Compute lanes, after the q/k/v publication of layer l: the slices of
    // layer l's o, gate/up and down and of layer l + 1's q/k/v, staged while
    // the attention runs (nothing else then reads weights), so that no
    // weight stream competes with the exchanges of the later phases.
    // `parts`: 1 the o slice and the next layer's q/k/v, 2 gate/up and
    // down, 3 all.
    auto stage_window = [&](int l, int parts) __attribute__((always_inline)) {
      const auto& Ly = LT[l];
      // The piece addresses are recomputed here each layer rather than kept
      // in registers across the loop.
      int cl = ct;
      asm volatile("" : "+v"(cl));
      if (parts & 1) stage_slice<QW, SO>(kv_s + OO, Ly.wo, Ly.so, ro.count, cl, row_at);
      if (parts & 2) {
        stage_slice<W, SG>(kv_s + OG, Ly.wgu, Ly.sgu, 2 * rf.count, cl, gu_at);
        stage_slice<FF, SD>(kv_s + OD, Ly.wd, Ly.sd, ro.count, cl, row_at);
      }
      if ((parts & 1) && l + 1 < L) stage_slice<W, SQ>(kv_s + OQ, LT[l + 1].wqkv, LT[l + 1].sqkv, rq.count, cl, qkv_at);
    };
    // Layer-0 input: a host row or the embedding of the device token
    // (QwenDecoder.Embed, Gguf.cs:340-344). Its loads go first so that they
    // do not wait behind the weight slices.
    constexpr int XI = W / kPT;
    int8_t eq[XI];
    _Float16 es[XI];
    float xr[XI];
    if (a.mode == 2) {
      int token = *a.token;
      if (token < 0 || token >= a.vocab) token = 0;
#pragma unroll
      for (int k = 0; k < XI; ++k) {
        const size_t at = (size_t)token * W + tid + k * kPT;
        eq[k] = a.embed_q[at];
        es[k] = a.embed_s[at / 32];
      }
    } else {
#pragma unroll
      for (int k = 0; k < XI; ++k) xr[k] = a.x_in[tid + k * kPT];
    }
    if (ct >= 0) {
      stage_slice<W, SQ>(kv_s + OQ, LT[0].wqkv, LT[0].sqkv, rq.count, ct, qkv_at);
    } else if (wave == 0) {
      dma(LT[0].attn_norm, norm_s, W * 4);
      __builtin_amdgcn_s_waitcnt(0);
    }
#pragma unroll
    for (int k = 0; k < XI; ++k)
      tag_s[tid + k * kPT] = (u64)f2u(a.mode == 2 ? fmul((float)eq[k], (float)es[k]) : xr[k]);
    lds_barrier_p();
    // The layer-0 input's norm partials (later inputs get theirs in the gather).
    norm_chunk_partial<W>(tag_s, wave, red_s);
    lds_barrier_p();

    // The next phase's input. An input that is RMS-normalised (W values, one
    // 1 KB chunk per wave) is gathered by all eight waves (wave 0 also copies
    // the constants `pre` names), each polling its chunk whole and adding
    // that chunk's part of the square sum as soon as it is in; the quantised
    // attention output is gathered by the memory waves (a quarter each) while
    // the compute waves stage weight slices.
    auto gather_norm = [&](const u64* src, uint32_t gn, auto pre) {
      constexpr int parts = W / 128;
      bool ok = true;
      if (wave < parts) {
        ok = wave == 0 ? gather(src, W, 0, nullptr, 0, 0, nullptr, 0, 0, gn, tag_s, a.error, pre, wave, parts)
                       : gather(src, W, 0, nullptr, 0, 0, nullptr, 0, 0, gn, tag_s, a.error, NoPre{}, wave, parts);
        if (ok) norm_chunk_partial<W>(tag_s, wave, red_s);
      } else if (lane == 0) {
        red_s[wave] = 0.0;
      }
      if (lane == 0) okw_s[wave] = ok ? 1 : 0;
    };
    auto gather_q = [&](const u64* src, int count, uint32_t gn) {
      bool ok = true;
      if (ct < 0)
        ok = gather(src, count, 0, nullptr, 0, 0, nullptr, 0, 0, qtag(gn), tag_s, a.error, NoPre{}, wave, 4, NoChunk{},
                    nullptr, kQTagMask);
      if (lane == 0) okw_s[wave] = ok ? 1 : 0;
    };
    auto gathered = [&] {
      lds_barrier_p();
      t_in = __builtin_amdgcn_s_memrealtime();
      int all = 1;
#pragma unroll
      for (int i = 0; i < kPT / kWave; ++i) all &= okw_s[i];
      return all != 0;
    };
    // Long caches, after the q/k/v publication of layer l: this workgroup's
    // share [t0, t1) of the earlier positions of kv head fx, scored against
    // both of its query heads (lane pair per position, the attention
    // workgroups' arithmetic: QK-norm + RoPE of each q by one wave, then
    // pair_score), stored as tagged words; the last share also tags the
    // words up to the next multiple of 128, so that the attention
    // workgroups gather whole chunks. The K rows are requested first, into
    // the K/V area (free from P1's products until stage_window): row r of the
    // share at byte 256 r, its 16-byte piece i at slot i ^ (r & 15).
    static_assert(kLongPositions <= (kPT / 2) * NX && (kLongPositions + NX - 1) / NX * 256 <= kKvBytes,
                  "one position per lane pair, the share's K rows in the K/V area");
    auto score_earlier = [&](int l, auto rows_in) __attribute__((always_inline)) -> bool {
      const auto& Ly = LT[l];
      const int j = (w >> 3) - G;
      const int t0 = pos * j / NX, t1 = pos * (j + 1) / NX;
      const int h = tid & 1, r = tid >> 1, t = t0 + r;
      {
        const char* kb = reinterpret_cast<const char*>(a.kcache + ((size_t)l * HKV + fx) * a.capacity * HS) +
                         (size_t)t0 * 256;
        const int bytes = (t1 - t0) * 256;
        for (int c = wave * 1024; c < bytes; c += kPT / kWave * 1024) {
          const int b = c + 16 * lane, br = b >> 8;
          if (b < bytes)
            __builtin_amdgcn_global_load_lds(kb + (size_t)br * 256 + ((((b >> 4) & 15) ^ (br & 15)) << 4),
                                             (lds_ptr)(kv_s + c), 16, 0, 0);
        }
      }
      // q comes through this XCD's L2 (as to the attention workgroups), so
      // it is polled at once, two reads in flight, without the cross-XCD
      // gather delay; wave s takes query head G fx + s.
      bool ok = true;
      if (wave < G) {
        if (wave == 0) {
          dma(Ly.q_norm, norm_s, HS * 4);
          dma(a.rope_cos + (size_t)pos * (HS / 2), norm_s + 2 * HS, HS * 2);
          dma(a.rope_sin + (size_t)pos * (HS / 2), norm_s + 2 * HS + HS / 2, HS * 2);
        }
        ok = poll_words<HS>(a.tqkv + (size_t)(G * fx + wave) * HS, gen(l, 1), tag_s + wave * HS, a.error, nullptr);
      }
      if (lane == 0) okw_s[wave] = ok ? 1 : 0;
      if (!gathered()) return false;
      if (wave < G) {
        const float2 qn = head_norm_rope<true>(tag_value(tag_s, wave * HS + lane), tag_value(tag_s, wave * HS + HS / 2 + lane),
                                         norm_s, norm_s + 2 * HS, a.eps);
        cur_s[wave][lane] = qn.x;
        cur_s[wave][HS / 2 + lane] = qn.y;
      }
      __builtin_amdgcn_s_waitcnt(0);  // this wave's K rows
      lds_barrier_p();
      rows_in();
      if (t < t1) {
        uint2 kk[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) kk[i] = *reinterpret_cast<const uint2*>(kv_s + r * 256 + 8 * h + ((i ^ (r & 15)) << 4));
#pragma unroll
        for (int s = 0; s < G; ++s) {
          float qr[64];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(&cur_s[s][8 * i + 4 * h]);
            qr[4 * i] = v.x;
            qr[4 * i + 1] = v.y;
            qr[4 * i + 2] = v.z;
            qr[4 * i + 3] = v.w;
          }
          const float sd = pair_score(kk, qr, h, a.divisor);
          if (h == (s & 1)) {
            u64* dst = a.tscore + (size_t)(G * fx + s) * a.score_stride + t;
            if (a.local_l2) tag_store_local(dst, gen(l, 1), sd);
            else tag_store(dst, gen(l, 1), sd);
          }
        }
      }
      const int pad = ((pos + 127) & ~127) - pos;
      if (j == NX - 1 && pad > 0) {
        for (int i = tid; i < G * pad; i += kPT) {
          u64* dst = a.tscore + (size_t)(G * fx + i / pad) * a.score_stride + pos + i % pad;
          if (a.local_l2) tag_store_local(dst, gen(l, 1), 0.0f);
          else tag_store(dst, gen(l, 1), 0.0f);
        }
      }
      return true;
    };

    // Long caches, value workgroups: projection workgroup j < G HS / kValCh
    // of XCD fx < HKV takes query head vhq = G fx + j / (HS / kValCh) and its
    // channels [kValCh vb, +kValCh), vb = j % (HS / kValCh): the time-ordered
    // value sums over the earlier positions (AttentionAvx.cs:173-224), one
    // chain per channel, from the probabilities the attention workgroup
    // publishes, then the block quantised for the o projection. Chains of
    // different channels are independent, so spreading them over
    // workgroups keeps the reference's order. Waves: 0 adds (one add per
    // position and chain), 1 streams the V slice and 2 the probabilities
    // through a ring of kValSlots blocks at the end of the K/V area (each
    // wave waiting on its own load counter), 3 and 5-7 form the products
    // p v of the block two ahead into a three-slot product ring (at OG,
    // where gate/up and down are staged afterwards), 4 (sharing the adding
    // wave's SIMD) checks the probabilities' tags.
    constexpr int kValBlocks = HS / kValCh;
    static_assert(HS % kValCh == 0 && G * kValBlocks <= NX, "one value workgroup per (query head, block)");
    static_assert(OG + 3 * kValPSlot <= kValRing && (kLongPositions + NX - 1) / NX * 256 <= kValRing && OO <= OG,
                  "value buffers clear of the o and q/k/v slices and of the score K rows");
    // The value role's block, query head and block count, recomputed where
    // used (opaque inputs keep them out of registers across the layer loop,
    // whose register budget is full).
    struct ValRole {
      int vb, vhq, nvb;
    };
    auto val_role = [&]() __attribute__((always_inline)) {
      int ww = w, pp = pos;
      asm volatile("" : "+s"(ww), "+s"(pp));
      const int vj = (ww >> 3) - G;
      return ValRole{vj % kValBlocks, G * (ww & 7) + vj / kValBlocks, (pp + kValPos - 1) / kValPos};
    };
    using lds_char = __attribute__((address_space(3))) char;
    auto vslot = [&](int k) { return (lds_char*)(kv_s + kValRing + (k % kValSlots) * kValSlot); };
    // Wave 1: the V slice of block k (rows past pos - 1 repeat it, never used).
    auto v_issue = [&](int l, int k, const ValRole& r) __attribute__((always_inline)) {
      const char* src =
          reinterpret_cast<const char*>(a.vcache + ((size_t)l * HKV + fx) * a.capacity * HS) + 2 * kValCh * r.vb;
      lds_char* dst = vslot(k);
#pragma unroll
      for (int i = 0; i < kValVBytes / 1024; ++i) {
        const int t = min(k * kValPos + 16 * i + (lane >> 2), pos - 1);
        __builtin_amdgcn_global_load_lds(src + (size_t)t * (2 * HS) + 16 * (lane & 3), (lds_ptr)(dst + i * 1024), 16, 0, 0);
      }
    };
    auto value_prefetch = [&](int l) __attribute__((always_inline)) {  // wave 1, once the score K rows are in LDS
      const ValRole r = val_role();
      for (int k = 0; k < min(kValSlots, r.nvb); ++k) v_issue(l, k, r);
    };
    auto value_sums = [&](int l) __attribute__((always_inline)) -> bool {
      const ValRole r = val_role();
      const int vb = r.vb, vhq = r.vhq, nvb = r.nvb;
      float* vprod = reinterpret_cast<float*>(kv_s + OG);
      // Wave 2 (and 4 on a retry): the tagged probabilities of block k.
      auto p_issue = [&](int k) {
        const u64* src = a.tscore + (size_t)vhq * a.score_stride + (size_t)k * kValPos;
        if (lane < kValPos / 2) __builtin_amdgcn_global_load_lds(src + 2 * lane, (lds_ptr)(vslot(k) + kValVBytes), 16, 0, 16);
      };
      // Block k's probabilities of positions below pos all current; stale
      // ones (the ready pair came first) are read again.
      auto p_settle = [&](int k) -> bool {
        const uint32_t g = gen(l, 2);
        for (long spin = 0;; ++spin) {
          bool ok = true;
          if (lane < kValPos / 2) {
            const uint4 t = lds_read16_nodma(vslot(k) + kValVBytes + 16 * lane);
            const int t0 = k * kValPos + 2 * lane;
            ok = (t0 >= pos || t.y == g) && (t0 + 1 >= pos || t.w == g);
          }
          if (__all(ok)) return true;
          if (spin > kSpinLimit || ((spin & 63) == 63 && error_load(a.error))) {
            if (lane == 0) __hip_atomic_fetch_or(a.error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);
            return false;
          }
          p_issue(k);
          __builtin_amdgcn_s_waitcnt(0);
        }
      };
      // Products of block k: task (four positions, channel pair), 16 x 16
      // per block over the 256 lanes of waves 3, 5, 6, 7; rows 2cp and
      // 2cp + 1 of the product slot, four positions as one float4.
      // Positions from pos on get +0, so that every block adds 64 products:
      // acc + 0 is acc, since a sum from +0 is never -0.
      auto produce = [&](int k) {
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        using lds_u32 = const __attribute__((address_space(3))) uint32_t;
        using lds_u4 = const __attribute__((address_space(3))) u32x4;
        const lds_char* vsl = vslot(k);
        float* pr = vprod + (k % 3) * (kValPSlot / 4);
        // The lane's offsets are recomputed each block rather than kept in
        // registers across the loop.
        int lp = (wave == 3 ? 0 : wave - 4) * kWave + lane;
        asm volatile("" : "+v"(lp));
        const int quad = lp >> 4, cp = lp & 15;
        const u32x4 w0 = *(lds_u4*)(vsl + kValVBytes + 32 * quad);
        const u32x4 w1 = *(lds_u4*)(vsl + kValVBytes + 32 * quad + 16);
        uint32_t d[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) d[u] = *(lds_u32*)(vsl + (4 * quad + u) * (2 * kValCh) + 4 * cp);
        // All six reads in flight before the first product.
        __builtin_amdgcn_sched_barrier(0);
        const float p[4] = {u2f(w0.x), u2f(w0.z), u2f(w1.x), u2f(w1.z)};
        float lo[4], hi[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          lo[u] = fmul(from_half(__builtin_bit_cast(_Float16, (uint16_t)d[u])), p[u]);
          hi[u] = fmul(from_half(__builtin_bit_cast(_Float16, (uint16_t)(d[u] >> 16))), p[u]);
        }
        if ((k + 1) * kValPos > pos) {
          // The last block: +0 (all bits clear) from pos on, without branches.
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const uint32_t keep = 0u - (uint32_t)(k * kValPos + 4 * quad + u < pos);
            lo[u] = u2f(f2u(lo[u]) & keep);
            hi[u] = u2f(f2u(hi[u]) & keep);
          }
        }
        *reinterpret_cast<float4*>(pr + (2 * cp) * kValRow + 4 * quad) = make_float4(lo[0], lo[1], lo[2], lo[3]);
        *reinterpret_cast<float4*>(pr + (2 * cp + 1) * kValRow + 4 * quad) = make_float4(hi[0], hi[1], hi[2], hi[3]);
      };
      const bool producer = wave == 3 || wave >= 5;
      lds_barrier_nodma();  // every wave's score K rows read: the value buffers and the q/k/v slice overlap them
      if (ct >= 0) stage_window(l, 1);
      u64* rdy = tag_s + 2048;  // the ready pair: p[pos]
      u64* vcw = tag_s + 2176;  // this position's v, this block's channels
      // Blocks in the ring; the last one whose V (and probabilities) the
      // prologue waits for; the last one whose probabilities it waits for.
      const int m = min(kValSlots, nvb), first = min(2, nvb - 1), pfirst = min(3, nvb - 1);
      bool ok = true;
      if (wave == 0) {
        ok = poll_words<kValCh>(a.tqkv + QW + KVW + fx * HS + kValCh * vb, gen(l, 1), vcw, a.error, nullptr);
      } else if (wave == 1) {
        if (nvb > 0) vm_wait<4 * kValSlots>(4 * (m - 1 - first));
      } else if (wave == 2) {
        ok = poll_words<2>(a.tready + 2 * vhq, gen(l, 2), rdy, a.error, nullptr);
        if (ok && nvb > 0) {
          for (int k = 0; k < m; ++k) p_issue(k);
          vm_wait<kValSlots>(m - 1 - pfirst);
          for (int k = 0; ok && k <= first; ++k) ok = p_settle(k);
        }
      }
      if (lane == 0) okw_s[wave] = ok ? 1 : 0;
      lds_barrier_nodma();
      {
        int all = 1;
#pragma unroll
        for (int i = 0; i < kPT / kWave; ++i) all &= okw_s[i];
        if (!all) return false;
      }
      if (producer)
        for (int k = 0; k < min(2, nvb); ++k) produce(k);
      lds_barrier_nodma();
      // Block j: wave 0 adds slot j % 3 (reading the next block's groups as
      // it goes, from block j + 1's slot, formed the step before), the
      // producers form block j + 2, waves 1 and 2 issue block j + kValSlots
      // into block j's ring slot (its products were formed two steps ago)
      // and wait for blocks j + 3 (V) and j + 4 (probabilities), wave 4
      // checks block j + 3's probabilities. Each role runs its own loop, one
      // barrier a block, so that no role's registers are live in another's.
      float acc = 0.0f;
      if (wave == 0) {
        auto load_group = [&](int j, int g, float4* dst) {
          const float* row = vprod + (j % 3) * (kValPSlot / 4) + (lane & (kValCh - 1)) * kValRow + 16 * g;
#pragma unroll
          for (int k = 0; k < 4; ++k) dst[k] = *reinterpret_cast<const float4*>(row + 4 * k);
        };
        // The whole block in registers: group i of the next block is read
        // as soon as group i of this one is added (stale past the last
        // block, never added), three groups ahead of its use.
        float4 q[4][4];
        if (lane < kValCh)
#pragma unroll
          for (int g = 0; g < 4; ++g) load_group(0, g, q[g]);
        for (int j = 0; j < nvb; ++j) {
          if (lane < kValCh) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                acc = fadd(acc, q[i][k].x);
                acc = fadd(acc, q[i][k].y);
                acc = fadd(acc, q[i][k].z);
                acc = fadd(acc, q[i][k].w);
              }
              __builtin_amdgcn_sched_barrier(0);
              load_group(j + 1, i, q[i]);
            }
          }
          // Its reads in flight are of slots j and j + 1, which the
          // producers overwrite two and three steps on.
          lds_barrier_nodma<true>();
        }
      } else if (wave == 1) {
        for (int j = 0; j < nvb; ++j) {
          if (j + kValSlots < nvb) v_issue(l, j + kValSlots, r);
          if (j + 3 < nvb) vm_wait<4 * kValSlots>(4 * (min(j + kValSlots, nvb - 1) - (j + 3)));
          lds_barrier_nodma();
        }
      } else if (wave == 2) {
        // Block j + 4 in LDS by the end of step j.
        for (int j = 0; j < nvb; ++j) {
          if (j + kValSlots < nvb) p_issue(j + kValSlots);
          if (j + 4 < nvb) vm_wait<kValSlots>(min(j + kValSlots, nvb - 1) - (j + 4));
          lds_barrier_nodma();
        }
      } else if (wave == 4) {
        // Block j + 3's probabilities (in LDS since step j - 1) all current
        // before the producers read them in step j + 1; stale ones are read
        // again (with this wave's own loads).
        for (int j = 0; j < nvb; ++j) {
          if (ok && j + 3 < nvb) ok = p_settle(j + 3);
          lds_barrier_nodma();
        }
      } else {
        for (int j = 0; j < nvb; ++j) {
          if (producer && j + 2 < nvb) produce(j + 2);
          lds_barrier_nodma();
        }
      }
      if (lane == 0) okw_s[wave] = ok ? 1 : 0;
      if (wave == 0 && lane < kValCh) {
        // This position's term, then the block's values for quantisation.
        const float vc = from_half(to_half(tag_value(vcw, lane)));
        acc = fadd(acc, fmul(vc, tag_value(rdy, 0)));
        cur_s[2][lane] = acc;
      }
      lds_barrier_p();
      {
        int all = 1;
#pragma unroll
        for (int i = 0; i < kPT / kWave; ++i) all &= okw_s[i];
        if (!all) return false;
      }
      if (wave == 0) {
        float d;
        const uint32_t qw = quantize_lane4(*reinterpret_cast<const float4*>(&cur_s[2][4 * (lane & 7)]), &d);
        if (lane < 8) qword_store(a.tattq + 32 * vhq + 8 * vb + lane, gen(l, 2), qside(lane, d), qw);
        // The output values themselves, for tracing.
        if (lane < kValCh) tag_store(a.tatt + vhq * HS + kValCh * vb + lane, gen(l, 2), cur_s[2][lane]);
        // The attention's publication time, on its attention workgroup's
        // timeline (the latest of its value workgroups).
        if (a.timeline && lane == 0)
          __hip_atomic_fetch_max(a.timeline + (size_t)(fx + 8 * (vhq - G * fx)) * kTimelineEvents + 16 * l + 1 + 7,
                                 (unsigned long long)__builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      }
      return true;
    };

    // Each phase: all threads quantise (or unpack) the gathered input and
    // form the block products of the LDS slice, then wave 0 sums the rows in
    // order and publishes them, and the memory waves gather
    // the next phase's input. After the q/k/v publication (and a barrier, so
    // that the stores leave ahead of the burst) the compute waves stage the
    // slices of the rest of the layer and the next layer's q/k/v.
    // Value workgroups (long caches): the time-ordered value sums between
    // the scores and the attention-output gather.
    const int pvj = (w >> 3) - G;
    const bool valued = lng && fx < HKV && pvj >= 0 && pvj < G * kValBlocks;
    for (int l = 0; l < L; ++l) {
      const auto& Ly = LT[l];
      const auto& Nx = LT[l + 1 < L ? l + 1 : l];
      const int e = 16 * l + 1;
      // ---- P1: attn_norm + qkv ----------------------------------------------
      quantize_norm_chunks<W>(tag_s, norm_s, a.eps, red_s, xq_s, xs_s);
      if (ct >= 0 && l == 0) __builtin_amdgcn_s_waitcnt(0);  // layer 0's staged q/k/v slice
      lds_barrier_p();
      sub(0);
      lds_products<NPQ, B1>(kv_s + OQ, rq.count, xq_s, xs_s, prod_s);
      lds_barrier_p();
      sub(1);
      // This workgroup's residual rows of x (read in the o epilogue), while
      // wave 0 sums the q/k/v rows; the gather area keeps x until the
      // attention output arrives, after the next barrier.
      if (wave == 1 && lane < ro.count) row_s[0][lane] = tag_value(tag_s, row_at(lane));
      if (wave == 0) {
        if (lane < rq.count) {
          const float v = ordered_sum<B1>(prod_s, lane);
          u64* dst = a.tqkv + qkv_row(rq.r0 + lane);
          if (a.local_l2) tag_store_local(dst, gen(l, 1), v);
          else tag_store(dst, gen(l, 1), v);
        }
        stamps(e + 0, e + 2, e + 1, 1);
        if (tl && lane == 0) tl[e + 4] = t_sub[1];
      }
      lds_barrier_p();
      if (valued) {
        if (!score_earlier(l, [&] {
              if (wave == 1) value_prefetch(l);
            }))
          return;
        if (!value_sums(l)) return;
        if (ct >= 0) stage_window(l, 2);
      } else {
        if (lng && fx < HKV && !score_earlier(l, [] {})) return;
        if (ct >= 0) stage_window(l, 3);
      }
      gather_q(a.tattq, QWA, gen(l, 2));
      if (ct >= 0) __builtin_amdgcn_s_waitcnt(0);  // the staged slices are in LDS before the barrier
      if (!gathered()) return;

      // ---- P3: o projection + residual -------------------------------------
      unpack_qblocks<QW>(tag_s, xq_s, xs_s);
      lds_barrier_p();
      lds_products<NPO, Bq>(kv_s + OO, ro.count, xq_s, xs_s, prod_s);
      lds_barrier_p();
      if (wave == 0) {
        if (lane < ro.count) {
          const float v = fadd(ordered_sum<Bq>(prod_s, lane), row_s[0][lane]);
          row_s[1][lane] = v;
          tag_store(a.ta + row_at(lane), gen(l, 3), v);
        }
        stamps(e + 8, e + 9);
      }
      gather_norm(a.ta, gen(l, 3), [&] { dma(Ly.ffn_norm, norm_s, W * 4); });
      if (!gathered()) return;

      // ---- P4: ffn_norm + gate/up + SwiGLU -----------------------------------
      quantize_norm_chunks<W>(tag_s, norm_s, a.eps, red_s, xq_s, xs_s);
      lds_barrier_p();
      sub(0);
      lds_products<NPG, B1>(kv_s + OG, 2 * rf.count, xq_s, xs_s, prod_s);
      lds_barrier_p();
      if (wave == 0) {
        // Lanes [0, n) sum the gate rows, [n, 2n) the matching up rows.
        const int nr = rf.count;
        const float gs = lane < 2 * nr ? ordered_sum<B1>(prod_s, lane) : 0.0f;
        const float u = __shfl(gs, lane + nr, kWave);
        if (lane < nr) {
          const float silu = fdiv(gs, fadd(1.0f, exp_ref(-gs)));
          u64* dst = a.th + persistent_xcd_row(fx, rf.r0 + lane, 64);
          if (a.local_l2) tag_store_local(dst, gen(l, 4), fmul(silu, u));
          else tag_store(dst, gen(l, 4), fmul(silu, u));
        }
        stamps(e + 10, e + 12, e + 11, 1);
      }
      // The pair owners quantise their blocks (read through this XCD's L2)
      // and publish them; every projection workgroup gathers the quantised
      // vector.
      // The quantised ffn vector (QWH / 128 <= 8 chunks) is gathered one
      // chunk per wave, polled whole; wave 0 (the owner's publisher) and as
      // few others as possible take none.
      {
        bool ok = true;
        if (wave == 0 && own >= 0) {
          u64 seen = 0;
          ok = publish_pair(a.th, a.thq, own, gen(l, 4), tag_s + kTagWords - 64, a.error, &seen);
          if (tl && lane == 0) {
            tl[e + 6] = seen;
            tl[e + 7] = __builtin_amdgcn_s_memrealtime();
          }
        }
        if (ok)
          ok = gather(a.thq, QWH, 0, nullptr, 0, 0, nullptr, 0, 0, qtag(gen(l, 4)), tag_s, a.error, NoPre{}, wave,
                      kPT / kWave, NoChunk{}, nullptr, kQTagMask);
        if (lane == 0) okw_s[wave] = ok ? 1 : 0;
      }
      if (!gathered()) return;

      // ---- P5: down projection + residual ------------------------------------
      unpack_qblocks<FF>(tag_s, xq_s, xs_s);
      lds_barrier_p();
      sub(0);
      lds_products<NPD, Bf>(kv_s + OD, ro.count, xq_s, xs_s, prod_s);
      lds_barrier_p();
      sub(1);
      if (wave == 0) {
        if (lane < ro.count) {
          const float v = fadd(ordered_sum<Bf>(prod_s, lane), row_s[1][lane]);
          tag_store(a.tx + row_at(lane), gen(l, 5), v);
        }
        stamps(e + 13, e + 15, e + 14, 1);
        if (tl && lane == 0) tl[e + 5] = t_sub[1];
      }
      // Next layer's input with its attn_norm, or the lm_head input with output_norm.
      const float* next_norm = l + 1 < L ? Nx.attn_norm : a.output_norm;
      gather_norm(a.tx, gen(l, 5), [&] { dma(next_norm, norm_s, W * 4); });
      if (!gathered()) return;
    }
  }

  if (a.mode == 0) {
    if (w == 0 && tid == 0) {
      *a.position = pos + 1;
      *a.epoch = *a.epoch + 1;
    }
    return;
  }

  // ---- output_norm + tied lm_head + greedy (every workgroup) -----------------
  // Chunks of HR rows, round-robin over workgroups, three in flight per
  // compute lane; wave 0 sums chunk c (logits staged in LDS) while the compute
  // waves form chunk c+1.
  Slot<kSlotPairs> ha, hb, hc;
  // Chunk c goes to the workgroup with hw = c mod NB, hw = NB - 1 - w: the
  // chunks that do not divide evenly land on the projection workgroups,
  // which start the lm_head before the attention ones.
  const int hw = NB - 1 - w;
  auto load_head = [&](Slot<kSlotPairs>& sl, int c) {
    const int cc = c < chunks ? c : chunks - 1;  // clamped chunks are never summed
    const int row0 = cc * HR;
    load_slot<NPH>(sl, a.head_q + (size_t)row0 * W, a.head_s + (size_t)row0 * B1, ct, min(HR, a.vocab - row0) * B1);
  };
  if (ct >= 0) {
    load_head(ha, hw);
    load_head(hb, hw + NB);
    load_head(hc, hw + 2 * NB);
  }
  // The attention workgroups' lm_head input was gathered whole by wave 0;
  // the projection workgroups already hold its norm partials.
  if (is_attn) quantize_input<W, true>(tag_s, norm_s, a.eps, xq_s, xs_s, red_s);
  else quantize_norm_chunks<W>(tag_s, norm_s, a.eps, red_s, xq_s, xs_s);
  lds_barrier_p();
  constexpr int HP = HR * (B1 + 4);                 // one chunk's padded products
  float* hprod = reinterpret_cast<float*>(kv_s);  // two buffers of HP products
  float* hlog = hprod + 2 * HP;                   // this workgroup's logits, chunk by chunk
  u64 best = 0ull;
  bool nan_first = false;
  int parity = 0, k = 0;
  auto head_chunk = [&](const Slot<kSlotPairs>& sl, int c) {
    float* pr = hprod + parity * HP;
    const int row0 = c * HR;
    const int rows = c < chunks ? min(HR, a.vocab - row0) : 0;
    if (ct >= 0) slot_products<NPH, B1>(sl, ct, xq_s, xs_s, pr, rows * B1);
    lds_barrier_p();
    if (tid < rows) {
      const float v = ordered_sum<B1>(pr, tid);
      hlog[k * HR + tid] = v;
      const u64 key = greedy_key(v, (uint32_t)(row0 + tid));
      best = key > best ? key : best;
      if (row0 + tid == 0 && v != v) nan_first = true;  // NaN first logit: Greedy returns 0
    }
    parity ^= 1;
    ++k;
  };
  for (int c = hw; c < chunks; c += 3 * NB) {
    head_chunk(ha, c);
    if (ct >= 0) load_head(ha, c + 3 * NB);
    head_chunk(hb, c + NB);
    if (ct >= 0) load_head(hb, c + 4 * NB);
    head_chunk(hc, c + 2 * NB);
    if (ct >= 0) load_head(hc, c + 5 * NB);
  }
  if (wave == 0) {
    // Wave 0: logits out, then this workgroup's best key.
    for (int i = 0; i < k; ++i) {
      const int row0 = (hw + i * NB) * HR;
      for (int r = lane; r < HR; r += kWave)
        if (row0 + r < a.vocab) a.logits[row0 + r] = hlog[i * HR + r];
    }
    best = wave_max_u64(best);
    if (tl && lane == 0) tl[16 * L + 1] = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
      if (nan_first) best = ~0ull;  // (only the holder of chunk 0) forces token 0 below
      tag_store_bits(a.tkeys + 2 * w, gen(L, 1), (uint32_t)(best >> 32));
      tag_store_bits(a.tkeys + 2 * w + 1, gen(L, 1), (uint32_t)best);
    }
  }
  if (w != 0) return;
  // Workgroup 0: the 2 NB key words (one chunk per wave, polled whole).
  {
    constexpr int kKeyParts = 2 * NB / 128;
    static_assert(2 * NB % 128 == 0 && kKeyParts <= kPT / kWave, "one key chunk per wave");
    bool ok = true;
    if (wave < kKeyParts)
      ok = gather(a.tkeys, 2 * NB, 0, nullptr, 0, 0, nullptr, 0, 0, gen(L, 1), tag_s, a.error, NoPre{}, wave, kKeyParts);
    if (lane == 0) okw_s[wave] = ok ? 1 : 0;
    lds_barrier_p();
    if (wave != 0) return;
    int all = 1;
#pragma unroll
    for (int i = 0; i < kPT / kWave; ++i) all &= okw_s[i];
    if (!all) return;
  }
  // The workgroups' keys, a quarter of the grid per lane group, then the wave.
  u64 b = 0ull;
  bool first_nan = false;
  for (int i = lane; i < NB; i += kWave) {
    const u64 key = ((u64)(uint32_t)tag_s[2 * i] << 32) | (uint32_t)tag_s[2 * i + 1];
    if (key == ~0ull) first_nan = true;
    else b = key > b ? key : b;
  }
  b = wave_max_u64(b);
  first_nan = __any(first_nan);
  if (lane != 0) return;
  *a.token = (first_nan || b == 0ull) ? 0 : (int)greedy_index(b);
  if (tl) tl[16 * L + 2] = __builtin_amdgcn_s_memrealtime();
  *a.position = pos + 1;
  *a.epoch = *a.epoch + 1;
}

// Shapes with a persistent instantiation: Qwen3-0.6B and the reduced
// Qwen3-shaped decoder used by the quick parity runs.
bool persistent_shape_supported(int width, int heads, int kv_heads, int head_size, int ffn, int blocks) {
  if (head_size != 128 || blocks != 256) return false;
  return (width == 1024 && heads == 16 && kv_heads == 8 && ffn == 3072) ||
         (width == 512 && heads == 4 && kv_heads == 2 && ffn == 1024);
}

// Attention probabilities of every position live in the gather area after
// the q/k/v words.
int persistent_max_positions() { return kLongPositions; }
int persistent_exact_positions() { return kExactPositions; }

hipError_t launch_decode_step(const PersistentArgs& a, int blocks, hipStream_t s, bool long_cache) {
  if (!persistent_shape_supported(a.width, a.heads, a.kv_heads, a.head_size, a.ffn, blocks)) return hipErrorInvalidValue;
  // lm_head: two product buffers and this workgroup's logits share the K/V stage.
  const int rows = kSlotPairs * kComp / (a.width / 32);
  const int per_wg = ((a.vocab + rows - 1) / rows + 3 * blocks - 1) / (3 * blocks) * 3;
  if ((2 * rows * (a.width / 32 + 4) + per_wg * rows) * 4 > kKvBytes) return hipErrorInvalidValue;
  if (a.width == 1024) {
    if (long_cache) decode_step_kernel<1024, 16, 8, 3072, 256, true><<<blocks, kPT, 0, s>>>(a);
    else decode_step_kernel<1024, 16, 8, 3072, 256, false><<<blocks, kPT, 0, s>>>(a);
  } else {
    if (long_cache) decode_step_kernel<512, 4, 2, 1024, 256, true><<<blocks, kPT, 0, s>>>(a);
    else decode_step_kernel<512, 4, 2, 1024, 256, false><<<blocks, kPT, 0, s>>>(a);
  }
  return hipGetLastError();
}

// One workgroup per CU (its LDS alone exceeds half a CU's), each records
// the XCD it runs on.
__global__ __launch_bounds__(kPT) void placement_probe_kernel(int* out) {
  extern __shared__ int lds_pad[];
  if (threadIdx.x == 0) {
    lds_pad[0] = xcc_id();
    out[blockIdx.x] = lds_pad[0];
  }
}

bool persistent_xcd_round_robin(hipStream_t s) {
  constexpr int n = 256;
  int* d = nullptr;
  if (hipMalloc(&d, n * sizeof(int)) != hipSuccess) return false;
  int h[n];
  bool ok = hipMemsetAsync(d, 0xff, n * sizeof(int), s) == hipSuccess;
  if (ok) {
    placement_probe_kernel<<<n, kPT, 96 * 1024, s>>>(d);
    ok = hipGetLastError() == hipSuccess &&
         hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, s) == hipSuccess && hipStreamSynchronize(s) == hipSuccess;
  }
  (void)hipFree(d);
  // Eight XCDs dealt in turn: consecutive workgroups on consecutive XCDs.
  for (int w = 1; ok && w < n; ++w) ok = h[w] >= 0 && h[w] < 8 && h[w] == (h[w - 1] + 1) % 8;
  return ok && h[0] >= 0 && h[0] < 8;
}


int persistent_threads() { return kPT; }

// Workgroups of the persistent kernel that fit on one CU at once.
int persistent_blocks_per_cu(int width) {
  int blocks = 0;
  auto fit = [&](auto kernel) {
    int b = 0;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, kernel, kPT, 0) == hipSuccess ? b : 0;
  };
  if (width == 1024)
    blocks = std::min(fit(decode_step_kernel<1024, 16, 8, 3072, 256, false>), fit(decode_step_kernel<1024, 16, 8, 3072, 256, true>));
  else
    blocks = std::min(fit(decode_step_kernel<512, 4, 2, 1024, 256, false>), fit(decode_step_kernel<512, 4, 2, 1024, 256, true>));
  return blocks;
}

}  // namespace fah
