// Native worker threads for the step-batcher measurement (host code only,
// no HIP): the reference's callers are .NET thread-pool workers, each
// stepping its own decoder (BoundedInferencePool.cs:22-230 over
// FunAsr.cs:167-178), so the batcher is measured from native threads rather
// than from Python threads, which return through the interpreter lock one at
// a time between steps. The batcher's step entry point comes in as a
// function pointer, so this library does not link the HIP one.
#include <atomic>
#include <chrono>
#include <cstdint>
#include <thread>
#include <vector>

namespace {
using StepFn = int (*)(void* batcher, void* session, int32_t* token);
}

// Thread i calls step(batcher, sessions[i], &token) `steps` times after a
// common start and writes token k to tokens[i * steps + k]. *seconds is the
// wall time from the start to the last thread's last step. Returns 0, or the
// first nonzero code a step returned (that thread stops; the others finish).
extern "C" int fah_bench_batcher_threads(void* step_fn, void* batcher, void* const* sessions, int count, int steps,
                                         int32_t* tokens, double* seconds) {
  if (!step_fn || !batcher || !sessions || !tokens || !seconds || count <= 0 || steps < 0) return -1;
  const StepFn step = reinterpret_cast<StepFn>(step_fn);
  std::atomic<int> ready{0}, error{0};
  std::atomic<bool> go{false};
  std::vector<std::chrono::steady_clock::time_point> ends(count);
  std::vector<std::thread> threads;
  threads.reserve(count);
  for (int i = 0; i < count; ++i) {
    threads.emplace_back([&, i] {
      ready.fetch_add(1);
      while (!go.load(std::memory_order_acquire)) std::this_thread::yield();
      for (int k = 0; k < steps; ++k) {
        int32_t t = -1;
        const int rc = step(batcher, sessions[i], &t);
        if (rc != 0) {
          int expected = 0;
          error.compare_exchange_strong(expected, rc);
          break;
        }
        tokens[(size_t)i * steps + k] = t;
      }
      ends[i] = std::chrono::steady_clock::now();
    });
  }
  while (ready.load() < count) std::this_thread::yield();
  const auto start = std::chrono::steady_clock::now();
  go.store(true, std::memory_order_release);
  for (auto& t : threads) t.join();
  auto last = start;
  for (const auto& e : ends) last = e > last ? e : last;
  *seconds = std::chrono::duration<double>(last - start).count();
  return error.load();
}
