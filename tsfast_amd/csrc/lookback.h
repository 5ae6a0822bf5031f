// Shared protocol of the single-pass look-back scans (diag.hip, allpole.hip): published 8-byte
// words with a per-word ready marker, the in-order tile counter and the per-call reset kernel.
// Included inside each file's anonymous namespace (after common.h and `using namespace tsf`).
#pragma once

// Published words start as kUnset, a signalling NaN: arithmetic results and float -> double
// conversions are never signalling NaNs, so a word that differs from kUnset has been written.
// Each 8-byte word is stored and polled with agent-scope atomics (coherent across the L2s of
// the XCDs) and validated on its own, so no fence has to order data against a flag.
constexpr uint64_t kUnset = 0x7FF00000DEADBEEFull;
// Polls without progress before a look-back gives up and yields NaN (about a second): every
// wait ends even if an invariant below were broken, and the NaN shows in the outputs. The bound
// a scan uses is the library's current limit (tsfast_hip_set_lookback_spin_limit, default
// kSpinMax), passed to its kernels at enqueue (LbCfg below).
constexpr uint32_t kSpinMax = 1u << 20;

TSF_DEV void put_word(double* p, double x) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), static_cast<uint64_t>(__double_as_longlong(x)), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
TSF_DEV bool get_word(const double* p, double& x) {
  const uint64_t b = __hip_atomic_load(const_cast<uint64_t*>(reinterpret_cast<const uint64_t*>(p)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  x = __longlong_as_double(static_cast<long long>(b));
  return b != kUnset;
}
TSF_DEV void put(double* p, double x) { put_word(p, x); }
TSF_DEV void put(double2* p, double2 x) {
  put_word(&p->x, x.x);
  put_word(&p->y, x.y);
}
TSF_DEV bool get(const double* p, double& x) { return get_word(p, x); }
TSF_DEV bool get(const double2* p, double2& x) {
  const bool a = get_word(&p->x, x.x);
  const bool b = get_word(&p->y, x.y);
  return a && b;
}
template <typename W>
TSF_DEV W quiet_nan();
template <>
TSF_DEV double quiet_nan<double>() {
  return __longlong_as_double(0x7FF8000000000000ll);
}
template <>
TSF_DEV double2 quiet_nan<double2>() {
  return make_double2(quiet_nan<double>(), quiet_nan<double>());
}

// What a tile publishes, in scan order j = 0, 1, ... (the last tile publishes nothing):
//  * spacing 0 (the fast mode): every tile but the first publishes its aggregate (agg) and every
//    tile the state leaving it (inc). A look-back stops at the nearest published inc, so the maps
//    it composes depend on which tiles have finished: results agree run to run to fp64 rounding.
//  * spacing s > 0 (deterministic mode, the library's default): an anchor tile (j % s == 0)
//    publishes only its inc, every other tile only its agg. A look-back then composes exactly the
//    aggregates of tiles a+1 .. j-1 onto inc_a (a = the last anchor before j) in the same order on
//    every run, so the entering states and everything computed from them are bitwise
//    reproducible; a tile waits for its anchor's look-back, which costs time when the anchor runs
//    concurrently. s must not exceed the slots a look-back examines.
TSF_DEV bool lb_pub_agg(int64_t j, int spacing) { return spacing == 0 ? j > 0 : j % spacing != 0; }
TSF_DEV bool lb_pub_inc(int64_t j, int spacing) { return spacing == 0 || j % spacing == 0; }

// What a launch tells its look-back kernel: the anchor spacing (0 unless the deterministic mode
// is on) and the wait bound, the rounds without progress after which a look-back gives up
// (tsfast_hip_set_lookback_spin_limit). Both are kernel arguments: a bound read from memory would
// make each round's comparison wait for every outstanding memory operation of the wave,
// the look-back's own published stores included.
struct LbCfg {
  int spacing;
  uint32_t spin_max;
};
TSF_DEV bool lb_pub_agg(int64_t j, LbCfg c) { return lb_pub_agg(j, c.spacing); }
TSF_DEV bool lb_pub_inc(int64_t j, LbCfg c) { return lb_pub_inc(j, c.spacing); }
// Deterministic-mode anchor spacing of the look-backs whose window moves. Spacing 1 (every tile an
// anchor: a chained scan, each tile waiting for its predecessor's state) is cheapest when many
// lane groups run side by side, so each group's chain is short; few, long chains want the
// longer spans.
constexpr int kAnchorSpacing = 8;
inline int anchor_spacing_for_groups(int64_t groups) { return groups >= 128 ? 1 : kAnchorSpacing; }

// Give-up flag: the word kErrWord words after the tile counter (inside the kCounterBytes header
// of the workspace, byte offset 64) is set to 1 by any look-back that gives up after kSpinMax
// rounds without progress, whose lanes then carry NaN; lookback_reset clears it before every
// scan, so after a scan it tells a give-up apart from NaNs that came with the inputs.
// A give-up also writes the scan's call number (kEpochWord, nonzero) into the library's alarm
// word, a 4-byte word in mapped host memory whose device address the reset kernel writes into the
// header at word kAlarmWord (8 bytes; zero when the library has no alarm word), so that the host
// sees it without a device synchronisation and reports each failing call once
// (tsfast_hip_lookback_gave_up).
constexpr int kErrWord = 16;
constexpr int kAlarmWord = 18;  // 8-byte aligned: byte offset 72
constexpr int kEpochWord = 20;
TSF_DEV void lb_gave_up(unsigned* counter) {
  __hip_atomic_store(counter + kErrWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned* alarm = reinterpret_cast<unsigned*>(*reinterpret_cast<const uint64_t*>(counter + kAlarmWord));
  if (alarm) __hip_atomic_store(alarm, counter[kEpochWord], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

TSF_DEV unsigned take_tile(unsigned* counter) {
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Resets the look-back words to kUnset and the tile counter to zero before every scan (a
// kernel rather than a memset node, so that a captured graph replays it reliably).
// A reset as a job of `blocks` workgroups: lookback_reset runs it alone, and a kernel launched
// right before a scan (the transfer-matrix kernels) can run it in extra workgroups of its own
// launch, which saves a launch per scan call.
struct ResetJob {
  uint64_t* words;
  int64_t n;
  unsigned* counter;
  unsigned* alarm;
  uint32_t epoch;
  unsigned blocks;
};
TSF_DEV void run_reset(const ResetJob& r, unsigned block) {
  const int64_t stride = (int64_t)r.blocks * blockDim.x;
  for (int64_t i = block * (int64_t)blockDim.x + threadIdx.x; i < r.n; i += stride) r.words[i] = kUnset;
  if (block == 0 && threadIdx.x == 0) {
    r.counter[0] = 0u;
    r.counter[kErrWord] = 0u;
    r.counter[kEpochWord] = r.epoch;
    *reinterpret_cast<uint64_t*>(r.counter + kAlarmWord) = reinterpret_cast<uint64_t>(r.alarm);
  }
}
__global__ void __launch_bounds__(256) lookback_reset(ResetJob r) { run_reset(r, blockIdx.x); }


// Host side. A workspace starts with the tile counter (kCounterBytes), followed by the published
// words that lookback_reset_launch marks unset.
constexpr int64_t kCounterBytes = 256;

// Workgroups that stay resident at once (persistent grid size), per kernel and block size.
template <typename F>
int64_t resident_wgs(F kern, int threads, int* cache) {
  int& c = cache[threads / 64];
  if (c == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, 0) != hipSuccess || n < 1) n = 1;
    c = n;
  }
  return (int64_t)c * device_cus();
}

// The look-back arguments of a launch: anchor spacing 0 unless the deterministic mode is on
// (tsfast_hip_set_deterministic), then `deterministic_spacing`; the library's current wait bound.
inline LbCfg lb_spacing_for(int deterministic_spacing) {
  return LbCfg{tsf_deterministic() ? deterministic_spacing : 0, tsf_lookback_spin_limit()};
}

// The reset of a scan call's workspace (the tile counter, then `words` published words) as a job
// of workgroups of `threads` threads (at most 2^19 threads in all, striding over the words).
inline ResetJob reset_job(char* ws, int64_t words, int threads) {
  int64_t blocks = (words + threads - 1) / threads;
  const int64_t cap = (int64_t)(1 << 19) / threads;
  if (blocks < 1) blocks = 1;
  if (blocks > cap) blocks = cap;
  return ResetJob{reinterpret_cast<uint64_t*>(ws + kCounterBytes), words, reinterpret_cast<unsigned*>(ws),
                  tsf_lookback_alarm(), tsf_next_epoch(), (unsigned)blocks};
}
void lookback_reset_launch(char* ws, int64_t words, hipStream_t s) {
  const ResetJob r = reset_job(ws, words, 256);
  hipLaunchKernelGGL(lookback_reset, dim3(r.blocks), dim3(256), 0, s, r);
}
