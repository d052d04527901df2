// Host-side input compaction for the transfer of a flat-layout batch to the GPU.
//
// The reference moves its flat layout with `.to(device, non_blocking=True)` of int64 tensors
// (online_best/infer.py:742-779). Ids narrowed to int32 halve those bytes. The narrowing
// saturates to [INT32_MIN, INT32_MAX]: every table has fewer than 2^31 rows, so
// clamp(saturate(v), 0, rows-1) == clamp(v, 0, rows-1) for every int64 id v, and the pooled
// result is the int64 result bit for bit. It is written into the caller's (pinned) staging
// buffer in one pass, split over a persistent pool of worker threads: creating threads per call
// costs more than the pass itself (a batch of ~1M ids takes well under 100 us on 16 threads).
// cti_ebag_stage_copy does the whole host side of one batch: its parts (ids, offsets, ...) are
// converted into one contiguous pinned region, which one hipMemcpyAsync sends to the device.
#include <stdint.h>

#include <pthread.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include "ebag_internal.h"

namespace cti {
namespace {

// Clones for AVX-512 / AVX2 hosts (vector 64-bit compares; AVX-512 narrows with saturation in
// one instruction), chosen when the library loads; the baseline x86-64 build has no 64-bit
// vector compare and runs the loop scalar.
__attribute__((target_clones("avx512f", "avx2", "default")))
void narrow_range(const int64_t* src, int32_t* dst, int64_t n) {
  constexpr int64_t lo = INT32_MIN, hi = INT32_MAX;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t v = src[i];
    dst[i] = static_cast<int32_t>(v < lo ? lo : (v > hi ? hi : v));
  }
}

__attribute__((target_clones("avx512f", "avx2", "default")))
void widen_range(const int32_t* src, int64_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = src[i];
}

// Elements [b, e) of one part: src of type st (CTI_EBAG_I64 / I32) into dst of type dt.
void convert_range(const void* src, int st, void* dst, int dt, int64_t b, int64_t e) {
  if (b >= e) return;
  const int64_t n = e - b;
  if (st == CTI_EBAG_I64 && dt == CTI_EBAG_I32) {
    narrow_range(static_cast<const int64_t*>(src) + b, static_cast<int32_t*>(dst) + b, n);
  } else if (st == CTI_EBAG_I32 && dt == CTI_EBAG_I64) {
    widen_range(static_cast<const int32_t*>(src) + b, static_cast<int64_t*>(dst) + b, n);
  } else {
    const size_t w = st == CTI_EBAG_I64 ? 8 : 4;
    memcpy(static_cast<char*>(dst) + b * w, static_cast<const char*>(src) + b * w, static_cast<size_t>(n) * w);
  }
}

// One job of the pool: either a conversion of up to kMaxParts arrays, each cut into chunks of at
// most `chunk` elements, or `tasks` calls of task(ctx, i).
constexpr int kMaxParts = 8;
struct Job {
  void (*task)(const void* ctx, int64_t i) = nullptr;
  const void* ctx = nullptr;
  int64_t tasks = 0;
  int parts = 0;
  const void* src[kMaxParts];
  int st[kMaxParts];
  void* dst[kMaxParts];
  int dt = CTI_EBAG_I32;
  int64_t count[kMaxParts];
  int64_t first_chunk[kMaxParts + 1];  // prefix of per-part chunk counts
  int64_t chunk = 1;

  int64_t chunks() const { return task ? tasks : first_chunk[parts]; }
  void run_chunk(int64_t c) const {
    if (task) {
      task(ctx, c);
      return;
    }
    int p = 0;
    while (c >= first_chunk[p + 1]) ++p;
    const int64_t b = (c - first_chunk[p]) * chunk;
    convert_range(src[p], st[p], dst[p], dt, b, std::min(count[p], b + chunk));
  }
};

// Workers sleep on a condition variable between jobs (after a short spin, so the several jobs
// of one batch find them awake); a job's chunks are claimed with an atomic counter by the
// workers and the calling thread. Callers are serialised. A job's parameters change only while
// no worker is inside work() (busy_ == 0, checked under m_), and run() returns only when every
// chunk is done and no worker is busy, so a worker that wakes late finds either the job it was
// woken for (with nothing left to claim) or the next one, never a mix. The pool is never
// destroyed: its threads end with the process; a forked child starts a new pool.
class Pool {
 public:
  static Pool& get() {
    static std::once_flag registered;
    std::call_once(registered, [] { pthread_atfork(nullptr, nullptr, &Pool::forget_in_child); });
    Pool* pool = instance().load(std::memory_order_acquire);
    if (!pool) {
      std::lock_guard<std::mutex> lk(create_mutex());
      pool = instance().load(std::memory_order_relaxed);
      if (!pool) {
        pool = new Pool();
        instance().store(pool, std::memory_order_release);
      }
    }
    return *pool;
  }

  void run(const Job& job, int workers) {
    std::lock_guard<std::mutex> serial(call_m_);
    grow(workers);
    {
      std::unique_lock<std::mutex> lk(m_);
      idle_cv_.wait(lk, [&] { return busy_ == 0; });
      job_ = job;
      next_.store(0, std::memory_order_relaxed);
      remaining_ = job.chunks();
      active_ = workers;
      ++gen_;
      gen_seen_.store(gen_, std::memory_order_release);
      ++busy_;  // the calling thread
    }
    cv_.notify_all();
    const int64_t done = work();
    std::unique_lock<std::mutex> lk(m_);
    remaining_ -= done;
    --busy_;
    idle_cv_.wait(lk, [&] { return remaining_ == 0 && busy_ == 0; });
  }

 private:
  static std::atomic<Pool*>& instance() {
    static std::atomic<Pool*> p{nullptr};
    return p;
  }
  static std::mutex& create_mutex() {
    static std::mutex m;
    return m;
  }
  // A forked child has none of the parent's worker threads and may inherit a mutex locked by a
  // job that was running in another thread: it starts a pool of its own (the old one is leaked).
  static void forget_in_child() {
    instance().store(nullptr, std::memory_order_relaxed);
    new (&create_mutex()) std::mutex();
  }

  // Claim chunks until none are left; returns how many this thread completed.
  int64_t work() {
    int64_t done = 0;
    const int64_t total = job_.chunks();
    for (;;) {
      const int64_t c = next_.fetch_add(1, std::memory_order_relaxed);
      if (c >= total) break;
      job_.run_chunk(c);
      ++done;
    }
    return done;
  }

  void grow(int workers) {
    while (static_cast<int>(threads_.size()) < workers) {
      const int id = static_cast<int>(threads_.size());
      threads_.emplace_back([this, id] { loop(id); });
    }
  }

  void loop(int id) {
    uint64_t seen = 0;
    for (;;) {
      for (int i = 0; i < kSpin && gen_seen_.load(std::memory_order_acquire) == seen; ++i) std::this_thread::yield();
      {
        std::unique_lock<std::mutex> lk(m_);
        cv_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
        if (id >= active_) continue;  // this job uses fewer workers
        ++busy_;
      }
      const int64_t done = work();
      {
        std::lock_guard<std::mutex> lk(m_);
        remaining_ -= done;
        --busy_;
      }
      idle_cv_.notify_all();
    }
  }

  static constexpr int kSpin = 2000;  // yields before sleeping (tens of microseconds)
  std::mutex call_m_;
  std::mutex m_;
  std::condition_variable cv_, idle_cv_;
  std::vector<std::thread> threads_;
  Job job_;
  int64_t remaining_ = 0;
  std::atomic<int64_t> next_{0};
  std::atomic<uint64_t> gen_seen_{0};
  int active_ = 0, busy_ = 0;
  uint64_t gen_ = 0;
};

constexpr int64_t kMinPerThread = 1 << 15;  // elements below which waking workers costs more than it saves

// Run a job on min(num_threads, elements / kMinPerThread) threads (the caller included).
void run_job(Job& job, int64_t elements, int num_threads) {
  const int64_t t = std::min<int64_t>(num_threads, std::max<int64_t>(1, elements / kMinPerThread));
  // 4 chunks per thread even out threads that start late
  job.chunk = std::max<int64_t>(1, (elements + 4 * t - 1) / (4 * t));
  job.first_chunk[0] = 0;
  for (int p = 0; p < job.parts; ++p) job.first_chunk[p + 1] = job.first_chunk[p] + (job.count[p] + job.chunk - 1) / job.chunk;
  if (t == 1) {
    for (int64_t c = 0; c < job.chunks(); ++c) job.run_chunk(c);
    return;
  }
  Pool::get().run(job, static_cast<int>(t - 1));
}

// ---------------------------------------------------------------------------------------------
// Dispatch order made on the host (the layout is the one the pooling launch's own order pass
// writes): each XCD's contiguous range of tile positions, in chunks of kOrderChunk tiles, holds
// the chunk's tiles by rows per bag, most first (a stable counting sort). Chunks are independent
// tasks for the pool.
struct OrderJob {
  const void* offsets;
  int32_t offset_type;
  int64_t stride;     // offsets between consecutive fields' first bags (B or B + 1)
  int64_t batch;
  int64_t per_field;  // tiles per field
  int64_t n;          // tiles
  int nb_log2;        // bags per tile (a power of two)
  int32_t* order;
  int64_t chunks_per_range;
};

template <typename OT>
void order_chunk_typed(const OrderJob& j, int64_t lo, int64_t c0, int64_t m) {
  const OT* const off = static_cast<const OT*>(j.offsets);
  const int64_t nb = int64_t{1} << j.nb_log2;
  unsigned char bucket[kOrderChunk];
  // four interleaved counts, so that runs of tiles in one bucket do not form one chain of
  // dependent increments
  int32_t count[4][kOrderBuckets] = {};
  // tiles of a chunk are consecutive: take them field by field, each field's run of tiles a plain
  // strided walk over its offsets
  int64_t fi = (lo + c0) / j.per_field, local = lo + c0 - fi * j.per_field;
  for (int64_t k = 0; k < m;) {
    const OT* const f_off = off + fi * j.stride;
    const int64_t run = std::min<int64_t>(m - k, j.per_field - local);
    // every tile of the run but the field's last spans nb full bags
    const int64_t full = local + run < j.per_field ? run : run - 1;
    for (int64_t t = 0; t < full; ++t) {
      const int64_t b0 = (local + t) << j.nb_log2;
      const int64_t rows = static_cast<int64_t>(f_off[b0 + nb]) - static_cast<int64_t>(f_off[b0]);
      int64_t per_bag = rows > 0 ? rows >> j.nb_log2 : 0;
      per_bag = per_bag > kOrderBuckets - 1 ? kOrderBuckets - 1 : per_bag;
      bucket[k + t] = static_cast<unsigned char>(kOrderBuckets - 1 - per_bag);
    }
    if (full < run) {  // the field's last tile ends at the batch's last bag
      const int64_t b0 = (local + full) << j.nb_log2;
      const int64_t rows = static_cast<int64_t>(f_off[j.batch]) - static_cast<int64_t>(f_off[b0]);
      int64_t per_bag = rows > 0 ? rows >> j.nb_log2 : 0;
      per_bag = per_bag > kOrderBuckets - 1 ? kOrderBuckets - 1 : per_bag;
      bucket[k + full] = static_cast<unsigned char>(kOrderBuckets - 1 - per_bag);
    }
    k += run;
    local = 0;
    ++fi;
  }
  for (int64_t k = 0; k < m; ++k) ++count[k & 3][bucket[k]];
  int32_t next[kOrderBuckets];
  int32_t total = 0;
  for (int b = 0; b < kOrderBuckets; ++b) {
    next[b] = total;
    total += count[0][b] + count[1][b] + count[2][b] + count[3][b];
  }
  int32_t* const dst = j.order + kOrderHeader + lo + c0;
  const int32_t t0 = static_cast<int32_t>(lo + c0);
  for (int64_t k = 0; k < m; ++k) dst[next[bucket[k]]++] = t0 + static_cast<int32_t>(k);
}

void order_chunk(const void* ctx, int64_t task) {
  const OrderJob& j = *static_cast<const OrderJob*>(ctx);
  const int64_t x = task / j.chunks_per_range, c0 = (task % j.chunks_per_range) * kOrderChunk;
  const int64_t q = j.n >> 3, r = j.n & 7;
  const int64_t lo = x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q;
  const int64_t cnt = q + (x < r ? 1 : 0);
  if (c0 >= cnt) return;
  const int64_t m = cnt - c0 < kOrderChunk ? cnt - c0 : kOrderChunk;
  if (j.offset_type == CTI_EBAG_I32) order_chunk_typed<int32_t>(j, lo, c0, m);
  else order_chunk_typed<int64_t>(j, lo, c0, m);
}

}  // namespace
}  // namespace cti

using namespace cti;

extern "C" int cti_ebag_order_host(const void* offsets, int32_t offset_type, int64_t offsets_stride,
                                   int64_t batch_size, int32_t num_slots, int32_t table_dtype, int32_t emb_dim,
                                   int32_t* order, int64_t order_bytes, int32_t num_threads) {
  clear_error();
  if (offset_type != CTI_EBAG_I64 && offset_type != CTI_EBAG_I32)
    return set_error(CTI_EBAG_EINVAL, "unknown offset type code %d", offset_type);
  if (dtype_bytes(table_dtype) == 0) return set_error(CTI_EBAG_EINVAL, "unknown table dtype code %d", table_dtype);
  if (batch_size < 1 || num_slots < 1 || emb_dim < 1)
    return set_error(CTI_EBAG_EINVAL, "batch_size, num_slots and emb_dim must be >= 1");
  if (offsets_stride != batch_size && offsets_stride != batch_size + 1)
    return set_error(CTI_EBAG_EINVAL, "offsets_stride must be batch_size (global offsets) or batch_size + 1 (slot "
                     "row offsets), got %lld", (long long)offsets_stride);
  if (!offsets || !order) return set_error(CTI_EBAG_EINVAL, "NULL host pointer among offsets/order");
  if (num_threads < 1 || num_threads > 256)
    return set_error(CTI_EBAG_EINVAL, "num_threads must be in [1, 256] (got %d)", num_threads);
  if (num_slots > kOrderMaxFields)
    return set_error(CTI_EBAG_EUNSUPPORTED, "a dispatch order covers at most %d slots (got %d)", kOrderMaxFields,
                     num_slots);
  const int nb = order_bags_per_tile(table_dtype, emb_dim);
  if (nb == 0)
    return set_error(CTI_EBAG_EUNSUPPORTED, "rows of %d elements of this type take the element-wise kernel, which "
                     "follows no order", emb_dim);
  if ((nb & (nb - 1)) != 0)  // every tiled shape holds 2 x (a power of two) bags; the walk below shifts by it
    return set_error(CTI_EBAG_EUNSUPPORTED, "internal: %d bags per tile is not a power of two", nb);
  OrderJob oj;
  oj.offsets = offsets;
  oj.offset_type = offset_type;
  oj.stride = offsets_stride;
  oj.batch = batch_size;
  oj.per_field = (batch_size + nb - 1) / nb;
  oj.n = oj.per_field * num_slots;
  oj.nb_log2 = __builtin_ctz(static_cast<unsigned>(nb));
  oj.order = order;
  if (oj.n > INT32_MAX / 2)
    return set_error(CTI_EBAG_EUNSUPPORTED, "batch of %lld samples has too many tiles", (long long)batch_size);
  if (order_bytes < (kOrderHeader + oj.n) * 4)
    return set_error(CTI_EBAG_EINVAL, "order buffer of %lld bytes; this batch needs %lld", (long long)order_bytes,
                     (long long)((kOrderHeader + oj.n) * 4));
  oj.chunks_per_range = ((oj.n + 7) / 8 + kOrderChunk - 1) / kOrderChunk;
  Job job;
  job.task = order_chunk;
  job.ctx = &oj;
  job.tasks = 8 * oj.chunks_per_range;
  // one task per chunk of an XCD range; below ~2k tiles one thread is faster than waking others
  const int threads = static_cast<int>(std::min<int64_t>(num_threads, std::max<int64_t>(1, oj.n / 2048)));
  if (threads <= 1) {
    for (int64_t t = 0; t < job.tasks; ++t) order_chunk(&oj, t);
  } else {
    Pool::get().run(job, std::min(threads, static_cast<int>(job.tasks)) - 1);
  }
  order[0] = static_cast<int32_t>(oj.n);
  order[1] = kOrderMagic;
  order[2] = 0;
  order[3] = 0;
  return CTI_EBAG_OK;
}

extern "C" int cti_ebag_narrow_ids(const int64_t* src, int64_t n, int32_t* dst, int32_t num_threads) {
  clear_error();
  if (n < 0) return set_error(CTI_EBAG_EINVAL, "n must be >= 0 (got %lld)", (long long)n);
  if (n == 0) return CTI_EBAG_OK;
  if (!src || !dst) return set_error(CTI_EBAG_EINVAL, "NULL host pointer among src/dst");
  if (num_threads < 1 || num_threads > 256)
    return set_error(CTI_EBAG_EINVAL, "num_threads must be in [1, 256] (got %d)", num_threads);
  Job job;
  job.parts = 1;
  job.src[0] = src;
  job.st[0] = CTI_EBAG_I64;
  job.dst[0] = dst;
  job.dt = CTI_EBAG_I32;
  job.count[0] = n;
  run_job(job, n, num_threads);
  return CTI_EBAG_OK;
}

extern "C" int64_t cti_ebag_stage_offset(const int64_t* counts, int32_t n_parts, int32_t dst_type, int32_t part) {
  if (!counts || n_parts < 0 || part < 0 || part > n_parts || (dst_type != CTI_EBAG_I64 && dst_type != CTI_EBAG_I32))
    return -1;
  const int64_t w = dst_type == CTI_EBAG_I64 ? 8 : 4;
  int64_t off = 0;
  for (int p = 0; p < part; ++p) {
    if (counts[p] < 0) return -1;
    off += (counts[p] * w + 255) / 256 * 256;
  }
  return off;
}

extern "C" int cti_ebag_stage_copy(const void* const* src, const int32_t* src_type, const int64_t* counts,
                                   int32_t n_parts, int32_t dst_type, void* pinned, int64_t pinned_bytes,
                                   void* device_dst, int32_t num_threads, void* stream) {
  clear_error();
  if (n_parts < 0 || n_parts > kMaxParts)
    return set_error(CTI_EBAG_EINVAL, "n_parts must be in [0, %d] (got %d)", kMaxParts, n_parts);
  if (dst_type != CTI_EBAG_I64 && dst_type != CTI_EBAG_I32)
    return set_error(CTI_EBAG_EINVAL, "unknown destination type code %d", dst_type);
  if (num_threads < 1 || num_threads > 256)
    return set_error(CTI_EBAG_EINVAL, "num_threads must be in [1, 256] (got %d)", num_threads);
  if (n_parts > 0 && (!src || !src_type || !counts)) return set_error(CTI_EBAG_EINVAL, "NULL host array argument");
  Job job;
  job.parts = n_parts;
  job.dt = dst_type;
  int64_t elements = 0;
  for (int p = 0; p < n_parts; ++p) {
    if (counts[p] < 0) return set_error(CTI_EBAG_EINVAL, "part %d: negative count", p);
    if (src_type[p] != CTI_EBAG_I64 && src_type[p] != CTI_EBAG_I32)
      return set_error(CTI_EBAG_EINVAL, "part %d: unknown source type code %d", p, src_type[p]);
    if (counts[p] > 0 && !src[p]) return set_error(CTI_EBAG_EINVAL, "part %d: NULL source", p);
    job.src[p] = src[p];
    job.st[p] = src_type[p];
    job.count[p] = counts[p];
    elements += counts[p];
  }
  const int64_t total = cti_ebag_stage_offset(counts, n_parts, dst_type, n_parts);
  if (total > pinned_bytes)
    return set_error(CTI_EBAG_EINVAL, "the parts need %lld staging bytes, the buffer has %lld", (long long)total,
                     (long long)pinned_bytes);
  if (total == 0) return CTI_EBAG_OK;
  if (!pinned || !device_dst) return set_error(CTI_EBAG_EINVAL, "NULL pinned or device buffer");
  for (int p = 0; p < n_parts; ++p)
    job.dst[p] = static_cast<char*>(pinned) + cti_ebag_stage_offset(counts, n_parts, dst_type, p);
  run_job(job, elements, num_threads);
  const hipError_t e = hipMemcpyAsync(device_dst, pinned, static_cast<size_t>(total), hipMemcpyHostToDevice,
                                      static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return set_error(CTI_EBAG_EHIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
  return CTI_EBAG_OK;
}
