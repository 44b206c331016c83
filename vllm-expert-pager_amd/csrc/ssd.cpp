// Host side of the SSD tier: answers the GPU's read requests from the pinned
// request ring.
//
// Protocol (layout and rules are the reference's, store.py:25-30, 83-251,
// gather.py:197-277):
//   req  = [re-publishes, give-ups] + `ring` slots of
//          [seq, layer, expert[block], row[block]]        (int64, pinned)
//   done = the last seq answered                          (int64, pinned)
// The GPU fills a slot and publishes its seq with a release store. Requests
// are answered in seq order: done = seq is release-stored once every listed
// record of that request (all names' pitches, back to back at
// (layer*E + expert)*record_bytes of the paging file) is in RAM-tier row
// `row`, and every earlier request is answered; a failed read still answers.
// A seq past the next expected one counts the skipped requests as missed.
// done is stored again when the GPU's re-publish counter moves and once per
// idle second. The first failure is kept for ssd_error.
//
// Structure:
//   * A watcher thread polls the slot of the next expected seq. It copies a
//     published request out of the slot at once, checks every entry, and
//     appends one read task per record to a queue shared by the readers.
//     It goes straight back to polling, so a request published while an
//     earlier one is still being read (prefill chunks are published one
//     ahead) starts at once.
//   * Reader threads take read tasks from a queue. A record is read whole,
//     in one preadv: the paging file's disk serves a record in about the
//     time it serves a third of one, so reads are never split. The read
//     goes straight into the record's pinned rows with O_DIRECT; where the
//     pinned memory cannot be an O_DIRECT target (preadv fails with EFAULT,
//     seen with the GPU driver's pinned allocations) it goes into the next of
//     the reader's kBounce aligned bounce buffers instead, in rotation, and
//     the copy into the rows is cut into 256 KiB chunks on a second queue.
//     Four copier threads take those chunks, and so do idle readers
//     (non-temporal stores), while the reader goes on to its next read in
//     its next bounce buffer: reads and copies overlap even with one reader,
//     and one record's copy is spread over up to a dozen threads (against 1
//     MiB chunks and two copiers, single-record requests were answered 7%
//     sooner on average in alternating runs on one disk). A reader whose
//     next bounce buffer is still being copied out helps with the copies
//     first. The rotation is long because a read into a buffer that was just
//     copied out is slower (0.52 against 0.34 ms for a record in a plain
//     loop): with 32 buffers instead of 2 the server moved 9% to 100% more
//     per second in alternating runs on one disk.
//   * Each request counts its records down. The thread that completes a
//     record (its read, or the last chunk of its copy) counts it; the one
//     that finishes a request's last record marks it, then answers every
//     marked request at the head of the in-flight list in seq order.
//   * Idle readers sleep on a condition variable, and the watcher yields
//     the CPU between polls instead of spinning on pause instructions: on a
//     virtual machine host, pause loops exit to the hypervisor, and a
//     watcher that spun on them served single-record requests in about
//     twice the time of one that yields (0.78 against 0.43 ms, measured).
//   * Time is kept per phase (queue, read, copy: summed over threads, so
//     overlapping reads and copies both count), and the time with any
//     request in flight, for xp_ssd_phase_stats.
//
// Exported with the reference's C ABI (store.py:253-308).
#include <immintrin.h>
#include <sched.h>
#include <sys/uio.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <chrono>
#include <condition_variable>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

namespace {

constexpr int kMaxNames = 4;
constexpr int kHead = 2;                  // [re-publishes, give-ups]
constexpr long kAlign = 4096;             // O_DIRECT alignment of offsets, lengths and buffers
constexpr long kCopyChunk = 1L << 18;     // longest run of a bounce copy one thread takes
constexpr int kBounce = 32;               // bounce buffers per reader, allocated when first used
constexpr int kMaxInFlight = 64;          // requests picked up and not yet answered
constexpr int kCopiers = 4;               // copier threads (one copies about 6 GB/s into pinned rows)

inline void cpu_relax() {
#if defined(__x86_64__) || defined(__i386__)
  __builtin_ia32_pause();
#endif
}

inline int64_t now_ns() {
  using namespace std::chrono;
  return duration_cast<nanoseconds>(steady_clock::now().time_since_epoch()).count();
}

// Copy n bytes (a multiple of 128, both pointers 32-byte aligned) with
// non-temporal stores: the destination is read next by the GPU over the host
// link, so it is not worth a place in the CPU's caches, and streaming stores
// skip the read-for-ownership of each destination line.
__attribute__((target("avx2"))) void stream_copy_avx2(uint8_t* dst, const uint8_t* src, size_t n) {
  for (size_t i = 0; i < n; i += 128) {
    const __m256i a = _mm256_load_si256(reinterpret_cast<const __m256i*>(src + i));
    const __m256i b = _mm256_load_si256(reinterpret_cast<const __m256i*>(src + i + 32));
    const __m256i c = _mm256_load_si256(reinterpret_cast<const __m256i*>(src + i + 64));
    const __m256i d = _mm256_load_si256(reinterpret_cast<const __m256i*>(src + i + 96));
    _mm256_stream_si256(reinterpret_cast<__m256i*>(dst + i), a);
    _mm256_stream_si256(reinterpret_cast<__m256i*>(dst + i + 32), b);
    _mm256_stream_si256(reinterpret_cast<__m256i*>(dst + i + 64), c);
    _mm256_stream_si256(reinterpret_cast<__m256i*>(dst + i + 96), d);
  }
  _mm_sfence();  // the streaming stores land before the release that answers the request
}

void copy_out(uint8_t* dst, const uint8_t* src, size_t n) {
  static const bool avx2 = __builtin_cpu_supports("avx2");
  if (avx2 && n % 128 == 0 && (reinterpret_cast<uintptr_t>(dst) & 31) == 0 &&
      (reinterpret_cast<uintptr_t>(src) & 31) == 0)
    stream_copy_avx2(dst, src, n);
  else
    std::memcpy(dst, src, n);
}

}  // namespace

struct ssd_t {
  // One request between pickup and answer.
  struct Request {
    int64_t seq = 0;
    int64_t picked_ns = 0;
    long records = 0;
    std::atomic<long> left{0};  // records not yet in their rows, plus the watcher's hold
    std::atomic<bool> finished{false};
  };

  // The copy chunks of one bounced record still to be done; one per bounce
  // buffer of a reader, which reuses the buffer once `left` is 0.
  struct CopyGroup {
    std::atomic<long> left{0};
  };

  // A queued task: the read of one record (group == nullptr), or one chunk
  // of the copy of a bounced record into its row (req is the record's
  // request, counted down when the group's last chunk is copied).
  struct Task {
    Request* req = nullptr;
    long layer = 0, expert = 0, row = 0;
    int64_t queued_ns = 0;
    CopyGroup* group = nullptr;
    uint8_t* dst = nullptr;
    const uint8_t* src = nullptr;
    long bytes = 0;
  };

  // ---- configuration ----
  int fd = -1;
  int64_t* req = nullptr;
  int64_t* done = nullptr;
  long ring = 0, block = 0, slot_words = 0;
  long L = 0, E = 0, rows = 0, record_bytes = 0;
  int names = 0;
  uint8_t* pinned[kMaxNames] = {};
  long pitch[kMaxNames] = {};
  int nreaders = 1;

  // ---- state ----
  std::atomic<bool> stopping{false};
  std::atomic<long long> delay_ns{0};
  std::atomic<bool> direct{true};  // O_DIRECT straight into the pinned rows works

  std::mutex queue_mu;  // queue, copies, sleepers
  std::condition_variable queue_cv;
  std::deque<Task> queue;   // reads
  std::deque<Task> copies;  // copy chunks of bounced records
  int sleepers = 0;

  std::mutex answer_mu;  // in_flight, free_requests, answered, busy time and every store to `done`
  std::condition_variable slot_cv;
  std::deque<Request*> in_flight;
  std::vector<std::unique_ptr<Request>> pool;
  std::vector<Request*> free_requests;
  int64_t answered = 0;
  int64_t busy_ns = 0, busy_since = 0;

  // ---- statistics ----
  std::atomic<long> fetches{0}, reads{0}, missed{0}, preads{0};
  std::atomic<long long> io_ns{0}, queue_ns{0}, read_ns{0}, copy_ns{0};
  std::atomic<bool> failed{false};
  std::atomic<bool> failing{false};
  char err[512] = {0};

  std::thread watcher;
  std::vector<std::thread> copiers;
  std::vector<std::thread> readers;

  void fail(const char* fmt, ...) __attribute__((format(printf, 2, 3)));
  Request* take_request();
  void finish_record(Request* r);
  void answer_ready();
  bool enqueue(int64_t seq, const int64_t* slot, int64_t picked_ns);
  void watch();
  void read_loop();
  void copy_loop();
  int next_task(Task* out);
  bool take_copy(Task* out);
  void run_copy(const Task& t);
  void help_until_copied(const CopyGroup& g);
  long preadv_full(iovec* iov, int n, off_t off, int* error);
  bool serve(const Task& t, uint8_t* (&bounce)[kBounce], CopyGroup (&group)[kBounce], int* cur);
};

void ssd_t::fail(const char* fmt, ...) {
  bool expected = false;
  if (!failing.compare_exchange_strong(expected, true)) return;  // the first failure is kept
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(err, sizeof err, fmt, ap);
  va_end(ap);
  failed.store(true, std::memory_order_release);
}

// A free request record; waits while kMaxInFlight requests are unanswered.
ssd_t::Request* ssd_t::take_request() {
  std::unique_lock<std::mutex> lock(answer_mu);
  slot_cv.wait(lock, [&] { return !free_requests.empty() || stopping.load(); });
  if (free_requests.empty()) return nullptr;
  Request* r = free_requests.back();
  free_requests.pop_back();
  return r;
}

void ssd_t::finish_record(Request* r) {
  if (r->left.fetch_sub(1, std::memory_order_acq_rel) != 1) return;
  r->finished.store(true, std::memory_order_release);
  answer_ready();
}

// Answer, in seq order, every finished request at the head of the list.
void ssd_t::answer_ready() {
  std::lock_guard<std::mutex> lock(answer_mu);
  bool freed = false;
  while (!in_flight.empty() && in_flight.front()->finished.load(std::memory_order_acquire)) {
    Request* r = in_flight.front();
    in_flight.pop_front();
    const int64_t t = now_ns();
    fetches.fetch_add(1, std::memory_order_relaxed);
    reads.fetch_add(r->records, std::memory_order_relaxed);
    io_ns.fetch_add(t - r->picked_ns, std::memory_order_relaxed);
    answered = r->seq;
    __atomic_store_n(done, answered, __ATOMIC_RELEASE);
    free_requests.push_back(r);
    if (in_flight.empty()) busy_ns += t - busy_since;
    freed = true;
  }
  if (freed) slot_cv.notify_one();
}

// Queue the reads of the request in `slot`. Returns false when stopping.
bool ssd_t::enqueue(int64_t seq, const int64_t* slot, int64_t picked_ns) {
  Request* r = take_request();
  if (!r) return false;
  const long layer = static_cast<long>(__atomic_load_n(&slot[1], __ATOMIC_RELAXED));
  std::vector<Task> tasks;
  long records = 0;
  for (long j = 0; j < block; ++j) {
    const long e = static_cast<long>(__atomic_load_n(&slot[2 + j], __ATOMIC_RELAXED));
    if (e < 0) continue;  // unused entry
    const long row = static_cast<long>(__atomic_load_n(&slot[2 + block + j], __ATOMIC_RELAXED));
    ++records;
    if (layer < 0 || layer >= L || e >= E) {
      fail("expert %ld of layer %ld is out of range (%ld layers, %ld experts)", e, layer, L, E);
      continue;
    }
    if (row < 0 || row >= rows) {
      fail("row %ld for expert %ld of layer %ld is outside the RAM tier of %ld rows", row, e, layer, rows);
      continue;
    }
    Task t;
    t.req = r;
    t.layer = layer;
    t.expert = e;
    t.row = row;
    tasks.push_back(t);
  }
  r->seq = seq;
  r->picked_ns = picked_ns;
  r->records = records;
  r->finished.store(false, std::memory_order_relaxed);
  r->left.store(static_cast<long>(tasks.size()) + 1, std::memory_order_relaxed);  // +1: the watcher's hold
  {
    std::lock_guard<std::mutex> lock(answer_mu);
    if (in_flight.empty()) busy_since = picked_ns;
    in_flight.push_back(r);
  }
  if (!tasks.empty()) {
    const int64_t t = now_ns();
    bool wake;
    {
      std::lock_guard<std::mutex> lock(queue_mu);
      for (Task& task : tasks) {
        task.queued_ns = t;
        queue.push_back(task);
      }
      wake = sleepers > 0;
    }
    if (wake) queue_cv.notify_all();
  }
  finish_record(r);  // drop the watcher's hold: a request with no readable record is answered here
  return true;
}

void ssd_t::watch() {
  int64_t expected = 1;  // the seq the watcher waits for next
  int64_t republished = __atomic_load_n(&req[0], __ATOMIC_ACQUIRE);
  int64_t idle_since = now_ns();
  unsigned polls = 0;
  while (!stopping.load(std::memory_order_acquire)) {
    const int64_t* slot = req + kHead + (expected % ring) * slot_words;
    const int64_t seq = __atomic_load_n(&slot[0], __ATOMIC_ACQUIRE);
    if (seq >= expected) {
      const int64_t picked = now_ns();
      if (seq > expected) missed.fetch_add(static_cast<long>(seq - expected), std::memory_order_relaxed);
      // Test hook: hold the request for delay_ns before reading it.
      for (;;) {
        const long long d = delay_ns.load(std::memory_order_acquire);
        if (d <= 0 || now_ns() - picked >= d || stopping.load(std::memory_order_acquire)) break;
        usleep(1000);
      }
      if (stopping.load(std::memory_order_acquire) || !enqueue(seq, slot, picked)) return;
      expected = seq + 1;
      idle_since = now_ns();
      polls = 0;
      continue;
    }
    const int64_t r = __atomic_load_n(&req[0], __ATOMIC_ACQUIRE);
    bool resend = r != republished;
    republished = r;
    if (++polls >= 4096) {
      polls = 0;
      const int64_t now = now_ns();
      if (now - idle_since > 1000000000LL) {
        idle_since = now;
        resend = true;
      }
    }
    sched_yield();
    if (resend) {
      std::lock_guard<std::mutex> lock(answer_mu);
      __atomic_store_n(done, answered, __ATOMIC_RELEASE);
    }
  }
}

// The next task of a reader: a read if one is queued, else a copy chunk
// (1: read, 2: copy); 0 when stopping.
int ssd_t::next_task(Task* out) {
  std::unique_lock<std::mutex> lock(queue_mu);
  for (;;) {
    if (stopping.load(std::memory_order_acquire)) return 0;
    if (!queue.empty()) {
      *out = queue.front();
      queue.pop_front();
      return 1;
    }
    if (!copies.empty()) {
      *out = copies.front();
      copies.pop_front();
      return 2;
    }
    ++sleepers;
    queue_cv.wait(lock);
    --sleepers;
  }
}

// A copy chunk, if one is queued.
bool ssd_t::take_copy(Task* out) {
  std::lock_guard<std::mutex> lock(queue_mu);
  if (copies.empty()) return false;
  *out = copies.front();
  copies.pop_front();
  return true;
}

// Copy one chunk; the chunk that completes its record counts the record.
void ssd_t::run_copy(const Task& t) {
  const int64_t t0 = now_ns();
  copy_out(t.dst, t.src, static_cast<size_t>(t.bytes));
  copy_ns.fetch_add(now_ns() - t0, std::memory_order_relaxed);
  if (t.group->left.fetch_sub(1, std::memory_order_acq_rel) == 1) finish_record(t.req);
}

// Wait until a bounce buffer's chunks are all copied, copying queued chunks
// (of any record) meanwhile.
void ssd_t::help_until_copied(const CopyGroup& g) {
  Task other;
  while (g.left.load(std::memory_order_acquire) > 0) {
    if (take_copy(&other))
      run_copy(other);
    else
      cpu_relax();  // the last chunks are being copied by other threads
  }
}

// preadv until the iovecs are full, end of file or an error; returns the
// bytes read. The iovecs are advanced past what was read.
long ssd_t::preadv_full(iovec* iov, int n, off_t off, int* error) {
  long got = 0;
  *error = 0;
  int first = 0;
  while (first < n) {
    const ssize_t r = preadv(fd, iov + first, n - first, off + got);
    if (r < 0) {
      if (errno == EINTR) continue;
      *error = errno;
      break;
    }
    if (r == 0) break;
    got += r;
    size_t left = static_cast<size_t>(r);
    while (first < n && left >= iov[first].iov_len) left -= iov[first++].iov_len;
    if (first < n && left) {
      iov[first].iov_base = static_cast<uint8_t*>(iov[first].iov_base) + left;
      iov[first].iov_len -= left;
    }
  }
  return got;
}

// Read one record into its rows. Returns true when the record is complete
// (read straight into the rows, or failed); false when its copy out of a
// bounce buffer was queued, whose last chunk counts the record.
bool ssd_t::serve(const Task& t, uint8_t* (&bounce)[kBounce], CopyGroup (&group)[kBounce], int* cur) {
  const int64_t t0 = now_ns();
  queue_ns.fetch_add(t0 - t.queued_ns, std::memory_order_relaxed);
  const off_t off = static_cast<off_t>(t.layer * E + t.expert) * record_bytes;
  int error = 0;
  long got = 0;
  bool via_bounce = !direct.load(std::memory_order_relaxed);
  if (!via_bounce) {
    iovec iov[kMaxNames];
    for (int n = 0; n < names; ++n) iov[n] = iovec{pinned[n] + t.row * pitch[n], static_cast<size_t>(pitch[n])};
    got = preadv_full(iov, names, off, &error);
    if (error == EFAULT) {
      direct.store(false, std::memory_order_relaxed);  // the rows cannot be an O_DIRECT target
      via_bounce = true;
    }
  }
  const int b = *cur;
  int64_t t1 = now_ns();
  if (via_bounce) {
    help_until_copied(group[b]);  // the buffer's previous record is out
    if (!bounce[b]) {
      void* mem = nullptr;
      if (posix_memalign(&mem, kAlign, static_cast<size_t>(record_bytes)) != 0) {
        fail("cannot allocate a %ld B read buffer", record_bytes);
        return true;
      }
      bounce[b] = static_cast<uint8_t*>(mem);
    }
    t1 = now_ns();
    iovec one{bounce[b], static_cast<size_t>(record_bytes)};
    got = preadv_full(&one, 1, off, &error);
  }
  read_ns.fetch_add(now_ns() - (via_bounce ? t1 : t0), std::memory_order_relaxed);
  preads.fetch_add(1, std::memory_order_relaxed);
  if (error) {
    fail("reading expert %ld of layer %ld from the paging file failed: %s", t.expert, t.layer, strerror(error));
    return true;
  }
  if (got != record_bytes) {
    fail("short read: %ld of %ld B of expert %ld of layer %ld", got, record_bytes, t.expert, t.layer);
    return true;
  }
  if (!via_bounce) return true;

  // Queue the copy out of the bounce buffer and go on with the next one.
  std::vector<Task> chunks;
  long pos = 0;
  for (int n = 0; n < names; ++n) {
    uint8_t* dst = pinned[n] + t.row * pitch[n];
    for (long at = 0; at < pitch[n]; at += kCopyChunk) {
      Task c;
      c.req = t.req;
      c.group = &group[b];
      c.dst = dst + at;
      c.src = bounce[b] + pos + at;
      c.bytes = pitch[n] - at < kCopyChunk ? pitch[n] - at : kCopyChunk;
      chunks.push_back(c);
    }
    pos += pitch[n];
  }
  group[b].left.store(static_cast<long>(chunks.size()), std::memory_order_relaxed);
  bool wake;
  {
    std::lock_guard<std::mutex> lock(queue_mu);
    for (const Task& c : chunks) copies.push_back(c);
    wake = sleepers > 0;
  }
  if (wake) queue_cv.notify_all();
  *cur = b + 1 < kBounce ? b + 1 : 0;
  return false;
}

void ssd_t::read_loop() {
  uint8_t* bounce[kBounce] = {};
  CopyGroup group[kBounce];
  int cur = 0;
  Task t;
  for (;;) {
    const int kind = next_task(&t);
    if (kind == 0) break;
    if (kind == 2) {
      run_copy(t);
      continue;
    }
    if (serve(t, bounce, group, &cur)) finish_record(t.req);
  }
  // Chunks still queued point into this reader's buffers: see them copied
  // before the buffers go.
  for (const CopyGroup& g : group) help_until_copied(g);
  for (uint8_t* b : bounce) std::free(b);
}

// A copier: copy chunks as they are queued; at stop, the ones left first.
void ssd_t::copy_loop() {
  std::unique_lock<std::mutex> lock(queue_mu);
  for (;;) {
    if (!copies.empty()) {
      const Task c = copies.front();
      copies.pop_front();
      lock.unlock();
      run_copy(c);
      lock.lock();
      continue;
    }
    if (stopping.load(std::memory_order_acquire)) return;
    ++sleepers;
    queue_cv.wait(lock);
    --sleepers;
  }
}

extern "C" {

// `nworkers` + 1 reader threads serve the records (the reference's server
// reads with itself and `nworkers` workers), beside the watcher and the
// copiers.
ssd_t* ssd_start(int fd, void* req, void* done, long ring, long block, long L, long E, long rows, long record_bytes,
                 int names, void** pinned, long* pitch, int nworkers) {
  if (names < 1 || names > kMaxNames || !req || !done || ring < 1 || block < 1 || nworkers < 0 || nworkers > 255 ||
      !pinned || !pitch || record_bytes <= 0)
    return nullptr;
  long sum = 0;
  for (int i = 0; i < names; ++i) {
    if (!pinned[i] || pitch[i] <= 0) return nullptr;
    sum += pitch[i];
  }
  if (sum != record_bytes) return nullptr;
  ssd_t* s = new (std::nothrow) ssd_t;
  if (!s) return nullptr;
  s->fd = fd;
  s->req = static_cast<int64_t*>(req);
  s->done = static_cast<int64_t*>(done);
  s->ring = ring;
  s->block = block;
  s->slot_words = 2 + 2 * block;
  s->L = L;
  s->E = E;
  s->rows = rows;
  s->record_bytes = record_bytes;
  s->names = names;
  s->nreaders = nworkers + 1;
  for (int i = 0; i < names; ++i) {
    s->pinned[i] = static_cast<uint8_t*>(pinned[i]);
    s->pitch[i] = pitch[i];
  }
  try {
    for (int i = 0; i < kMaxInFlight; ++i) {
      s->pool.emplace_back(new ssd_t::Request);
      s->free_requests.push_back(s->pool.back().get());
    }
    for (int i = 0; i < kCopiers; ++i) s->copiers.emplace_back([s] { s->copy_loop(); });
    for (int i = 0; i < s->nreaders; ++i) s->readers.emplace_back([s] { s->read_loop(); });
    s->watcher = std::thread([s] { s->watch(); });
  } catch (...) {
    {
      std::lock_guard<std::mutex> q(s->queue_mu);
      s->stopping.store(true);
    }
    s->queue_cv.notify_all();
    for (auto& t : s->readers)
      if (t.joinable()) t.join();
    for (auto& t : s->copiers)
      if (t.joinable()) t.join();
    delete s;
    return nullptr;
  }
  return s;
}

void ssd_stop(ssd_t* s) {
  if (!s) return;
  {
    std::lock_guard<std::mutex> a(s->answer_mu);
    std::lock_guard<std::mutex> q(s->queue_mu);
    s->stopping.store(true, std::memory_order_release);
  }
  s->queue_cv.notify_all();
  s->slot_cv.notify_all();
  if (s->watcher.joinable()) s->watcher.join();
  for (auto& t : s->readers)
    if (t.joinable()) t.join();
  for (auto& t : s->copiers)
    if (t.joinable()) t.join();
  delete s;
}

void ssd_stats(ssd_t* s, long* fetches, long* reads, double* io_seconds, long* missed) {
  *fetches = s->fetches.load();
  *reads = s->reads.load();
  *io_seconds = static_cast<double>(s->io_ns.load()) * 1e-9;
  *missed = s->missed.load();
}

const char* ssd_error(ssd_t* s) { return s->failed.load(std::memory_order_acquire) ? s->err : nullptr; }

void ssd_test_delay(ssd_t* s, double seconds) {
  s->delay_ns.store(static_cast<long long>(seconds * 1e9), std::memory_order_release);
}

void xp_ssd_test_bounce(ssd_t* s) { s->direct.store(false, std::memory_order_relaxed); }

void xp_ssd_phase_stats(ssd_t* s, double* busy_s, double* queue_s, double* read_s, double* copy_s, long* preads,
                        int* readers, int* bounce) {
  {
    std::lock_guard<std::mutex> lock(s->answer_mu);
    *busy_s = static_cast<double>(s->busy_ns + (s->in_flight.empty() ? 0 : now_ns() - s->busy_since)) * 1e-9;
  }
  *queue_s = static_cast<double>(s->queue_ns.load()) * 1e-9;
  *read_s = static_cast<double>(s->read_ns.load()) * 1e-9;
  *copy_s = static_cast<double>(s->copy_ns.load()) * 1e-9;
  *preads = s->preads.load();
  *readers = s->nreaders;
  *bounce = s->direct.load() ? 0 : 1;
}

}  // extern "C"
