// Host side of the SSD tier: a server thread that answers the GPU's read
// requests from the pinned request ring, with a pool of reader threads.
//
// Protocol (store.py:25-30, 83-251, gather.py:197-277):
//   req  = [re-publishes, give-ups] + `ring` slots of
//          [seq, layer, expert[block], row[block]]        (int64, pinned)
//   done = the last seq served                            (int64, pinned)
// The GPU writes a slot, then publishes its seq with a release store. The
// server serves requests strictly in seq order: it watches the slot of
// last+1, reads every listed expert (one record = all names' pitches, back to
// back, at (layer*E + expert)*record_bytes of the paging file) into RAM-tier
// row `row` with preadv, and release-stores done = seq. A seq that jumps past
// last+1 counts the skipped requests as missed. While idle, the server
// re-stores done when the GPU's re-publish counter moves, or every second, so
// a done that did not reach a waiting GPU is sent again. A read failure
// records the first error and still releases the GPU.
//
// Exported with the reference's C ABI (store.py:253-308) so the Python side
// binds it the same way.
//
// Reads go straight into the pinned rows when the kernel accepts them as an
// O_DIRECT target. Memory from the GPU driver's pinned allocator may not be
// (preadv fails with EFAULT); then every thread reads into its own aligned
// bounce buffer with O_DIRECT and copies the record into the rows, which
// still keeps the page cache from holding a second copy.
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
#include <cstring>
#include <cstdlib>
#include <memory>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

namespace {

constexpr int kMaxNames = 4;
constexpr int kHead = 2;  // [re-publishes, give-ups]

inline void cpu_relax() {
#if defined(__x86_64__) || defined(__i386__)
  __builtin_ia32_pause();
#endif
}

inline double mono_seconds() {
  using namespace std::chrono;
  return duration<double>(steady_clock::now().time_since_epoch()).count();
}

}  // namespace

struct ssd_t {
  int fd = -1;
  int64_t* req = nullptr;
  int64_t* done = nullptr;
  long ring = 0, block = 0, slot_words = 0;
  long L = 0, E = 0, rows = 0, record_bytes = 0;
  int names = 0;
  uint8_t* pinned[kMaxNames] = {};
  long pitch[kMaxNames] = {};

  std::atomic<long> fetches{0}, reads{0}, missed{0};
  std::atomic<long long> io_ns{0};
  std::atomic<int> failed{0};
  std::atomic<bool> failing{false};
  char err[512] = {0};
  std::atomic<long long> delay_ns{0};
  std::atomic<bool> direct{true};  // preadv straight into the pinned rows works

  // Job board of the request being served.
  std::mutex mu;
  std::condition_variable cv;
  long generation = 0;
  bool stop = false;
  std::atomic<bool> stop_flag{false};
  long layer = 0, njobs = 0, next_job = 0, finished = 0;
  std::vector<long> job_expert, job_row;
  std::vector<std::thread> workers;
  std::thread server;

  void fail(const char* fmt, ...) __attribute__((format(printf, 2, 3)));
  long read_iov(const iovec* iov, int n, off_t off, int* err);
  void read_job(long layer_, long e, long row);
  void drain_jobs();
  void worker_loop();
  void server_loop();
};

void ssd_t::fail(const char* fmt, ...) {
  bool expected = false;
  if (!failing.compare_exchange_strong(expected, true)) return;  // keep the first failure only
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(err, sizeof err, fmt, ap);
  va_end(ap);
  failed.store(1, std::memory_order_release);
}

// preadv until the iovecs are full, EOF or an error; returns the bytes read
// and the errno of a failure in *err.
long ssd_t::read_iov(const iovec* iov, int n, off_t off, int* err) {
  long got = 0, total = 0;
  for (int i = 0; i < n; ++i) total += static_cast<long>(iov[i].iov_len);
  *err = 0;
  while (got < total) {
    iovec part[kMaxNames];
    int np = 0;
    long skip = got;
    for (int i = 0; i < n; ++i) {
      if (skip >= static_cast<long>(iov[i].iov_len)) {
        skip -= static_cast<long>(iov[i].iov_len);
        continue;
      }
      part[np].iov_base = static_cast<uint8_t*>(iov[i].iov_base) + skip;
      part[np].iov_len = iov[i].iov_len - static_cast<size_t>(skip);
      skip = 0;
      ++np;
    }
    const ssize_t r = preadv(fd, part, np, off + got);
    if (r < 0) {
      if (errno == EINTR) continue;
      *err = errno;
      return got;
    }
    if (r == 0) break;
    got += r;
  }
  return got;
}

namespace {
struct Bounce {
  void* p = nullptr;
  size_t n = 0;
  ~Bounce() { std::free(p); }
  uint8_t* get(size_t bytes) {
    if (n < bytes) {
      std::free(p);
      p = nullptr;
      n = 0;
      if (posix_memalign(&p, 4096, bytes) != 0) return nullptr;
      n = bytes;
    }
    return static_cast<uint8_t*>(p);
  }
};
thread_local Bounce t_bounce;
}  // namespace

void ssd_t::read_job(long layer_, long e, long row) {
  if (layer_ < 0 || layer_ >= L || e < 0 || e >= E) {
    fail("expert %ld of layer %ld is out of range", e, layer_);
    return;
  }
  if (row < 0 || row >= rows) {
    fail("row %ld for expert %ld of layer %ld is outside the RAM tier of %ld rows", row, e, layer_, rows);
    return;
  }
  const off_t off = static_cast<off_t>(layer_ * E + e) * record_bytes;
  int err = 0;
  long got;
  if (direct.load(std::memory_order_relaxed)) {
    iovec iov[kMaxNames];
    for (int i = 0; i < names; ++i) {
      iov[i].iov_base = pinned[i] + row * pitch[i];
      iov[i].iov_len = static_cast<size_t>(pitch[i]);
    }
    got = read_iov(iov, names, off, &err);
    if (err != EFAULT) {
      if (err) fail("preadv of expert %ld of layer %ld failed: %s", e, layer_, strerror(err));
      else if (got != record_bytes)
        fail("short read: %ld of %ld B for expert %ld of layer %ld", got, record_bytes, e, layer_);
      return;
    }
    direct.store(false, std::memory_order_relaxed);  // the rows cannot be an O_DIRECT target
  }
  uint8_t* b = t_bounce.get(static_cast<size_t>(record_bytes));
  if (!b) {
    fail("cannot allocate a %ld B read buffer", record_bytes);
    return;
  }
  iovec one{b, static_cast<size_t>(record_bytes)};
  got = read_iov(&one, 1, off, &err);
  if (err) {
    fail("preadv of expert %ld of layer %ld failed: %s", e, layer_, strerror(err));
    return;
  }
  if (got != record_bytes) {
    fail("short read: %ld of %ld B for expert %ld of layer %ld", got, record_bytes, e, layer_);
    return;
  }
  long pos = 0;
  for (int i = 0; i < names; ++i) {
    std::memcpy(pinned[i] + row * pitch[i], b + pos, static_cast<size_t>(pitch[i]));
    pos += pitch[i];
  }
}

// Take jobs of the current request until none is left (server and workers).
void ssd_t::drain_jobs() {
  for (;;) {
    long j, e, row, lay;
    {
      std::lock_guard<std::mutex> lock(mu);
      if (next_job >= njobs) return;
      j = next_job++;
      e = job_expert[static_cast<size_t>(j)];
      row = job_row[static_cast<size_t>(j)];
      lay = layer;
    }
    read_job(lay, e, row);
    std::lock_guard<std::mutex> lock(mu);
    ++finished;
  }
}

void ssd_t::worker_loop() {
  long seen = 0;
  for (;;) {
    {
      std::unique_lock<std::mutex> lock(mu);
      cv.wait(lock, [&] { return stop || generation != seen; });
      if (stop) return;
      seen = generation;
    }
    drain_jobs();
  }
}

void ssd_t::server_loop() {
  int64_t last = 0;
  int64_t republished = __atomic_load_n(&req[0], __ATOMIC_ACQUIRE);
  for (;;) {
    int64_t* slot = req + kHead + ((last + 1) % ring) * slot_words;
    int64_t seq;
    long spins = 0;
    double idle_since = mono_seconds();
    while ((seq = __atomic_load_n(&slot[0], __ATOMIC_ACQUIRE)) <= last) {
      if (stop_flag.load(std::memory_order_acquire)) return;
      const int64_t r = __atomic_load_n(&req[0], __ATOMIC_ACQUIRE);
      if (r != republished) {
        republished = r;
        __atomic_store_n(done, last, __ATOMIC_RELEASE);
      }
      if (++spins >= 4096) {
        spins = 0;
        const double now = mono_seconds();
        if (now - idle_since > 1.0) {
          idle_since = now;
          __atomic_store_n(done, last, __ATOMIC_RELEASE);
        }
        sched_yield();
      } else {
        cpu_relax();
      }
    }
    const double t0 = mono_seconds();
    if (seq > last + 1) missed.fetch_add(static_cast<long>(seq - last - 1));
    for (;;) {  // test hook: hold the request for delay_ns
      const long long d = delay_ns.load(std::memory_order_acquire);
      if (d <= 0 || (mono_seconds() - t0) * 1e9 >= static_cast<double>(d)) break;
      if (stop_flag.load(std::memory_order_acquire)) return;
      usleep(1000);
    }
    long n = 0;
    {
      std::lock_guard<std::mutex> lock(mu);
      layer = static_cast<long>(__atomic_load_n(&slot[1], __ATOMIC_RELAXED));
      for (long j = 0; j < block; ++j) {
        const int64_t e = __atomic_load_n(&slot[2 + j], __ATOMIC_RELAXED);
        if (e < 0) continue;
        job_expert[static_cast<size_t>(n)] = static_cast<long>(e);
        job_row[static_cast<size_t>(n)] = static_cast<long>(__atomic_load_n(&slot[2 + block + j], __ATOMIC_RELAXED));
        ++n;
      }
      njobs = n;
      next_job = 0;
      finished = 0;
      if (n > 1) {  // a single read is done here without waking the pool
        ++generation;
        cv.notify_all();
      }
    }
    drain_jobs();
    for (spins = 0;;) {
      {
        std::lock_guard<std::mutex> lock(mu);
        if (finished >= n) break;
      }
      if (++spins >= 1024) {
        spins = 0;
        sched_yield();
      } else {
        cpu_relax();
      }
    }
    fetches.fetch_add(1);
    reads.fetch_add(n);
    io_ns.fetch_add(static_cast<long long>((mono_seconds() - t0) * 1e9));
    // Re-publishes made while this request was being read are not lost
    // handoffs.
    republished = __atomic_load_n(&req[0], __ATOMIC_ACQUIRE);
    __atomic_store_n(done, seq, __ATOMIC_RELEASE);  // also after a failed read
    last = seq;
  }
}

extern "C" {

ssd_t* ssd_start(int fd, void* req, void* done, long ring, long block, long L, long E, long rows, long record_bytes,
                 int names, void** pinned, long* pitch, int nworkers) {
  if (names < 1 || names > kMaxNames || !req || !done || ring < 1 || block < 1 || nworkers < 0 || !pinned || !pitch)
    return nullptr;
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
  for (int i = 0; i < names; ++i) {
    s->pinned[i] = static_cast<uint8_t*>(pinned[i]);
    s->pitch[i] = pitch[i];
  }
  try {
    s->job_expert.assign(static_cast<size_t>(block), 0);
    s->job_row.assign(static_cast<size_t>(block), 0);
    for (int i = 0; i < nworkers; ++i) s->workers.emplace_back([s] { s->worker_loop(); });
    s->server = std::thread([s] { s->server_loop(); });
  } catch (...) {
    {
      std::lock_guard<std::mutex> lock(s->mu);
      s->stop = true;
    }
    s->stop_flag.store(true);
    s->cv.notify_all();
    for (auto& t : s->workers)
      if (t.joinable()) t.join();
    delete s;
    return nullptr;
  }
  return s;
}

void ssd_stop(ssd_t* s) {
  if (!s) return;
  {
    std::lock_guard<std::mutex> lock(s->mu);
    s->stop = true;
  }
  s->stop_flag.store(true, std::memory_order_release);
  s->cv.notify_all();
  if (s->server.joinable()) s->server.join();
  for (auto& t : s->workers)
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

}  // extern "C"
