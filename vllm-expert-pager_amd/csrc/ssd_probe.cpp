// Read-throughput probe of the paging file: `count` whole records read with
// O_DIRECT at fixed file offsets, `depth` reads in flight, either from a pool
// of `depth` threads issuing pread (the way the SSD server reads) or from one
// thread driving an io_uring queue of `depth` entries (raw system calls; no
// library). It gives the disk's ceiling for record-sized reads in the same
// run as the server's own throughput.
#include <fcntl.h>
#include <linux/io_uring.h>
#include <sys/mman.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <chrono>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/xp.h"

namespace xp {
int fail(int code, const char* fmt, ...);
}

namespace {

double now_seconds() {
  using namespace std::chrono;
  return duration<double>(steady_clock::now().time_since_epoch()).count();
}

// One aligned buffer per read in flight.
struct Buffers {
  std::vector<void*> p;
  ~Buffers() {
    for (void* b : p) free(b);
  }
  bool make(int n, int64_t bytes) {
    for (int i = 0; i < n; ++i) {
      void* b = nullptr;
      if (posix_memalign(&b, 4096, static_cast<size_t>(bytes)) != 0) return false;
      p.push_back(b);
    }
    return true;
  }
};

int read_threads(int fd, int64_t record_bytes, const int64_t* offsets, int64_t count, int depth, Buffers& buf) {
  std::atomic<int64_t> next{0};
  std::atomic<int> err{0};
  std::vector<std::thread> pool;
  for (int t = 0; t < depth; ++t) {
    pool.emplace_back([&, t] {
      char* b = static_cast<char*>(buf.p[static_cast<size_t>(t)]);
      for (int64_t i; (i = next.fetch_add(1)) < count && err.load() == 0;) {
        int64_t got = 0;
        while (got < record_bytes) {
          const ssize_t r = pread(fd, b + got, static_cast<size_t>(record_bytes - got), offsets[i] + got);
          if (r <= 0) {
            int expected = 0;
            err.compare_exchange_strong(expected, r < 0 ? errno : EIO);
            return;
          }
          got += r;
        }
      }
    });
  }
  for (auto& th : pool) th.join();
  return err.load();
}

// A minimal io_uring: one submission queue entry per read in flight, reaped
// as they complete and refilled with the next record (or the rest of a
// short read).
struct Ring {
  int fd = -1;
  void* sq_ptr = MAP_FAILED;
  void* cq_ptr = MAP_FAILED;
  size_t sq_len = 0, cq_len = 0, sqe_len = 0;
  io_uring_sqe* sqes = static_cast<io_uring_sqe*>(MAP_FAILED);
  unsigned *sq_tail = nullptr, *sq_mask = nullptr, *sq_array = nullptr;
  unsigned *cq_head = nullptr, *cq_tail = nullptr, *cq_mask = nullptr;
  io_uring_cqe* cqes = nullptr;
  bool single = false;

  ~Ring() {
    if (sqes != MAP_FAILED) munmap(sqes, sqe_len);
    if (cq_ptr != MAP_FAILED && !single) munmap(cq_ptr, cq_len);
    if (sq_ptr != MAP_FAILED) munmap(sq_ptr, sq_len);
    if (fd >= 0) close(fd);
  }

  int open(unsigned entries) {
    io_uring_params p;
    memset(&p, 0, sizeof p);
    fd = static_cast<int>(syscall(__NR_io_uring_setup, entries, &p));
    if (fd < 0) return errno;
    single = (p.features & IORING_FEAT_SINGLE_MMAP) != 0;
    sq_len = p.sq_off.array + p.sq_entries * sizeof(unsigned);
    cq_len = p.cq_off.cqes + p.cq_entries * sizeof(io_uring_cqe);
    if (single) sq_len = cq_len = sq_len > cq_len ? sq_len : cq_len;
    sq_ptr = mmap(nullptr, sq_len, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd, IORING_OFF_SQ_RING);
    if (sq_ptr == MAP_FAILED) return errno;
    cq_ptr = single ? sq_ptr
                    : mmap(nullptr, cq_len, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd, IORING_OFF_CQ_RING);
    if (cq_ptr == MAP_FAILED) return errno;
    sqe_len = p.sq_entries * sizeof(io_uring_sqe);
    sqes = static_cast<io_uring_sqe*>(
        mmap(nullptr, sqe_len, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd, IORING_OFF_SQES));
    if (sqes == MAP_FAILED) return errno;
    char* sq = static_cast<char*>(sq_ptr);
    char* cq = static_cast<char*>(cq_ptr);
    sq_tail = reinterpret_cast<unsigned*>(sq + p.sq_off.tail);
    sq_mask = reinterpret_cast<unsigned*>(sq + p.sq_off.ring_mask);
    sq_array = reinterpret_cast<unsigned*>(sq + p.sq_off.array);
    cq_head = reinterpret_cast<unsigned*>(cq + p.cq_off.head);
    cq_tail = reinterpret_cast<unsigned*>(cq + p.cq_off.tail);
    cq_mask = reinterpret_cast<unsigned*>(cq + p.cq_off.ring_mask);
    cqes = reinterpret_cast<io_uring_cqe*>(cq + p.cq_off.cqes);
    return 0;
  }

  void queue_read(unsigned idx, int file, void* addr, unsigned len, int64_t off, uint64_t tag) {
    const unsigned tail = *sq_tail;
    io_uring_sqe* e = &sqes[idx];
    memset(e, 0, sizeof *e);
    e->opcode = IORING_OP_READ;
    e->fd = file;
    e->addr = reinterpret_cast<uint64_t>(addr);
    e->len = len;
    e->off = static_cast<uint64_t>(off);
    e->user_data = tag;
    sq_array[tail & *sq_mask] = idx;
    __atomic_store_n(sq_tail, tail + 1, __ATOMIC_RELEASE);
  }

  // Submits up to `submit` queued entries and waits for `wait` completions;
  // returns the entries the kernel took, or -errno.
  long enter(unsigned submit, unsigned wait) {
    const long r = syscall(__NR_io_uring_enter, fd, submit, wait, wait ? IORING_ENTER_GETEVENTS : 0, nullptr, 0);
    return r < 0 ? -errno : r;
  }
};

int read_uring(int fd, int64_t record_bytes, const int64_t* offsets, int64_t count, int depth, Buffers& buf) {
  Ring ring;
  int err = ring.open(static_cast<unsigned>(depth));
  if (err) return err;
  struct Slot {
    int64_t record = -1, got = 0;
  };
  std::vector<Slot> slot(static_cast<size_t>(depth));
  int64_t next = 0;
  // queued: entries written to the submission ring; submitted: taken by the
  // kernel; completed: reaped. Reads the kernel took are reaped before the
  // buffers can be freed, also after an error (then nothing new is queued).
  uint64_t queued = 0, submitted = 0, completed = 0;
  auto issue = [&](int s) {
    Slot& sl = slot[static_cast<size_t>(s)];
    const int64_t left = record_bytes - sl.got;
    ring.queue_read(static_cast<unsigned>(s), fd, static_cast<char*>(buf.p[static_cast<size_t>(s)]) + sl.got,
                    static_cast<unsigned>(left), offsets[sl.record] + sl.got, static_cast<uint64_t>(s));
    ++queued;
  };
  for (int s = 0; s < depth && next < count; ++s) {
    slot[static_cast<size_t>(s)] = Slot{next++, 0};
    issue(s);
  }
  while (completed < queued) {
    const unsigned to_submit = err ? 0u : static_cast<unsigned>(queued - submitted);
    if (submitted == completed && to_submit == 0) break;  // nothing the kernel holds; the rest never went in
    const long r = ring.enter(to_submit, 1);
    if (r < 0) {
      if (r != -EINTR && r != -EAGAIN && r != -EBUSY && !err) err = static_cast<int>(-r);
    } else {
      submitted += static_cast<uint64_t>(r);
    }
    unsigned head = *ring.cq_head;
    const unsigned tail = __atomic_load_n(ring.cq_tail, __ATOMIC_ACQUIRE);
    for (; head != tail; ++head) {
      const io_uring_cqe& c = ring.cqes[head & *ring.cq_mask];
      const int s = static_cast<int>(c.user_data);
      Slot& sl = slot[static_cast<size_t>(s)];
      ++completed;
      if (c.res <= 0) {
        if (!err) err = c.res < 0 ? -c.res : EIO;
        continue;
      }
      if (err) continue;
      sl.got += c.res;
      if (sl.got < record_bytes) {
        issue(s);  // short read: the rest of the record
      } else if (next < count) {
        sl = Slot{next++, 0};
        issue(s);
      }
    }
    __atomic_store_n(ring.cq_head, head, __ATOMIC_RELEASE);
  }
  return err;
}

}  // namespace

extern "C" {

int xp_ssd_read_probe(int fd, int64_t record_bytes, const int64_t* offsets, int64_t count, int depth,
                      int use_uring, double* seconds) {
  if (fd < 0 || record_bytes <= 0 || record_bytes % 4096 || record_bytes > (1LL << 30) || !offsets || count < 0 ||
      depth < 1 || depth > 256 || !seconds)
    return xp::fail(XP_E_ARG, "xp_ssd_read_probe: bad arguments (record %lld B, depth %d)",
                    static_cast<long long>(record_bytes), depth);
  for (int64_t i = 0; i < count; ++i)
    if (offsets[i] < 0 || offsets[i] % 4096)
      return xp::fail(XP_E_ARG, "xp_ssd_read_probe: offset %lld is not 4096-aligned",
                      static_cast<long long>(offsets[i]));
  Buffers buf;
  if (!buf.make(depth, record_bytes)) return xp::fail(XP_E_LIMIT, "xp_ssd_read_probe: out of host memory");
  const double t0 = now_seconds();
  const int e = use_uring ? read_uring(fd, record_bytes, offsets, count, depth, buf)
                          : read_threads(fd, record_bytes, offsets, count, depth, buf);
  *seconds = now_seconds() - t0;
  if (e) return xp::fail(XP_E_ARG, "xp_ssd_read_probe (%s): %s", use_uring ? "io_uring" : "pread", strerror(e));
  return XP_OK;
}

}  // extern "C"
