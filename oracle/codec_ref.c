/*
 * Oracle decoder of the fp8 exponent Huffman row format -- TEST
 * INFRASTRUCTURE ONLY (tests, smoke check, bench CPU baseline).
 *
 * The rule is the reference's sequential decoder (tests/test_codec.py:49-79,
 * the lane-by-lane restatement of codec.py:204-245): per group, lanes take
 * turns symbol by symbol; a lane whose 64-bit buffer holds fewer than LIMIT
 * bits first appends the next Huffman word of the group at its fill level;
 * the LUT entry (sym << 4 | len) of the low 9 bits gives the exponent; the
 * output byte is (s & 8) << 4 | sym << 3 | (s & 7) with s the lane's
 * sign/mantissa nibble. Returns non-zero if a group reads past its words.
 *
 * Rows are independent; oracle_decode_rows splits (row, group) tasks over
 * `threads` pthreads.
 */
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#define LIMIT 9
#define LANES 32

typedef struct {
  const uint8_t* records;
  long rows, pitch;
  const uint8_t* luts;
  uint8_t* out;
  long n, chunk, G;
  long next;
  int error;
  pthread_mutex_t mu;
} job_t;

static int32_t rd32(const uint8_t* p) {
  int32_t v;
  memcpy(&v, p, 4);
  return v;
}

static int decode_group(const uint8_t* rec, long pitch, const uint8_t* lut, uint8_t* out, long n, long chunk,
                        long G, long g) {
  const long nib_off = 4 * (G + 1), huff_off = nib_off + n / 2;
  const long max_words = (pitch - huff_off) / 4;
  long rp = rd32(rec + 4 * g);
  const long end = rd32(rec + 4 * (g + 1));
  if (rp < 0 || end > max_words || rp > end) return 1;
  uint64_t buf[LANES] = {0};
  int level[LANES] = {0};
  for (long i = 0; i < chunk; ++i) {
    const long m = i / 8, k = i % 8;
    for (int lane = 0; lane < LANES; ++lane) {
      if (level[lane] < LIMIT) {
        if (rp >= end) return 2;
        buf[lane] |= (uint64_t)(uint32_t)rd32(rec + huff_off + 4 * rp) << level[lane];
        level[lane] += 32;
        ++rp;
      }
      const uint8_t ent = lut[buf[lane] & 511];
      buf[lane] >>= (ent & 15);
      level[lane] -= (ent & 15);
      const uint32_t nib = (uint32_t)rd32(rec + nib_off + 4 * ((g * (chunk / 8) + m) * LANES + lane));
      const uint32_t s = (nib >> (4 * k)) & 15;
      out[(g * LANES + lane) * chunk + i] = (uint8_t)(((s & 8) << 4) | ((uint32_t)(ent >> 4) << 3) | (s & 7));
    }
  }
  return 0;
}

static void* worker(void* arg) {
  job_t* j = (job_t*)arg;
  for (;;) {
    pthread_mutex_lock(&j->mu);
    const long t = j->next++;
    pthread_mutex_unlock(&j->mu);
    if (t >= j->rows * j->G) return NULL;
    const long r = t / j->G, g = t % j->G;
    const int rc = decode_group(j->records + r * j->pitch, j->pitch, j->luts + r * 512, j->out + r * j->n, j->n,
                                j->chunk, j->G, g);
    if (rc) {
      pthread_mutex_lock(&j->mu);
      j->error = rc;
      pthread_mutex_unlock(&j->mu);
    }
  }
}

int oracle_decode_rows(const void* records, long rows, long pitch, const void* luts, void* out, long n, long chunk,
                       int threads) {
  if (chunk <= 0 || chunk % 8 || n % (chunk * LANES)) return 3;
  job_t j;
  j.records = (const uint8_t*)records;
  j.rows = rows;
  j.pitch = pitch;
  j.luts = (const uint8_t*)luts;
  j.out = (uint8_t*)out;
  j.n = n;
  j.chunk = chunk;
  j.G = n / (chunk * LANES);
  j.next = 0;
  j.error = 0;
  pthread_mutex_init(&j.mu, NULL);
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t tid[256];
  for (int i = 1; i < threads; ++i) pthread_create(&tid[i], NULL, worker, &j);
  worker(&j);
  for (int i = 1; i < threads; ++i) pthread_join(tid[i], NULL);
  pthread_mutex_destroy(&j.mu);
  return j.error;
}
