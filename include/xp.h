/*
 * xp.h -- C ABI of libxp, the gfx950 (MI355X) expert-paging library.
 *
 * Every entry point takes plain pointers and sizes, returns an int status
 * (XP_OK = 0) and never throws. On failure xp_last_error() describes the
 * problem (thread-local, valid until the next failing call on that thread).
 * GPU entry points take the hipStream_t they launch on as `void* stream`
 * (NULL = the null stream); they only enqueue work, allocate nothing and
 * never synchronise, so they can be captured into a hipGraph.
 *
 * Device pointers: all table, slab, staging, scale and LUT buffers live in
 * HBM. RAM-tier rows and the request ring live in pinned host memory
 * (xp_host_alloc); kernels read and write them over the host link through
 * their device-visible address (xp_host_device_pointer).
 *
 * Each declaration names the reference interface it replaces
 * (monochromegane/vllm-expert-pager v0.1.1, file:line).
 */
#ifndef XP_H
#define XP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define XP_OK 0
#define XP_E_ARG 1      /* bad argument (shape, size, null pointer) */
#define XP_E_PITCH 2    /* compressed row does not fit in its pitch */
#define XP_E_SHAPE 3    /* row length is not a multiple of the codec group */
#define XP_E_HIP 4      /* a HIP runtime call failed */
#define XP_E_LIMIT 5    /* a size exceeds what the kernel supports */

/* Description of the last failure on this thread ("" if none). */
const char* xp_last_error(void);
/* Library version string. */
const char* xp_version(void);

/* ---- LRU tables (device state) ----
 * One table per layer and tier. Same layout as ExpertTable
 * (table.py:28-54): int64 tensors with one trailing sink element.
 *   slot_of[E+1]    expert -> slot, -1 = not cached
 *   expert_in[S+1]  slot -> expert, -1 = free
 *   last_used[S+1]  step stamp, 0 = free
 *   step[1]         starts at 1
 *   hits[1], misses[1]
 */
typedef struct xp_table {
  int64_t* slot_of;
  int64_t* expert_in;
  int64_t* last_used;
  int64_t* step;
  int64_t* hits;
  int64_t* misses;
  int64_t num_experts; /* E */
  int64_t num_slots;   /* S (or R for the RAM tier) */
} xp_table;

/* Largest table the acquire kernels take (slots per table). */
#define XP_MAX_SLOTS 1024
/* Largest expert count the table kernels take. */
#define XP_MAX_EXPERTS 2048

/* Update the VRAM table and the RAM table from one step's routing, in one
 * launch. topk holds K expert ids (int32 if topk_elem_bytes == 4, int64 if 8);
 * negative ids are ignored. Requires K <= vram->num_slots and
 * K <= ram->num_slots. Writes expert_map[E] (int32, slot or -1 for unneeded
 * experts; from the VRAM table), vram_slot[E] / ram_slot[E] (slot of each
 * expert, meaningful for needed experts) and vram_todo[K] / ram_todo[K]
 * (misses in ascending expert id, then -1). pair_slot (nullable, int32[K])
 * receives the VRAM slot of each id in step order (-1 for an id outside
 * [0, E)), which xp_moe_decode_experts can take instead of looking each id
 * up in expert_map; the reference has no such output.
 * Replaces AcquirePair.__call__ (acquire.py:168-185) and its kernel
 * _acquire_pair_kernel / _acquire (acquire.py:25-141). */
int xp_acquire_pair(const void* topk, int topk_elem_bytes, int64_t K,
                    const xp_table* vram, const xp_table* ram,
                    int32_t* expert_map, int64_t* vram_slot, int64_t* vram_todo,
                    int64_t* ram_slot, int64_t* ram_todo, int32_t* pair_slot,
                    void* stream);

/* One table's acquire. expert_map_i64 (nullable) receives slot or -1 as
 * int64 (the torch version's return value), expert_map_i32 (nullable) the
 * same as int32. Requires K <= t->num_slots.
 * Replaces ExpertTable.acquire (table.py:75-128). */
int xp_table_acquire(const void* topk, int topk_elem_bytes, int64_t K,
                     const xp_table* t, int64_t* expert_map_i64,
                     int32_t* expert_map_i32, int64_t* slot_out, int64_t* todo,
                     void* stream);

/* need[e] = 1 if expert e appears among the n ids, else 0 (uint8[E]).
 * Replaces ExpertTable.need_mask (table.py:58-71). */
int xp_need_mask(const void* topk, int topk_elem_bytes, int64_t n,
                 int64_t num_experts, uint8_t* need, void* stream);

/* out[E]: the experts set in mask[E], packed from the front, then -1.
 * Replaces ExpertTable.pack (table.py:132-138). */
int xp_pack(const uint8_t* mask, int64_t num_experts, int64_t* out,
            void* stream);

/* Seed the RAM table `ram` from a prefill's routing: acquire the
 * max(R - S, 1) most referenced experts (ties: lower expert id first), then
 * the VRAM table's experts that are readable (in RAM or needed), without
 * counting hits or misses. need[E] is xp_need_mask of the same ids.
 * Replaces ExpertTable.seed (table.py:140-171). */
int xp_table_seed(const xp_table* ram, const xp_table* vram, const void* topk,
                  int topk_elem_bytes, int64_t n, const uint8_t* need,
                  void* stream);

/* Plan the chunks of a working-slab step after the RAM table update.
 * before[E] = RAM slot_of before the update, cached_row[E] = VRAM slot_of,
 * W = working rows. With N = ceil(E / W) + 1 chunks, writes dst_row[E],
 * src_row[E], maps[N*E] (int64, row or -1), and the listings todo, ssd,
 * late (int64[N*W] each).
 * Replaces ExpertTable.plan_chunks (table.py:173-247). */
int xp_plan_chunks(const xp_table* ram, const int64_t* before,
                   const uint8_t* need, const int64_t* cached_row, int64_t W,
                   int64_t ram_base, int64_t working_base, int64_t* dst_row,
                   int64_t* src_row, int64_t* maps, int64_t* todo,
                   int64_t* ssd, int64_t* late, void* stream);

/* The same five table operations on host memory, for tables kept in CPU
 * tensors: the reference's ExpertTable is device-agnostic torch code whose
 * tables also run on CPU tensors (table.py:1-9). Same arguments (minus the
 * stream), checks and results as the entry points above, computed by
 * sequential host code; every pointer is host memory. */
int xp_table_acquire_host(const void* topk, int topk_elem_bytes, int64_t K,
                          const xp_table* t, int64_t* expert_map_i64,
                          int32_t* expert_map_i32, int64_t* slot_out,
                          int64_t* todo);
int xp_need_mask_host(const void* topk, int topk_elem_bytes, int64_t n,
                      int64_t num_experts, uint8_t* need);
int xp_pack_host(const uint8_t* mask, int64_t num_experts, int64_t* out);
int xp_table_seed_host(const xp_table* ram, const xp_table* vram,
                       const void* topk, int topk_elem_bytes, int64_t n,
                       const uint8_t* need);
int xp_plan_chunks_host(const xp_table* ram, const int64_t* before,
                        const uint8_t* need, const int64_t* cached_row,
                        int64_t W, int64_t ram_base, int64_t working_base,
                        int64_t* dst_row, int64_t* src_row, int64_t* maps,
                        int64_t* todo, int64_t* ssd, int64_t* late);

/* ---- Gather (RAM tier / cache slab -> slab or staging) ---- */

/* One weight name (w13 or w2) of a gather. Sizes in bytes, multiples of 16;
 * all row bases 16-byte aligned. */
typedef struct xp_gather_name {
  const void* src;       /* RAM-tier rows, device-visible pinned memory */
  int64_t src_pitch;     /* bytes per RAM-tier row (pitch P, or N raw) */
  int64_t src_rows;      /* rows in src (row indices are checked against it) */
  const void* cache;     /* cache slab rows (raw, N bytes each), HBM */
  int64_t cache_rows;
  void* dst;             /* destination slab rows (raw, N bytes each), HBM */
  int64_t dst_rows;
  int64_t row_bytes;     /* N */
  void* stg;             /* compressed staging rows (P bytes each), or NULL */
  int64_t stg_rows;
  const void* scale;     /* scales of every expert, scale_bytes per expert */
  void* scale_dst;       /* scales in slot order (dst_rows rows) */
  int64_t scale_bytes;
} xp_gather_name;

/* Host<->device request ring (layout of store.py:434-457).
 * req = [re-publishes, give-ups] + ring slots of [seq, layer, expert[block],
 * row[block]] (int64, pinned coherent); done[1] (pinned coherent);
 * seq[1] (HBM). */
typedef struct xp_ring {
  int64_t* req;
  int64_t* done;
  int64_t* seq;
  int64_t block;
  int64_t ring;
} xp_ring;

/* Copy the rows and scales of the experts in todo[K] (-1 = empty).
 * Expert e with cache_row[e] >= 0 is copied raw from the cache slab row
 * cache_row[e] to dst row dst_row[e]; otherwise from RAM-tier row
 * src_row[e] + base: to staging row j (its index in todo) when the name has
 * stg, else to dst row dst_row[e]. The scale row of e is copied to
 * scale_dst row dst_row[e]. An expert whose dst_row[e] is outside
 * [0, dst_rows), or (with stg) whose staging row j is not below stg_rows,
 * is skipped (nothing of it is copied): with stg set and stg_rows = 0 the
 * launch copies only the cached experts, for a caller that expands the
 * others with xp_decode_rows_from_ram. With ring != NULL, the
 * same launch publishes the experts of ssd_todo[K] (K <= ring->block) to the
 * host ring for layer `layer`, waits for their done, and skips them in the
 * copy.
 * Replaces gather_rows (gather.py:328-393) and _gather_rows_kernel
 * (gather.py:51-194). */
int xp_gather_rows(const int64_t* todo, int64_t K, int64_t num_experts,
                   const int64_t* dst_row, const int64_t* cache_row,
                   const int64_t* src_row, int64_t base,
                   const xp_gather_name* names, int num_names,
                   const int64_t* ssd_todo, int64_t layer, const xp_ring* ring,
                   void* stream);

/* Number of copying workgroups of xp_gather_rows (the requests it keeps in
 * flight over the host link scale with it). Default 32. */
int xp_gather_set_blocks(int blocks);

/* Publish the experts of todo[K] to the ring and wait for done. Expert e
 * lands in RAM-tier row row[e] + base. No-op if todo is empty. A request slot
 * holds ring->block entries: the fetch entry points read only
 * todo[0 .. min(K, block)), as the reference's kernels do.
 * Replaces fetch_rows (gather.py:396-407). */
int xp_fetch_rows(const int64_t* todo, int64_t K, int64_t num_experts,
                  const int64_t* row,
                  int64_t base, int64_t layer, const xp_ring* ring,
                  void* stream);

/* Publish without waiting; the published seq goes to ticket[0] (HBM).
 * Replaces fetch_publish_rows (gather.py:410-431). */
int xp_fetch_publish_rows(const int64_t* todo, int64_t K,
                          int64_t num_experts, const int64_t* row,
                          int64_t base, int64_t layer, const xp_ring* ring,
                          int64_t* ticket, void* stream);

/* Wait until done >= ticket[0]; re-publish every `retry` interval and give up
 * after `giveup` re-publishes (both in xp_fetch_set_timing). No-op if todo is
 * empty. Replaces fetch_wait_rows (gather.py:434-439). */
int xp_fetch_wait_rows(const int64_t* todo, int64_t K, const xp_ring* ring,
                       const int64_t* ticket, void* stream);

/* Wait policy of the fetch kernels: re-publish after retry_us microseconds
 * without done, give up after giveup re-publishes. Defaults 500000 us and 8
 * (the reference: 2^18 spins, about 0.5 to 1.2 s, and 8; gather.py:36-48).
 * Affects launches made after the call. */
int xp_fetch_set_timing(int64_t retry_us, int64_t giveup);

/* ---- Codec (per-row fp8 exponent Huffman, format of codec.py:1-41) ---- */

#define XP_LIMIT 9
#define XP_LUT_BYTES 512
#define XP_CHUNK 512
#define XP_LANES 32

/* One weight name of a decode. */
typedef struct xp_decode_name {
  const void* stg;    /* compressed rows, pitch bytes apart (HBM) */
  int64_t pitch;      /* multiple of 16, below 2 GiB */
  int64_t stg_rows;
  void* dst;          /* raw destination rows, row_bytes apart (HBM) */
  int64_t dst_rows;
  int64_t row_bytes;  /* N, multiple of chunk * 32 */
} xp_decode_name;

/* Expand staging row j (the j-th entry of todo) into dst row dst_row[e] for
 * every name. Skips -1 entries, experts with cache_row[e] >= 0, experts
 * whose dst_row[e] is outside [0, dst_rows) and (when skip != NULL) experts
 * listed in skip[K]. lut is the layer's
 * uint8[E][num_names][512]. chunk = values per lane (512 in production;
 * any multiple of 32 up to 4096). A record's reads stay inside its pitch
 * whatever its contents, so a corrupt record yields wrong bytes in its own
 * destination row only.
 * Replaces decode_rows (codec.py:297-327) and _decode_rows_kernel /
 * _decode_group (codec.py:204-289). */
int xp_decode_rows(const int64_t* todo, int64_t K, int64_t num_experts,
                   const int64_t* dst_row, const int64_t* cache_row,
                   const uint8_t* lut,
                   const xp_decode_name* names, int num_names,
                   const int64_t* skip, int64_t chunk, void* stream);

/* The scale rows that go with one weight name's records. */
typedef struct xp_decode_scale {
  const void* scale;      /* scale rows by expert: row e at scale + e * scale_bytes (HBM) */
  void* scale_dst;        /* destination scale rows, by dst_row */
  int64_t scale_bytes;    /* bytes per scale row, a positive multiple of 4 */
  int64_t scale_rows;     /* at least num_experts */
  int64_t scale_dst_rows; /* at least the name's dst_rows */
} xp_decode_scale;

/* xp_decode_rows reading the records straight from the RAM tier: the
 * record of expert e = todo[j] is row src_row[e] + base of names[n].stg
 * (the tier's device address, stg_rows rows; a row outside [0, stg_rows)
 * is skipped, never clamped), and the expert's scale row is copied from
 * scales[n].scale[e] to scales[n].scale_dst[dst_row[e]]. The decoder's
 * ring loads then read the host link directly, so a decode step needs no
 * gather of its misses into staging first. Experts with cache_row[e] >= 0
 * are skipped entirely (records and scales), as are the other skips of
 * xp_decode_rows. No counterpart in the reference, whose decode reads a
 * staging copy (codec.py:297-327) that gather fills (gather.py:328-393);
 * it is for callers that decode a few misses per step from pinned RAM. */
int xp_decode_rows_from_ram(const int64_t* todo, int64_t K, int64_t num_experts,
                            const int64_t* dst_row, const int64_t* cache_row,
                            const int64_t* src_row, int64_t base,
                            const uint8_t* lut,
                            const xp_decode_name* names, int num_names,
                            const xp_decode_scale* scales,
                            const int64_t* skip, int64_t chunk, void* stream);

/* Host encoder: compress raw[n] (n multiple of chunk*32) into record[pitch]
 * (zero padded) and lut[512]. *needed receives the record's used bytes.
 * Returns XP_E_PITCH if it does not fit, XP_E_SHAPE if n is not a multiple.
 * Replaces encode (codec.py:125-193). */
int xp_encode_row(const uint8_t* raw, int64_t n, int64_t chunk,
                  uint8_t* record, int64_t pitch, uint8_t* lut,
                  int64_t* needed);

/* GPU encoder: compress `rows` device rows (raw + r*raw_stride, n values
 * each, n a multiple of chunk*32, chunk a power of two in 16..1024) into
 * records + r*pitch (zero padded) and luts + r*lut_stride (512 bytes), the
 * bytes xp_encode_row writes. needed[r] (device) receives each record's used
 * bytes; a row whose needed[r] exceeds pitch writes only its LUT, and the
 * caller reports it as xp_encode_row's XP_E_PITCH. All pointers are device
 * memory; enqueued on `stream`.
 * Replaces encode (codec.py:125-198), called per row at load time
 * (store.py:588). */
int xp_encode_rows(const uint8_t* raw, int64_t rows, int64_t raw_stride,
                   int64_t n, int64_t chunk, uint8_t* records, int64_t pitch,
                   uint8_t* luts, int64_t lut_stride, int64_t* needed,
                   void* stream);

/* Code of a 16-symbol histogram: lengths[16], bit-reversed codes[16] and
 * lut[512] ((sym << 4) | len). Replaces code_lengths / Code
 * (codec.py:61-114). */
int xp_code_build(const int64_t* hist, int32_t* lengths, int32_t* codes,
                  uint8_t* lut);

/* ---- Pinned host memory ---- */

/* hipHostMalloc of `bytes` (coherent != 0: fine-grained, else
 * coarse-grained), mapped for the device. */
int xp_host_alloc(void** ptr, int64_t bytes, int coherent);
int xp_host_free(void* ptr);
/* The device-visible address of pinned host memory. */
int xp_host_device_pointer(void** dev, void* host);

/* ---- SSD request server (host threads). Same ABI as the reference's
 * embedded C server (store.py:253-308). ---- */
typedef struct ssd_t ssd_t;
ssd_t* ssd_start(int fd, void* req, void* done, long ring, long block, long L,
                 long E, long rows, long record_bytes, int names,
                 void** pinned, long* pitch, int nworkers);
void ssd_stop(ssd_t* s);
void ssd_stats(ssd_t* s, long* fetches, long* reads, double* io_seconds,
               long* missed);
const char* ssd_error(ssd_t* s);
void ssd_test_delay(ssd_t* s, double seconds);
/* No counterpart in the reference, whose stats give fetches, reads and the
 * summed request time only: the seconds with at least one request in flight
 * (requests overlap, so this is below the summed time), and where the time
 * went, summed over the records read -- seconds a record waited in the
 * readers' queue, seconds in preadv, seconds copying out of bounce buffers
 * (all copy chunks) -- with the records read (one preadv each), the reader
 * threads, and whether reads go through bounce buffers (the pinned rows
 * refused O_DIRECT). */
/* No counterpart in the reference (a test hook like ssd_test_delay): read
 * through the bounce buffers from now on, as when the pinned rows refuse
 * O_DIRECT, so tests on ordinary host memory cover that path. */
void xp_ssd_test_bounce(ssd_t* s);
void xp_ssd_phase_stats(ssd_t* s, double* busy_s, double* queue_s, double* read_s,
                        double* copy_s, long* preads, int* readers, int* bounce);

/* ---- MoE expert compute on the slab (prefill overflow and decode) ----
 * These replace the vLLM fused fp8 MoE the reference hands expert_map to
 * (super().forward_modular in _expert_pager_run, experts.py:579-604) and its
 * moe_sum intercept (collect, experts.py:538-556). Weights are fp8 e4m3 (OCP)
 * with 128x128 fp32 block scales; activations are quantised per token and
 * 128-column group.
 *   w13 slab: [slots][2I][H] fp8 (gate rows, then up rows),
 *             scale [slots][2I/128][H/128] fp32
 *   w2  slab: [slots][H][I] fp8, scale [slots][H/128][I/128] fp32
 * A pair is p = t*topk + k. Each listed pair's contribution is computed from
 * its own token and expert alone, so splitting the experts over several
 * expert_maps (chunks) writes the same bits as one call over all of them.
 */

/* Quantise x[T][H] (bf16) to fp8 xq[T][H] and scales xs[T][H/128] (fp32):
 * s = max(amax, 1e-10) / 448, q = rne(clamp(x / s, -448, 448)).
 * H is a multiple of 128; x and xq 16-byte aligned. */
int xp_quant_tokens(const uint16_t* x, int64_t T, int64_t H, uint8_t* xq,
                    float* xs, void* stream);

/* Size of route's tile lists for `npairs` pairs over `slots` slots: size
 * `tiles` as 1 + 2 * xp_moe_max_tiles(npairs, slots) ints. */
int64_t xp_moe_max_tiles(int64_t npairs, int64_t slots);

/* List the pairs whose expert e (0 <= e < num_experts) has
 * 0 <= expert_map[e] < slots under that slot, in CSR form:
 * offsets[slots + 1], pairs[offsets[s] .. offsets[s+1]) (any order within a
 * slot; pairs holds up to T*topk entries). tiles[0] = tile count, then
 * (slot, first position) per tile of at most 64 pairs; from
 * tiles[1 + 2 * tb], tb = ceil(npairs / 64) + min(slots, npairs), the wide
 * tiles the prefill kernels run over: count, then (slot, first position,
 * pair count) per wide tile of at most 128 pairs. slots <= 1024. */
int xp_moe_route(const void* topk_ids, int topk_elem_bytes, int64_t T,
                 int64_t topk, const int32_t* expert_map, int64_t num_experts,
                 int64_t slots, int32_t* offsets, int32_t* pairs,
                 int32_t* tiles, void* stream);

/* xp_quant_tokens and xp_moe_route in one launch (the decode step's
 * quantisation and routing). Same arguments and results as the two calls. */
int xp_moe_quant_route(const uint16_t* x, int64_t T, int64_t H, uint8_t* xq,
                       float* xs, const void* topk_ids, int topk_elem_bytes,
                       int64_t topk, const int32_t* expert_map,
                       int64_t num_experts, int64_t slots, int32_t* offsets,
                       int32_t* pairs, int32_t* tiles, void* stream);

/* Bytes of the workspace xp_moe_experts needs for npairs = T*topk pairs
 * (bf16 and fp8 activations with their scales). */
int64_t xp_moe_workspace_bytes(int64_t npairs, int64_t I);

/* Expert activations (vLLM's "silu" and "gelu" with act-and-mul): the
 * activation of the gate in fp32, rounded to bf16, times up, rounded to
 * bf16, as silu_and_mul / gelu_and_mul compute it in bf16
 * (layers/activation.py). SiLU: g / (1 + exp(-g)); GELU, the erf form:
 * g / 2 * (1 + erf(g / sqrt(2))). */
#define XP_ACT_SILU 0
#define XP_ACT_GELU 1

/* Expert FFN of every routed pair, on the slab slot route chose:
 *   h = w13 . xq (block-scaled, fp32), gate = bf16(h[:I]), up = bf16(h[I:])
 *   a = bf16(bf16(act(gate)) * up) for act = `activation` (XP_ACT_*),
 *   quantised like xp_quant_tokens per 128 columns
 *   out[pair][H] = bf16(topk_weight[pair] * (w2 . a)) (bf16 bits)
 * topk_weight is fp32 [T*topk]; work is a 256-byte aligned device buffer of
 * xp_moe_workspace_bytes(T*topk, I) bytes (no initial contents needed).
 * Pairs that were not routed are not written. Two launches, gate/up (with
 * the activation quantisation) and down projection: at prefill sizes
 * (64 or more tiles can exist) persistent workgroups over the wide tiles,
 * otherwise 16-row subtiles. H and I are multiples of 128, at most 8192;
 * at prefill sizes T*H and T*topk*I are below 2^32; fp8 buffers and out
 * 16-byte aligned. */
int xp_moe_experts(const uint8_t* xq, const float* xs, int64_t T,
                   int64_t topk, const float* topk_weight, int64_t H,
                   int64_t I, const uint8_t* w13, const float* w13_scale,
                   const uint8_t* w2, const float* w2_scale, int64_t slots,
                   const int32_t* offsets, const int32_t* pairs,
                   const int32_t* tiles, void* work, int64_t work_bytes,
                   uint16_t* out, int activation, void* stream);

/* Workspace bytes xp_moe_experts_noalloc holds per device (32 MiB: a
 * 2048-token top-8 prefill at I = 512 needs 27.5 MB). */
#define XP_MOE_SCRATCH_BYTES (32LL << 20)

/* xp_moe_experts without a workspace argument, for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * workspace is a device array inside the library, XP_MOE_SCRATCH_BYTES on
 * every device it runs on, kept until the process ends; the call allocates
 * nothing. A call whose xp_moe_workspace_bytes(T * topk, I) exceeds
 * XP_MOE_SCRATCH_BYTES fails with XP_E_LIMIT before launching anything. All
 * calls on one device share that array, and nothing in it needs to start
 * zeroed: calls that overlap on one device (several streams, or several
 * threads without ordering) race; calls ordered on one stream do not.
 * Same arguments, results and bits as xp_moe_experts otherwise. */
int xp_moe_experts_noalloc(const uint8_t* xq, const float* xs, int64_t T,
                           int64_t topk, const float* topk_weight, int64_t H,
                           int64_t I, const uint8_t* w13,
                           const float* w13_scale, const uint8_t* w2,
                           const float* w2_scale, int64_t slots,
                           const int32_t* offsets, const int32_t* pairs,
                           const int32_t* tiles, uint16_t* out, int activation,
                           void* stream);

/* A decode step's expert FFN in two launches, for at most 64 pairs
 * (T * topk), H <= 4096 and topk * I <= 32768: out[T][H] gets the bits of
 * xp_moe_quant_route + xp_moe_experts + xp_moe_topk_sum, but the routing and
 * quantisation run inside the gate/up launch and each token's top-k sum
 * inside the down-projection launch (one workgroup per token and 8
 * columns). Replaces, like those calls, fused_experts + moe_sum of a step
 * whose experts are all in the slab (experts.py:579-604): every pair with a
 * valid id should have a slot (one without adds nothing here). work is
 * xp_moe_workspace_bytes(T * topk, I) bytes, 256-byte aligned. Fails with
 * XP_E_LIMIT (launching nothing) above those sizes. pair_slot (nullable)
 * gives each pair's slot directly, as xp_acquire_pair writes it; then
 * topk_ids and expert_map are not read (same bits when it equals
 * expert_map[topk_ids]). */
int xp_moe_decode_experts(const uint16_t* x, int64_t T, int64_t H,
                          const void* topk_ids, int topk_elem_bytes,
                          int64_t topk, const float* topk_weight,
                          const int32_t* expert_map, const int32_t* pair_slot,
                          int64_t num_experts, int64_t I, const uint8_t* w13,
                          const float* w13_scale, const uint8_t* w2,
                          const float* w2_scale, int64_t slots, void* work,
                          int64_t work_bytes, uint16_t* out, int activation,
                          void* stream);

/* The single top-k combine (moe_sum after collect, experts.py:546-552):
 * out[t][H] = bf16(sum over k ascending of fp32(contrib[t*topk + k])),
 * skipping pairs whose id is outside [0, num_experts). */
int xp_moe_topk_sum(const uint16_t* contrib, int64_t T, int64_t topk,
                    int64_t H, const void* topk_ids, int topk_elem_bytes,
                    int64_t num_experts, uint16_t* out, void* stream);

/* ---- measurement ---- */

/* Reads `count` records of record_bytes (a multiple of 4096) at the given
 * 4096-aligned offsets of fd (opened with O_DIRECT) into host buffers of the
 * library's own, `depth` (1..256) reads in flight: from `depth` threads
 * issuing pread, the way the SSD server's reader pool does (use_uring 0),
 * or from one io_uring queue of `depth` entries (use_uring 1). Writes the
 * elapsed seconds. Host only; no counterpart in the reference: it measures
 * the disk's ceiling for the paging file's record reads beside the server's
 * own rate. */
int xp_ssd_read_probe(int fd, int64_t record_bytes, const int64_t* offsets,
                      int64_t count, int depth, int use_uring,
                      double* seconds);

#ifdef __cplusplus
}
#endif

#endif /* XP_H */
