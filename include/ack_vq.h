/*
 * ack_vq.h -- C ABI of the MI355X (gfx950) vq4/v1 library, libackvq.so.
 *
 * vq4/v1 stores one 4-bit index per group of 8, 16 or 32 FP32 values, eight
 * indices per little-endian u32 word (vector v in word v/8, bits 4*(v%8)),
 * with one 16-entry FP32 codebook (16 x group values) per tensor.
 *
 * The first block of entry points is the drop-in surface: each one replaces
 * the reference entry of the same name in
 * src/alelyon_compute_kit/_kit/src/ffi.rs and keeps its argument meaning,
 * check order, return codes and refusal messages. Handles are registry ids,
 * never dereferenced: a device handle is a process-wide counter value, a
 * buffer handle is (device id << 32) | sequence (ffi.rs:10-24).
 *
 * ACK_OK from ack_vq means the work was enqueued on the device's stream, not
 * that it finished (ffi.rs:46-60). ack_download is a synchronisation point:
 * download the status word before trusting any output.
 *
 * The second block holds extensions with no reference counterpart; each says
 * who it is for.
 */
#ifndef ACK_VQ_H
#define ACK_VQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct AckDevice AckDevice; /* opaque; the pointer value is an id */
typedef struct AckBuffer AckBuffer; /* opaque; the pointer value is an id */

/* Return codes, values as ffi.rs:726-760. ACK_ERR_DEVICE is the reference's
 * ACK_ERR_VULKAN: a failure reported by the device runtime (HIP here). */
#define ACK_OK 0
#define ACK_ERR_NULL (-1)
#define ACK_ERR_DEVICE (-2)
#define ACK_ERR_SHAPE (-3)
#define ACK_ERR_SIZE (-4)
#define ACK_ERR_LIVE_BUFFERS (-5)
#define ACK_ERR_CLOSED (-6)
#define ACK_ERR_FOREIGN (-7)
#define ACK_ERR_FREED (-8)
#define ACK_ERR_ABI (-9)
#define ACK_ERR_POISONED (-10)
#define ACK_ERR_UNSUPPORTED_OP (-11)

/* Status-word bits written by every vq kernel (vq4.comp:4-7). */
#define ACK_VQ_STATUS_NONFINITE 1u
#define ACK_VQ_STATUS_LAYOUT 2u
#define ACK_VQ_STATUS_OPTIMIZER 4u

#define ACK_VQ_PLAN_BYTES 32

/* ---- drop-in surface ---------------------------------------------------- */

/* Replaces ack_vq_schema (ffi.rs:6004-6009). Returns 1. */
uint32_t ack_vq_schema(void);

/* Replaces ack_vq (ffi.rs:6037-6151). plan = 8 LE u32
 * [op, m, n, k, group, 16, flags, 0]; op 0 encode, 1 decode, 2 packed-pair
 * matmul (flags bit0: A stored (k,m); bit1: B stored (n,k)), 3 AdamW from
 * four packed states into dense [W'|M'|V'] scratch. Check order: null plan
 * (-1), plan length (-4), plan words (-3/-4), device (-1/-6), poisoned
 * (-10), six handles (-1/-7/-8), capacities/aliases/grid (-4/-3), launch. */
int32_t ack_vq(const AckDevice* dev, const AckBuffer* b0, const AckBuffer* b1,
               const AckBuffer* b2, const AckBuffer* b3, const AckBuffer* out,
               const AckBuffer* status, const uint8_t* plan, size_t plan_len);

/* Replaces ack_open (ffi.rs:2037). Opens the HIP device ACK_DEVICE names
 * ("gpu:<n>", default gpu:0). Null with ack_last_error set on failure. */
AckDevice* ack_open(void);

/* Replaces ack_close (ffi.rs:2365-2401). ACK_ERR_LIVE_BUFFERS while buffers
 * are allocated on the device. */
int32_t ack_close(AckDevice* dev);

/* Replaces ack_device_name (ffi.rs:3296-3318). */
int32_t ack_device_name(const AckDevice* dev, char* out, size_t len);

/* Replaces ack_last_error (ffi.rs:3325-3339): this thread's last message. */
int32_t ack_last_error(char* out, size_t len);

/* The library's ABI description, the layout of ffi.rs:1005-1060 (96 bytes).
 * This library implements the vq4/v1 entries only, so `operators`, every
 * op_schema_* and every capability_* read 0 (absent, as the reference
 * defines 0); `version` is the layout's ABI version (14); `shaders` is a
 * hash of the kernel sources this library was built from and `build` the
 * FNV-1a of the library name and that hash. */
typedef struct AckAbiInfo {
  uint32_t size;
  uint32_t version;
  uint64_t operators;
  uint64_t shaders;
  uint64_t build;
  uint32_t op_schema_matmul_bf16;
  uint32_t op_schema_cast;
  uint32_t capability_streams;
  uint32_t capability_rng;
  uint32_t capability_optimizer;
  uint32_t capability_serialization;
  uint32_t op_schema_matmul_f32;
  uint32_t op_schema_pointwise;
  uint32_t op_schema_reduce;
  uint32_t op_schema_rowwise;
  uint32_t op_schema_loss;
  uint32_t op_schema_embedding;
  uint32_t op_schema_matmul_f16;
  uint32_t op_schema_index;
  uint32_t op_schema_convert;
  uint32_t op_schema_intwise;
} AckAbiInfo;

/* Replaces ack_abi_info (ffi.rs:1981-2027): ACK_ERR_NULL for a null `out`,
 * ACK_ERR_ABI when `size` is smaller than this library's struct. */
int32_t ack_abi_info(AckAbiInfo* out, size_t size);

/* An open device's identity and limits, the layout of ffi.rs:1212-1250
 * (616 bytes), filled from the HIP runtime: vendor and PCI product ids, the
 * device UUID (the driver UUID has no HIP counterpart and reads zero), HIP
 * runtime and driver versions (api_version packed major << 22 | minor << 12
 * | patch as the reference packs Vulkan's), device type 2 (discrete GPU),
 * feature bits for what the hardware has (matrix cores with bf16 and fp16
 * 16x16x16 shapes, bf16 and 16-bit types, bf16 dot products; no subgroup
 * size control: waves are 64 wide), wave size, the 64-bit wall clock,
 * global memory, launch limits. The matmul and cast fields describe the
 * reference's bf16 matmul and cast families, which this library does not
 * implement: they read 0. `identity` is FNV-1a over bytes 8 to 160 and then
 * the library's `shaders` hash, as the reference defines it. */
typedef struct AckDeviceInfo {
  uint32_t size;
  uint32_t version;
  uint32_t api_version;
  uint32_t driver_version_raw;
  uint32_t driver_id;
  uint32_t vendor_id;
  uint32_t device_id;
  uint32_t device_type;
  uint8_t device_uuid[16];
  uint8_t driver_uuid[16];
  uint64_t features;
  uint32_t subgroup_size;
  uint32_t timestamp_valid_bits;
  float timestamp_period_ns;
  uint32_t max_push_constant_bytes;
  uint64_t device_local_bytes;
  uint64_t max_storage_buffer_bytes;
  uint32_t max_workgroup_invocations;
  uint32_t max_workgroup_count[3];
  uint32_t max_workgroup_size[3];
  uint32_t matmul_tile;
  uint32_t matmul_k_multiple;
  uint32_t matmul_layouts;
  uint32_t matmul_operand_dtype;
  uint32_t matmul_result_dtype;
  uint32_t cast_modes;
  uint32_t reserved;
  uint64_t identity;
  char device_name[256];
  char driver_name[64];
  char driver_info[128];
} AckDeviceInfo;

/* Replaces ack_device_info (ffi.rs:2410-2530): ACK_ERR_NULL for a null
 * `out`, ACK_ERR_ABI when `size` is smaller than this library's struct, then
 * the device lookup codes of ack_device_name. */
int32_t ack_device_info(const AckDevice* dev, AckDeviceInfo* out, size_t size);

/* Replaces ack_buffer_alloc (ffi.rs:3345-3375): device memory of `bytes`
 * (> 0); null with ack_last_error set on failure. */
AckBuffer* ack_buffer_alloc(const AckDevice* dev, uint64_t bytes);

/* Replaces ack_buffer_free (ffi.rs:3413-3441). */
int32_t ack_buffer_free(const AckDevice* dev, AckBuffer* buf);

/* Replaces ack_upload (ffi.rs:3477-3511): len must equal the buffer size. */
int32_t ack_upload(const AckDevice* dev, const AckBuffer* buf, const uint8_t* data, size_t len);

/* Replaces ack_download (ffi.rs:3525-3569): len must equal the buffer size;
 * waits for every operation enqueued on the device before copying. */
int32_t ack_download(const AckDevice* dev, const AckBuffer* buf, uint8_t* data, size_t len);

/* ---- extensions (no counterpart in the reference) ----------------------- */

/* Host-only admission query for bindings and tests, which cannot reach the
 * reference's Rust VqPlan: fills the six required byte counts, the work-item
 * count and the reference grid for `plan`. bounds 0 = this library's
 * multiply-add bound (2^38), 1 = the reference's scalar-shader bound (2^28).
 * Returns ack_vq's code for a refused plan, with the same message. Any
 * output pointer may be null. */
int32_t ack_vq_plan_query(const uint8_t* plan, size_t plan_len, uint32_t bounds,
                          uint64_t* required_bytes6, uint32_t* work_items,
                          uint32_t* dispatch3);

/* Host-only buffer admission, for the same callers: the reference's
 * validate_buffers on caller-supplied capacities and ids. */
int32_t ack_vq_plan_check_buffers(const uint8_t* plan, size_t plan_len,
                                  const uint64_t* capacities6, const uint64_t* ids6);

/* Batched ack_vq for callers that hold many equally shaped tensors (an
 * expert bank): `count` independent instances of `plan` in one launch. Slot
 * i holds `count` back-to-back images, each of the plan's required_bytes[i];
 * `out` likewise; one status word collects every instance's bits. Same check
 * order and codes as ack_vq, capacities scaled by `count` (count >= 1). */
int32_t ack_vq_batch(const AckDevice* dev, const AckBuffer* b0, const AckBuffer* b1,
                     const AckBuffer* b2, const AckBuffer* b3, const AckBuffer* out,
                     const AckBuffer* status, const uint8_t* plan, size_t plan_len,
                     uint32_t count);

/* ack_vq that allocates nothing. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same arguments,
 * check order, codes and results as ack_vq; the workspace some product paths
 * need (split-k partials of the GEMV kernels, gemv-direct's slice partials
 * and the nibble columns and split-k partials of onehot-mfma) comes from a
 * fixed 16 MiB device array that each GPU holds until the process ends, in
 * place of memory ack_vq would allocate. A plan needing more than 16 MiB of
 * it is refused with ACK_ERR_SIZE. The array belongs to one device handle at a time: calls on
 * one handle are ordered on its stream, and a call through another handle
 * of the same GPU is refused with ACK_ERR_DEVICE (the message names the
 * scratch) while the previous owner's enqueued noalloc work has not
 * finished; after ack_sync on that handle it proceeds. */
int32_t ack_vq_noalloc(const AckDevice* dev, const AckBuffer* b0, const AckBuffer* b1,
                       const AckBuffer* b2, const AckBuffer* b3, const AckBuffer* out,
                       const AckBuffer* status, const uint8_t* plan, size_t plan_len);

/* One fused VQAdamW step for VQAdamW.step on this library (vq.py:388-410):
 * the op-3 inputs (b0 = codes of W, M, V, G back to back; b1 = their four
 * books; b2 = seven FP32 coefficients; plan = the op-3 plan) are decoded and
 * updated per element exactly as op 3 computes them, but no dense scratch is
 * written. Instead: AdamW is evaluated at fit_codebook's strided sample of
 * whole vectors, each of W', M', V' gets a codebook fitted on the device
 * warm-started from its current book (vq.py:182-229, `iterations` and
 * `sample_vectors` as there, including the whole-tensor keep pass; the same
 * books as the CPU fit, bit for bit), and a last pass recomputes every
 * element and encodes it against its new book (op 0's FP32 rule) straight
 * into `out_codes` (3 x words(m) u32: W', M', V'). `out_books` receives the
 * three books (3 x 16 x group FP32), `changed` (one u32, cleared by the step)
 * the number of W values whose decoded value differs from the old W's.
 * Enqueued on the device stream like ack_vq: ACK_OK means accepted, and a
 * download waits for it. Status bits as op 3 and op 0; a nonzero status
 * means the outputs must be discarded. Both write slots and the status word
 * must be distinct buffers that alias no input. */
int32_t ack_vq_adamw_step(const AckDevice* dev, const AckBuffer* b0, const AckBuffer* b1,
                          const AckBuffer* b2, const AckBuffer* out_codes,
                          const AckBuffer* out_books, const AckBuffer* changed,
                          const AckBuffer* status, const uint8_t* plan, size_t plan_len,
                          uint32_t iterations, uint32_t sample_vectors);

/* Dense-activation product: C = op(X) . op(B) with op 2's plan, geometry and
 * flags (the 32-byte op-2 block), where X is a dense row-major FP32 array of
 * m x k values (k x m with flags & 1) instead of a packed image, so the
 * activations need no lossy encode (the harness encodes them,
 * src/alelyon_compute_kit/harness.py:140-149). B is packed as in op 2. A
 * separate entry: op 2 itself is unchanged. Status bit 1 on a nonfinite
 * value of X, of B's book or of an output. Results: the General path is
 * bit-identical to the op-2 loop with A read from X; the factorised paths
 * (m <= 8, m >= 64) agree within FP32 rounding. Enqueued like ack_vq. The
 * output and status must be distinct and alias no input. No counterpart in
 * the reference: for callers whose activations are dense float32, which the
 * reference harness must first encode, lossily, to call op 2. */
int32_t ack_vq_matmul_dense(const AckDevice* dev, const AckBuffer* x, const AckBuffer* b_codes,
                            const AckBuffer* b_book, const AckBuffer* out, const AckBuffer* status,
                            const uint8_t* plan, size_t plan_len);

/* The kernel path ack_vq_matmul_dense takes for an op-2 plan. */
int32_t ack_vq_dense_path_name(const uint8_t* plan, size_t plan_len, char* out, size_t len);

/* Codebook calibration on the device (fit_codebook, vq.py:182-257) of the m
 * FP32 values in `values`: bounded Lloyd on the strided sample of at most
 * `sample_vectors` complete vectors, farthest-point reseed, and, with a warm
 * start `init` (16 x group FP32; null for a cold start) on a sample smaller
 * than the tensor, the whole-tensor keep pass. `book_out` receives 16 x group
 * FP32, bit-identical to ack_vq_host_fit_codebook and the reference's
 * Python. The reference refuses nonfinite input before fitting; here a
 * nonfinite sampled value or init entry sets status bit 1, so read status
 * first. Enqueued like ack_vq. book_out and status must be distinct and
 * alias no input. For callers whose values already live on the device (the
 * optimizer's refit, a resident harness). */
int32_t ack_vq_fit_codebook(const AckDevice* dev, const AckBuffer* values, const AckBuffer* init,
                            const AckBuffer* book_out, const AckBuffer* status, uint64_t m,
                            uint32_t group, uint32_t iterations, uint32_t sample_vectors);

/* Stream timer for benchmarks: phase 0 records a start event on the device
 * stream, phase 1 records a stop event, waits for it and writes the elapsed
 * milliseconds to *ms_out. */
int32_t ack_stream_timer(const AckDevice* dev, uint32_t phase, float* ms_out);

/* Device-to-device copy of `bytes` from src + src_offset to dst + dst_offset,
 * enqueued on the device stream. Ranges must lie inside their buffers and
 * must not overlap. For callers that keep images resident and move one
 * between the slots of a multi-image buffer (the resident harness places the
 * gradient image into the fused optimizer step's input). */
int32_t ack_buffer_copy(const AckDevice* dev, const AckBuffer* dst, uint64_t dst_offset,
                        const AckBuffer* src, uint64_t src_offset, uint64_t bytes);

/* Sum of squares of `count` float32 values at the start of buffer `x`, in
 * float64, written to the first 8 bytes of `out` (enqueued like ack_vq). No
 * counterpart in the reference, whose harness takes the gradient's norm on the
 * host (src/alelyon_compute_kit/harness.py:196): for the resident harness,
 * which keeps the gradient on the device. Each square is exact in float64 and
 * the sum is taken in a fixed order, within (count / 65536 + 15) ulp-units
 * (2^-53) of the exact sum, relatively. ACK_ERR_SIZE when `count` values or 8
 * bytes do not fit the buffers. */
int32_t ack_vq_sum_squares(const AckDevice* dev, const AckBuffer* x, uint64_t count,
                           const AckBuffer* out);

/* x[i] = x[i] * factor for the first `count` float32 values of `x`, one
 * rounded FP32 multiply each, in place (enqueued like ack_vq). No counterpart
 * in the reference, whose harness scales the clipped gradient on the host
 * (src/alelyon_compute_kit/harness.py:200): for the resident harness. The
 * results equal numpy's float32 multiply bit for bit. ACK_ERR_SIZE when
 * `count` values do not fit the buffer. */
int32_t ack_vq_scale(const AckDevice* dev, const AckBuffer* x, uint64_t count, float factor);

/* Wait for every operation enqueued on the device. */
int32_t ack_sync(const AckDevice* dev);

/* Name of the kernel path ack_vq would take for `plan` on this library
 * (for tests that must know a fast path ran). */
int32_t ack_vq_path_name(const uint8_t* plan, size_t plan_len, char* out, size_t len);

/* The same for `count` instances launched together by ack_vq_batch (a batch
 * whose row instances fill the chip can take a path a single product does
 * not). No counterpart in the reference: for tests and benchmarks that must
 * know which kernel served a batched launch. */
int32_t ack_vq_batch_path_name(const uint8_t* plan, size_t plan_len, uint32_t count, char* out,
                               size_t len);

/* Path policy for one device: 0 = automatic, 1 = the general tiled kernel
 * for every matmul (a second implementation to cross-check fast paths),
 * 2 = a factorised path wherever its shape applies, below the size at which
 * the automatic choice would keep the general kernel (tests of small shapes);
 * it never takes gemv-direct, and onehot-mfma only from 64 rows (where no bin
 * kernel applies), so the bin kernels those replace in the automatic choice
 * are exercised at the same shapes. */
int32_t ack_vq_set_policy(const AckDevice* dev, uint32_t policy);

/* CPU reference encode (vq.py:154-179): nearest entry by float64 squared
 * distance, lowest index on ties, the final partial vector compared on its
 * valid values only. codes_out receives words(m) u32. */
int32_t ack_vq_host_encode(const float* values, uint64_t m, const float* book, uint32_t group,
                           uint32_t* codes_out);

/* Codebook calibration (vq.py:182-257): bounded Lloyd on a strided sample
 * with farthest-point reseed and the warm-start keep rule. init may be null.
 * book_out receives 16 x group FP32. */
int32_t ack_vq_host_fit_codebook(const float* values, uint64_t m, uint32_t group,
                                 uint32_t iterations, uint32_t sample_vectors,
                                 const float* init, float* book_out);

#ifdef __cplusplus
}
#endif

#endif /* ACK_VQ_H */
