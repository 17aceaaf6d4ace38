/*
 * praghip - MI355X (gfx950) backend for the BFV polynomial engine and the
 * party-local Z_2^64 share GEMM of HaoR265/privacy-rag.
 *
 * C ABI: plain pointers and sizes, integer status codes, a thread-local error
 * string, no exceptions across the boundary and no silent CPU fallback.  Each
 * entry point names the reference interface it replaces (paths relative to
 * implementation_v1/).
 *
 * Layouts are the reference's: coefficient-major little-endian u64,
 * [batch][component][prime][N] for ciphertexts (ntt.hpp:20, switch.cu:65,71),
 * [digit][component][key prime][N] NTT-form keys (keyswitch/seal_adapter.cpp:37-39),
 * [prime][N][2] (operand, quotient) NTT tables (seal_tables.cpp:22-33) and
 * [out][in] weights (bfv_matrix.inc:101-105, artifacts.hpp:86-92).
 *
 * Pointers documented "device" are HIP device pointers on the plan's device;
 * "host" pointers are ordinary host memory.  `stream` is a hipStream_t used as
 * given (NULL is the HIP null stream).  Device-pointer entry points are
 * asynchronous on that stream; host-pointer entry points run on the plan's own
 * stream and are synchronous.
 *
 * After a HIP runtime error a plan releases itself (wipes and frees its
 * buffers) and every later call returns PRAGHIP_E_CLOSED, as the reference's
 * backends do (switch.cu:124, ntt.cu:163-167).
 *
 * A plan owns one set of scratch buffers that every call on it uses.  Calls on
 * one plan must therefore be ordered: device-pointer calls on one stream at a
 * time, and a host-pointer call (which runs on the plan's own stream) only
 * after the caller's earlier device calls on that plan have completed.  Two
 * calls that overlap on one plan - on different streams, or from different
 * threads - race on that scratch.  This is the reference's single-caller rule
 * (switch.cu:133, "single-threaded session caller only"); independent plans
 * may run concurrently.
 */
#ifndef PRAGHIP_H
#define PRAGHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; praghip_last_error() returns the reference's public code text
 * (E_NTT_SHAPE, E_NTT_CANONICAL_REQUIRED, E_SWITCH_CLOSED, ...). */
#define PRAGHIP_OK 0
#define PRAGHIP_E_SHAPE 1     /* E_NTT_SHAPE / E_SWITCH_SHAPE (ntt.cu:106, switch.cu:114) */
#define PRAGHIP_E_CANONICAL 2 /* E_NTT_CANONICAL_REQUIRED (ntt.cu:107) */
#define PRAGHIP_E_CONTEXT 3   /* E_NTT_CONTEXT: primes/tables rejected (seal_tables.cpp:11) */
#define PRAGHIP_E_CLOSED 4    /* E_NTT_CLOSED / E_SWITCH_CLOSED (ntt.cu:146, switch.cu:114) */
#define PRAGHIP_E_DEVICE 5    /* E_NTT_CUDA equivalent: HIP runtime error (ntt.cu:11) */
#define PRAGHIP_E_ARGUMENT 6  /* null pointer, bad Galois element, bad dtype */
#define PRAGHIP_E_STATE 7     /* E_CLIENT_KEY_STATE (ntt.cu:175,182) */

/* Cleanup report of close(): Cleanup{first_cuda_error, wipe_synchronized_bytes,
 * freed_bytes, closed} (ntt.hpp:15-19, switch.hpp:11). */
typedef struct praghip_cleanup {
  int32_t first_hip_error;
  int32_t closed;
  uint64_t wipe_synchronized_bytes;
  uint64_t freed_bytes;
} praghip_cleanup;

/* Timing of the last host-buffer call (ntt.hpp:10-14, switch.hpp:10). */
typedef struct praghip_timing {
  double upload_ms, kernel_ms, download_ms;
  uint64_t device_bytes, sensitive_bytes;
} praghip_timing;

/* Switch::Timing (switch.hpp:10): the phases of the last host-buffer keyswitch
 * (apply / evaluate), from events on the plan's stream between its launches.
 * At N = 16384 (digits of one to three primes) the keyswitch runs in three
 * kernel phases, whose boundaries are not the reference's:
 *   rns_ntt_ms  - ModUp (decompose, base conversion) and forward stages 0-3
 *                 of every expanded digit limb (the column kernel);
 *   product_ms  - forward stages 4-13, the key inner product and inverse
 *                 stages 0-9 of both sums (the row kernel);
 *   inverse_ms  - inverse stages 10-13 of the special prime's limbs;
 *   moddown_ms  - inverse stages 10-13 of the data primes' limbs with ModDown.
 * At other sizes the whole-limb kernel (ModUp, transforms and product) is
 * product_ms, its ModDown moddown_ms, and rns_ntt_ms = inverse_ms = 0.
 * setup_upload_ms is the plan's table, constant and key upload at creation.
 * The phases sum to kernel_ms of praghip_switch_timing. */
typedef struct praghip_switch_phases {
  double setup_upload_ms, upload_ms, rns_ntt_ms, product_ms, inverse_ms, moddown_ms, download_ms;
  uint64_t device_bytes, sensitive_bytes;
} praghip_switch_phases;

/* TokenWeights::Timing (resident.hpp:11-12): the phases of the last
 * host-buffer token evaluation (evaluate, evaluate_finished,
 * evaluate_local_finished).  lift_ms is 0 when every prime is on the integer
 * path (the transform lifts the ring words in its loads, so that time is in
 * ntt_ms); ntt_ms is the forward transform of the weight limbs (one kernel,
 * so there is no per-stage split like ntt_stages_ms); dyadic_ms the product
 * summed over the blocks; finish_ms the inverse transform, the local dot with
 * Delta scaling (bound shares) and the shift-and-add (0 for evaluate, which
 * returns NTT-form products).  initial_input_upload_ms is the creation's
 * ciphertext upload.  The phases sum to kernel_ms of praghip_token_timing. */
typedef struct praghip_token_phases {
  double initial_input_upload_ms, weight_upload_ms, lift_ms, ntt_ms, dyadic_ms, download_ms, finish_ms;
  uint64_t input_bytes, ring_weight_bytes, ntt_weight_bytes, output_bytes, device_bytes;
} praghip_token_phases;

const char *praghip_last_error(void);
int praghip_version(void);
/* Number of visible gfx950 devices (0 without a GPU; never initialises HIP
 * when the runtime reports no device). */
int praghip_device_count(void);

/* Device binding (the UUID + PCI-bus binding of ntt.cu:86-90, which reads
 * PRAG_ENC0_GPU_UUID / PRAG_ENC0_GPU_PCI; bfv_matrix.inc:35 and
 * silu_gpu_bridge.cpp:27 read the same pair under other names).
 * praghip_device_identity writes the two strings a binding compares:
 * uuid "GPU-" + the 16 bytes of hipDeviceProp_t.uuid (as characters when all
 * 16 are hex digits, the form rocminfo prints; else as 32 hex digits grouped
 * 8-4-4-4-12), pci the hipDeviceGetPCIBusId string ("0000:c1:00.0").
 * uuid_size >= 40, pci_size >= 16.  praghip_device_bind returns in *device
 * the gfx950 device whose identity equals both (hex digits compared
 * case-insensitively); praghip_device_bind_env reads the two values from the
 * named environment variables (NULL names: PRAG_ENC0_GPU_UUID and
 * PRAG_ENC0_GPU_PCI).  Errors: a variable unset or empty -> PRAGHIP_E_DEVICE
 * "E_PHASE_DEVICE_BINDING"; no gfx950 device matches -> PRAGHIP_E_DEVICE
 * "E_GFX950_REQUIRED" (the reference's E_RTX2060_REQUIRED). */
int praghip_device_identity(int device, char *uuid, size_t uuid_size, char *pci, size_t pci_size);
int praghip_device_bind(const char *uuid, const char *pci, int *device);
int praghip_device_bind_env(const char *uuid_var, const char *pci_var, int *device);

/* ---------------------------------------------------------------- tables */
/* SEAL NTTTables for one prime q == 1 mod 2N, q < 2^62 (the arrays
 * seal_tables.cpp:22-33 extracts): fwd_pairs/inv_pairs [N][2], invn_pair [2].
 * Also returns the minimal primitive 2N-th root if psi != NULL. */
int praghip_ntt_tables(uint64_t q, uint32_t log_n, uint64_t *fwd_pairs, uint64_t *inv_pairs,
                       uint64_t *invn_pair, uint64_t *psi);

/* ------------------------------------------------------------- NttBatch */
/* prag::experimental::ntt::NttBatch (ntt.hpp:22-40).  Tables may be NULL
 * (generated from q); when given they are validated against q.  `batches`
 * sizes the plan's own buffer for the host-vector calls; 4 <= log_n <= 14. */
typedef struct praghip_ntt_plan praghip_ntt_plan;
int praghip_ntt_plan_create(int device, const uint64_t *q, size_t primes, uint32_t log_n,
                            const uint64_t *fwd_pairs, const uint64_t *inv_pairs,
                            const uint64_t *invn_pairs, size_t batches, praghip_ntt_plan **plan);
/* In-place batched transforms over device [limbs][N], limb l on prime l % primes
 * (ntt.cu:104-127 stage loop).  forward: natural -> bit-reversed order;
 * inverse: bit-reversed -> natural.  Inputs must be canonical; data must be
 * 16-byte aligned. */
int praghip_ntt_forward(praghip_ntt_plan *plan, uint64_t *data, size_t limbs, void *stream);
int praghip_ntt_inverse(praghip_ntt_plan *plan, uint64_t *data, size_t limbs, void *stream);
/* NttBatch::transform (ntt.cu:145-168): host [batches][primes][N] in and out,
 * canonical-input check, synchronous. */
int praghip_ntt_transform(praghip_ntt_plan *plan, const uint64_t *input, uint64_t *output, int inverse);
/* NttBatch::bind_client_key (ntt.hpp:28, seal_tables.cpp:39-53): host [primes][N]
 * NTT-form secret key, canonical. */
int praghip_ntt_bind_client_key(praghip_ntt_plan *plan, const uint64_t *key);
/* NttBatch::client_phase (ntt.cu:181-199): NTT -> (.) key -> INTT, host buffers. */
int praghip_ntt_client_phase(praghip_ntt_plan *plan, const uint64_t *input, uint64_t *output);
int praghip_ntt_sync(praghip_ntt_plan *plan);
int praghip_ntt_timing(const praghip_ntt_plan *plan, praghip_timing *out);
/* NttBatch::close (ntt.cu:103-121): idempotent wipe + free. */
int praghip_ntt_close(praghip_ntt_plan *plan, praghip_cleanup *out);
void praghip_ntt_destroy(praghip_ntt_plan *plan);

/* --------------------------------------------------------------- Switch */
/* prag::experimental_full_switch::Switch (switch.hpp:12-28), generalised to
 * dnum digits: q has L+1 primes, q[L] is the special prime; key is the host
 * [dnum][2][L+1][N] NTT-form switching key for `element` (NULL: keys are passed
 * per call).  dnum = L reproduces the reference exactly (one prime per digit,
 * no base conversion); dnum < L uses fast base conversion (ModUp).  max_batch
 * sizes the plan's scratch.  L+1 <= 16.
 * The SEAL arrays Switch::initialize(q, f, r, ni, invp, keys) receives
 * (switch.hpp:24, extracted by keyswitch/seal_adapter.cpp:24-41) may be
 * passed as they are: fwd_pairs / inv_pairs [L+1][N][2] (root powers and
 * inverse root powers, operand and quotient), invn_pairs [L+1][2] (N^-1) and
 * invp_pairs [L][2] (inv_q_last_mod_q: q[L]^-1 mod q_i).  Each may be NULL
 * (derived from q); when given it is compared with the derived one and a
 * mismatch returns PRAGHIP_E_CONTEXT "E_NTT_CONTEXT", so a caller's tables
 * and the keys it built with them are known to agree with the transforms.
 * Key words (here and in praghip_keyswitch) must be canonical residues mod
 * their prime. */
typedef struct praghip_switch_plan praghip_switch_plan;
int praghip_switch_plan_create(int device, const uint64_t *q, size_t data_primes, uint32_t log_n,
                               size_t dnum, const uint64_t *fwd_pairs, const uint64_t *inv_pairs,
                               const uint64_t *invn_pairs, const uint64_t *invp_pairs, const uint64_t *key,
                               uint32_t element, size_t max_batch, praghip_switch_plan **plan);
/* Switch::apply (keyswitch/seal_adapter.cpp:44-52 + switch.cu:113-125): host
 * [2][L][N] coefficient-form ciphertext -> Galois(element) + keyswitch -> host
 * [2][L][N]. */
int praghip_switch_apply(praghip_switch_plan *plan, const uint64_t *input, uint64_t *output);
/* Switch::evaluate (switch.hpp:26, switch.cu:113-125): keyswitch only, host
 * [2][L][N] coefficient-form ciphertext that the caller has already permuted
 * by the plan's element (as keyswitch/seal_adapter.cpp:49-51 does on the CPU
 * before calling evaluate) -> host [2][L][N].  No Galois gather. */
int praghip_switch_evaluate(praghip_switch_plan *plan, const uint64_t *input, uint64_t *output);
/* Batched device keyswitch: in/out device [batch][2][L][N] (8-byte aligned);
 * keys device [dnum][2][L+1][N] per ciphertext at key_stride words apart (0:
 * one shared key; NULL keys: the plan's key), 16-byte aligned with an even
 * key_stride (E_SWITCH_ALIGNMENT).  galois_elt odd, < 2N (1 = plain switch).
 * Device key words must be canonical (k < q_t): they are not checked here,
 * and with every key prime below 2^60 the key products are Montgomery
 * products whose lazy bounds assume it (a plan's own key is checked at
 * creation, E_SWITCH_KEY_CANONICAL). */
int praghip_keyswitch(praghip_switch_plan *plan, const uint64_t *input, uint64_t *output, size_t batch,
                      const uint64_t *keys, size_t key_stride, uint32_t galois_elt, void *stream);
int praghip_switch_sync(praghip_switch_plan *plan);
int praghip_switch_timing(const praghip_switch_plan *plan, praghip_timing *out);
/* Switch::timing (switch.hpp:10, printed by check_switch.cpp:23): per-phase
 * times of the last host-buffer call (praghip_switch_phases). */
int praghip_switch_phase_timing(const praghip_switch_plan *plan, praghip_switch_phases *out);
int praghip_switch_close(praghip_switch_plan *plan, praghip_cleanup *out);
void praghip_switch_destroy(praghip_switch_plan *plan);

/* ------------------------------------------------------ share GEMM (ring) */
/* Party-local share GEMM, the loop of bfv_matrix.inc:101-105/156-160/177-182
 * (and batch_matrix.inc:120-156) as a LocalShares operation
 * (local_shares.hpp:22-32): y[m][n] = ((sum_k x[m][k] * w[n][k]) << shifts[n])
 * mod 2^mask_bits, x u64 device [M][K], w signed device [N][K] (w_bits 8: int8;
 * 32: int32 in [-0x808080, 0x7F7F7F], three balanced signed bytes; the
 * reference f12 domain is |w| <= 2^20; 24: the same weights pre-split by
 * praghip_weights_split or praghip_weights_upload_split into three int8
 * planes [3][N][K], w = sum_e plane_e 256^e - the fast form of static f12
 * weights),
 * shifts device int8 [N] in [0,63] or NULL, y u64 device [M][N]; mask_bits 59
 * is the reference ring, 64 is no mask.  Asynchronous on `stream` (NULL: the
 * null stream of `device`). */
int praghip_share_gemm(int device, const uint64_t *x, const void *w, int w_bits, const int8_t *shifts,
                       uint64_t *y, size_t m, size_t k, size_t n, int mask_bits, void *stream);

/* praghip_share_gemm with int8 weights (w_bits 8) computed by VALU dot products
 * (v_dot4_i32_i8 on the same offset-binary digit planes) instead of the i8
 * matrix cores: the same results, kept as the measured alternative that the
 * MFMA kernels are chosen over (bfv_matrix.inc:101-105 is the operation). */
int praghip_share_gemm_valu(int device, const uint64_t *x, const int8_t *w, const int8_t *shifts, uint64_t *y,
                            size_t m, size_t k, size_t n, int mask_bits, void *stream);

/* Splits `count` int32 weights in [-0x808080, 0x7F7F7F] (device) into the
 * three balanced signed-byte planes of w_bits 24 (device int8 [3][count]),
 * once per weight matrix (the reference's weights are static,
 * quantize_weights.py:91,102).  Weights outside the range are not detected. */
int praghip_weights_split(int device, const int32_t *w, int8_t *planes, size_t count, void *stream);

/* A list of share GEMMs launched in order on one stream, for the per-layer
 * projections of Transformer::project_many / project_joint_many
 * (model.hpp:66-126): the joint q/k/v and gate/up products, o and down.  Each
 * entry has the meaning of praghip_share_gemm's arguments; the whole list is
 * validated before the first launch. */
typedef struct praghip_gemm_desc {
  const uint64_t *x;
  const void *w;
  const int8_t *shifts;
  uint64_t *y;
  size_t m, k, n;
  int w_bits, mask_bits;
} praghip_gemm_desc;
int praghip_share_gemm_batch(int device, const praghip_gemm_desc *list, size_t count, void *stream);

/* --------------------------------------------------------- ring ops (local) */
/* LocalShares add / scale / layout / sum_rows (local_shares.hpp:22-32, kernels
 * at local_shares.cu:9-12) on device buffers, asynchronous on `stream`, mod
 * 2^mask_bits (59 = the reference ring).  add/scale: 16-byte aligned a, b, c
 * [n].  layout: c[i] = a[map[i]] for i < n_out, map u64 device indices; an
 * index >= n_in reads nothing and gives 0 (the reference rejects such a map on
 * the host with E_CUDA_PUBLIC_MAP; the Python mirror does the same).
 * sum_rows: out[r] = sum of the cols words of row r of a [rows][cols]. */
int praghip_ring_add(int device, const uint64_t *a, const uint64_t *b, uint64_t *c, size_t n, int mask_bits,
                     void *stream);
int praghip_ring_scale(int device, const uint64_t *a, uint64_t factor, uint64_t *c, size_t n, int mask_bits,
                       void *stream);
int praghip_ring_layout(int device, const uint64_t *a, size_t n_in, const uint64_t *map, uint64_t *c, size_t n_out,
                        void *stream);
int praghip_ring_sum_rows(int device, const uint64_t *a, uint64_t *out, size_t rows, size_t cols, int mask_bits,
                          void *stream);

/* ShareStorage of LocalShares::allocate (local_shares.hpp:12-17,29,
 * local_shares.cu:14-24): `words` device words of one participant's ring-2^59
 * shares, zero-filled on allocation (E_CUDA_SHAPE for 0 words).  write: host
 * words[count] -> storage[offset..], each < 2^59 (E_CUDA_WORD), inside the
 * storage (E_CUDA_SHAPE); read: storage[offset..offset+count) -> host; both
 * synchronous on the storage's own stream.  data: the device address (for the
 * ring ops and the share GEMM).  clear (ShareStorage::clear): wipes with
 * zeros, synchronises and frees, idempotent, reported like a plan's close;
 * later calls return E_CUDA_STORAGE_CLOSED.  stats: bytes uploaded and
 * downloaded (LocalShareStats, local_shares.hpp:18-21). */
typedef struct praghip_share_storage praghip_share_storage;
int praghip_storage_allocate(int device, size_t words, praghip_share_storage **storage);
int praghip_storage_write(praghip_share_storage *storage, size_t offset, const uint64_t *words, size_t count);
int praghip_storage_read(praghip_share_storage *storage, size_t offset, size_t count, uint64_t *out);
int praghip_storage_data(praghip_share_storage *storage, uint64_t **data, size_t *words);
int praghip_storage_stats(const praghip_share_storage *storage, uint64_t *uploaded_bytes, uint64_t *downloaded_bytes);
int praghip_storage_clear(praghip_share_storage *storage, praghip_cleanup *out);
void praghip_storage_destroy(praghip_share_storage *storage);

/* Centred lift of ring-2^59 words into RNS residues (matrix.cu:23-26 lift for
 * width 0; resident.cu:23-30 lift for width > 0): out[b][k][z] = the signed
 * value of v (v - 2^59 when bit 58 is set) mod q_k, canonical; for q_k > 2^59
 * this is the reference's v + ((q_k - 2^59) & -(v >> 58)).  v = ring[b][z] (width 0, ring
 * [blocks][2^log_n]) or v = ring[b][width-1-z] for z < width and 0 above
 * (ring [blocks][width]).  out device [blocks][primes][2^log_n]. */
int praghip_lift59(int device, const uint64_t *ring, uint64_t *out, size_t blocks, uint32_t log_n, size_t width,
                   const uint64_t *q, size_t primes, void *stream);

/* Dyadic multiply-accumulate, Barrett-128 (resident.cu:38-45 accumulate,
 * matrix.cu:34-38 product): out[l][z] = sum_b a[b][l][z] * w[b][l % w_limbs][z]
 * mod q[l % primes]; a [blocks][limbs][2^log_n], w [blocks][w_limbs][2^log_n],
 * out [limbs][2^log_n], device. */
int praghip_dyadic_mac(int device, const uint64_t *a, const uint64_t *w, uint64_t *out, size_t blocks, size_t limbs,
                       uint32_t log_n, size_t w_limbs, const uint64_t *q, size_t primes, void *stream);

/* Party-local dot product with BFV Delta scaling (resident.cu:60-74
 * local_partials + local_scale, constants of resident/seal_adapter.cpp:43-53):
 * m = (sum_j shares[s][j] * weights[j] mod 2^64) & (2^59 - 1), then
 * scaled[s][k] = Delta_k * m + floor((r * m + 2^58) / 2^59) mod q_k, with
 * delta[k] = floor(Q/2^59) mod q_k and r = Q mod 2^59.  shares
 * [slots][words], weights [words], scaled [slots][primes], workspace of
 * praghip_local_dot_workspace_words(slots) u64, all device. */
size_t praghip_local_dot_workspace_words(size_t slots);
int praghip_local_dot_scale(int device, const uint64_t *shares, const uint64_t *weights, size_t words, size_t slots,
                            const uint64_t *delta, uint64_t r, const uint64_t *q, size_t primes, uint64_t *scaled,
                            uint64_t *workspace, void *stream);
/* Allocation-free praghip_local_dot_scale.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops).  Same arguments and results without the
 * workspace: the partial sums go to a static device array of
 * PRAGHIP_NOALLOC_MAX_SLOTS x 256 words (128 KiB), one per device, held until
 * the process ends.  slots above the limit: PRAGHIP_E_SHAPE
 * (E_LOCAL_NOALLOC_SLOTS).  Every call on a device shares that array, so
 * calls that overlap on one device (other streams, other threads) race; the
 * caller serialises them.  Calls no allocating routine. */
#define PRAGHIP_NOALLOC_MAX_SLOTS 64
int praghip_local_dot_scale_noalloc(int device, const uint64_t *shares, const uint64_t *weights, size_t words,
                                    size_t slots, const uint64_t *delta, uint64_t r, const uint64_t *q, size_t primes,
                                    uint64_t *scaled, void *stream);

/* ------------------------------------------------------- HE matrix product */
/* matrix_gpu::Matrix (matrix.hpp:9-24, matrix.cu:48-81).  create: `input` is
 * host [blocks][2][primes][2^log_n] ciphertexts in coefficient form
 * (canonical), kept on the device in NTT form.  evaluate: `ring` is host
 * [blocks][2^log_n] ring-2^59 words (MATRIX_GPU_RING above 2^59 - 1); the
 * result out[c][k][z] = INTT(sum_b NTT(ct_b[c][k]) (.) NTT(lift(ring_b))[k])
 * is written to host [2][primes][2^log_n].  With `targets` (1..512 strictly
 * increasing coefficient indices, evaluate_selective) the c0 coefficients
 * outside the targets are zero.  evaluate_device: the same on device buffers,
 * asynchronous on `stream`, full output.  reserve + evaluate_device_batch:
 * `groups` independent evaluations in one call (the loop the reference runs as
 * one Matrix::evaluate per output group, bfv_matrix.inc:101-105), rings
 * [groups][blocks][2^log_n] and out [groups][2][primes][2^log_n], both
 * 16-byte aligned device buffers; reserve(groups) allocates the batch scratch
 * once (MATRIX_GPU_BATCH above the reserved count or 4096,
 * MATRIX_GPU_BATCH_RESERVED on a larger second reserve).  Errors
 * MATRIX_GPU_SHAPE, MATRIX_GPU_TARGET_COUNT, MATRIX_GPU_TARGET_INDEX,
 * MATRIX_GPU_ALIGNMENT, E_NTT_CANONICAL_REQUIRED; a device error poisons the
 * plan. */
typedef struct praghip_matrix_plan praghip_matrix_plan;
int praghip_matrix_plan_create(int device, const uint64_t *q, size_t primes, uint32_t log_n, const uint64_t *input,
                               size_t blocks, praghip_matrix_plan **plan);
int praghip_matrix_evaluate(praghip_matrix_plan *plan, const uint64_t *ring, uint64_t *output,
                            const uint64_t *targets, size_t count);
int praghip_matrix_evaluate_device(praghip_matrix_plan *plan, const uint64_t *ring, uint64_t *output, void *stream);
int praghip_matrix_reserve(praghip_matrix_plan *plan, size_t groups);
int praghip_matrix_evaluate_device_batch(praghip_matrix_plan *plan, const uint64_t *rings, uint64_t *output,
                                         size_t groups, void *stream);
/* evaluate_selective for a batch, on the device (matrix.cu:65-81 with the
 * gather_c0 kernel of matrix.cu:41-44): as evaluate_device_batch, then c0 of
 * every group keeps only the `count` target coefficients `targets` (host,
 * 1..512 strictly increasing indices < 2^log_n; MATRIX_GPU_TARGET_COUNT,
 * MATRIX_GPU_TARGET_INDEX) and is zero elsewhere; c1 is complete.  selected
 * (device [groups][primes][count], 16-byte aligned, or NULL) receives the
 * gathered target coefficients of c0. */
int praghip_matrix_evaluate_device_batch_selective(praghip_matrix_plan *plan, const uint64_t *rings,
                                                   uint64_t *output, size_t groups, const uint64_t *targets,
                                                   size_t count, uint64_t *selected, void *stream);
size_t praghip_matrix_device_bytes(const praghip_matrix_plan *plan);
int praghip_matrix_close(praghip_matrix_plan *plan, praghip_cleanup *out);
void praghip_matrix_destroy(praghip_matrix_plan *plan);

/* Packing of a matrix product (prag::MatrixPacking, matrix_packing and
 * matrix_packing_qk_reverse64 at native/include/prag/bfv_layout.hpp:8-27,
 * called from bfv_matrix.inc:9 and bfv.cpp:689): for `batch` rows, `inner`
 * terms and `outputs` columns, the reduction width, output columns per
 * returned ciphertext, returned ciphertexts and input ciphertexts of the
 * cheapest packing (bytes = inputs x 1,572,960 + returns x 786,528; ties take
 * the smallest width).  E_MATRIX_SHAPE unless 1 <= batch <= 16,
 * 1 <= inner <= 8192, 1 <= outputs <= 155,648; qk_reverse64 != 0 is the
 * dedicated K = 128, one-output layout {128, 1, 1, 1} (E_QK_REVERSE64_SHAPE
 * unless 1 <= batch <= 64).  Host only. */
typedef struct praghip_matrix_packing_t {
  uint64_t reduction, columns, returns, inputs;
} praghip_matrix_packing_t;
int praghip_matrix_packing(size_t batch, size_t inner, size_t outputs, int qk_reverse64,
                           praghip_matrix_packing_t *out);

/* ------------------------------------------- public-key encryption of zero */
/* prag::enc0_gpu::PublicZero (enc0.hpp:15-25, enc0.cu:99-114): create takes
 * the K = data_primes + 1 key-level primes and the public key pk [2][K][N] in
 * NTT form (host, canonical).  evaluate takes one encryption's samples
 * [3][K][N] (u ternary, e0, e1, as residues; E_ENC0_SAMPLE_CANONICAL) and
 * writes out[c] = ModDown(INTT(NTT(u) (.) pk_c) + e_c), host [2][L][N], then
 * wipes every device intermediate.  evaluate_device: the same on device
 * buffers (samples [3][K][N], out [2][L][N]), asynchronous on `stream`.
 * reserve + evaluate_device_batch: `count` encryptions in one call (the
 * per-ciphertext loop of enc0.cu:99-114 callers), samples [count][3][K][N]
 * and out [count][2][L][N], 16-byte aligned device buffers; reserve(count)
 * allocates the batch scratch once (E_ENC0_BATCH above the reserved count or
 * 4096, E_ENC0_BATCH_RESERVED on a larger second reserve).  Errors as Switch
 * (E_SWITCH_SHAPE, E_SWITCH_CLOSED) and E_ENC0_ALIGNMENT; a device error
 * poisons the plan. */
typedef struct praghip_enc0_plan praghip_enc0_plan;
int praghip_enc0_plan_create(int device, const uint64_t *q, size_t data_primes, uint32_t log_n, const uint64_t *pk,
                             praghip_enc0_plan **plan);
int praghip_enc0_evaluate(praghip_enc0_plan *plan, const uint64_t *samples, uint64_t *output);
int praghip_enc0_evaluate_device(praghip_enc0_plan *plan, const uint64_t *samples, uint64_t *output, void *stream);
int praghip_enc0_reserve(praghip_enc0_plan *plan, size_t count);
int praghip_enc0_evaluate_device_batch(praghip_enc0_plan *plan, const uint64_t *samples, uint64_t *output,
                                       size_t count, void *stream);
int praghip_enc0_close(praghip_enc0_plan *plan, praghip_cleanup *out);
void praghip_enc0_destroy(praghip_enc0_plan *plan);

/* ------------------------------------------------------ token-resident path */
/* prag::experimental::resident::TokenWeights (resident.hpp:20-45,
 * resident.cu:104-195, resident/seal_adapter.cpp:22-61), generalised over
 * primes, slots, blocks and block width (the reference: 6 locked primes,
 * <= 4 slots, 19 blocks of 8192).
 * create: `input` is host [blocks][slots][2][primes][N] ciphertexts in
 *   coefficient form (the adapter's flat order, seal_adapter.cpp:27-33),
 *   canonical; the plan transforms them to NTT form on the device.  `levels`
 *   sizes the per-slot stack (levels + 1 ciphertexts).  Errors
 *   E_GPU_TOKEN_CONTEXT_LAYOUT (shape, non-canonical input), E_NTT_CONTEXT.
 * evaluate (resident.cu:135-151): ring host [blocks][width] ring-2^59 words,
 *   each |w| <= 2^20 as a signed value (E_RESIDENT_WEIGHT_SHAPE,
 *   E_RESIDENT_WEIGHT_BOUND); output host [slots][2][primes][N], NTT form:
 *   sum_b NTT(ct_b) (.) NTT(lift_rev(ring_b)).
 * bind_local_shares (seal_adapter.cpp:54-60, resident.cu:126-132): host
 *   [slots][blocks * width] words < 2^59, once (E_LOCAL_BINDING).
 * evaluate_finished (seal_adapter.cpp:43-53): `local` host [slots] plaintext
 *   words m < 2^59; *view receives a device pointer to [slots][2][primes][N]
 *   coefficient-form results  x^-(width-1) (INTT(product) + Delta m x^(width-1))
 *   valid until the next evaluation.  evaluate_local_finished
 *   (seal_adapter.cpp:61): m from the bound shares' local dot product with the
 *   ring words on the device (E_RESIDENT_LOCAL_SHAPE when none are bound).
 * evaluate_device (resident.cu:152-173): device ring [blocks][width] (not
 *   range-checked), device residues [slots][primes] (the scaled local terms)
 *   or NULL for the bound shares, device output [slots][2][primes][N];
 *   asynchronous on `stream`.
 * stack_store / stack_view / download (resident.cu:174-191): a view is a
 *   device pointer to one [2][primes][N] ciphertext; store copies it into
 *   stack[slot][level] on `stream` (the stream that produced the view; the
 *   reference waits on the view's ready event) (E_DEVICE_STACK_VIEW), view returns stack[slot][level]
 *   (E_DEVICE_STACK_INDEX), download copies a view inside `finished` or the
 *   stack to host (E_DEVICE_DOWNLOAD_VIEW).  All three wait for completion. */
typedef struct praghip_token_plan praghip_token_plan;
int praghip_token_plan_create(int device, const uint64_t *q, size_t primes, uint32_t log_n, size_t slots,
                              size_t blocks, size_t width, size_t levels, const uint64_t *input,
                              praghip_token_plan **plan);
int praghip_token_evaluate(praghip_token_plan *plan, const uint64_t *ring, size_t words, uint64_t *output);
int praghip_token_bind_local_shares(praghip_token_plan *plan, const uint64_t *shares, size_t words);
int praghip_token_evaluate_finished(praghip_token_plan *plan, const uint64_t *ring, size_t words,
                                    const uint64_t *local, const uint64_t **view);
int praghip_token_evaluate_local_finished(praghip_token_plan *plan, const uint64_t *ring, size_t words,
                                          const uint64_t **view);
int praghip_token_evaluate_device(praghip_token_plan *plan, const uint64_t *ring, const uint64_t *residues,
                                  uint64_t *output, void *stream);
/* Batched evaluate_device: the per-coordinate calls of the token loop
 * (bfv_token_batch.inc:186-192, one resident.cu:152-173 evaluation each) for
 * `coords` columns at once,
 * rings device [coords][blocks][width], residues device
 * [coords][slots][primes] or NULL (bound shares), output device
 * [coords][slots][2][primes][N]; each column's result equals its
 * evaluate_device result.  The resident inputs are read once per group of
 * columns instead of once per column.  reserve(coords) allocates the batch
 * scratch once (E_RESIDENT_BATCH_RESERVED when asked to grow it later);
 * evaluate_device_batch takes coords <= the reserved count (E_RESIDENT_BATCH). */
int praghip_token_reserve(praghip_token_plan *plan, size_t coords);
int praghip_token_evaluate_device_batch(praghip_token_plan *plan, const uint64_t *rings, const uint64_t *residues,
                                        uint64_t *output, size_t coords, void *stream);
int praghip_token_stack_store(praghip_token_plan *plan, size_t slot, unsigned level, const uint64_t *view,
                              void *stream);
int praghip_token_stack_view(praghip_token_plan *plan, size_t slot, unsigned level, const uint64_t **view);
int praghip_token_download(praghip_token_plan *plan, const uint64_t *view, uint64_t *output);
/* stack_store and download with the view's ready event, as the reference's
 * DeviceCipherBatch carries one (resident.hpp:17-20; resident.cu:176-179,
 * 187-189): `ready` is a hipEvent_t recorded after the producer's writes
 * (required: E_DEVICE_STACK_VIEW / E_DEVICE_DOWNLOAD_VIEW when NULL); the
 * plan's own stream waits on it, copies, and the call waits for the copy. */
int praghip_token_stack_store_ready(praghip_token_plan *plan, size_t slot, unsigned level, const uint64_t *view,
                                    void *ready);
int praghip_token_download_ready(praghip_token_plan *plan, const uint64_t *view, void *ready, uint64_t *output);
int praghip_token_timing(const praghip_token_plan *plan, praghip_timing *out);
/* TokenWeights::timing (resident.hpp:11-12, resident.cu:165-166,183-184):
 * per-phase times of the last host-buffer evaluation (praghip_token_phases). */
int praghip_token_phase_timing(const praghip_token_plan *plan, praghip_token_phases *out);
int praghip_token_close(praghip_token_plan *plan, praghip_cleanup *out);
void praghip_token_destroy(praghip_token_plan *plan);

/* ------------------------------------------------------- acyclic packing */
/* prag::experimental_full_switch::Packing (bfv_gpu_packing.hpp:10-45) over
 * the keys of bfv_acyclic_pack.hpp:23-42: `keys` is host
 * [levels][2][dnum][2][data_primes+1][N] NTT form; key [l][0] switches element
 * 1 and key [l][1] element 2^(l+1) + 1 (the reference: 9 levels, dnum = 6;
 * E_PACK_KEY_LEVELS for levels outside 1..log_n).  A pair at level l is
 *   ks_{l,0}(L + x^s R) + ks_{l,1}(sigma_g(L - x^s R)),  s = N >> (l+1)
 * (switch.cu:49-61,157-185), ciphertexts [2][data_primes][N] in coefficient
 * form.  max_pairs bounds the pairs one batched keyswitch takes (scratch
 * about 9.5 x 2 L N x 8 bytes per pair).
 * pair (Packing::pair, bfv_gpu_packing.hpp:20-32): host ciphertexts,
 *   synchronous (E_PACK_LEVEL, E_PACK_CIPHERTEXT, E_PACK_CLOSED).
 * pair_device (Packing::pair_device, bfv_gpu_packing.hpp:33-37): `count`
 *   pairs at one level, device [count][2][L][N] each, output not overlapping
 *   the inputs (E_PACK_DEVICE_LEVEL, E_PACK_DEVICE_VIEW); asynchronous.
 * tree_device: the stack merge of bfv_token_batch.inc:194-206 for `leaves`
 *   (a power of two, <= 2^levels) consecutive coordinates at once, level by
 *   level: `nodes` device [leaves][slots][2][L][N] is reduced in place and the
 *   root of slot s is left in nodes[0][s].  Bit-identical to merging the
 *   leaves one by one through the stack; every level is one batched call. */
typedef struct praghip_pack_plan praghip_pack_plan;
int praghip_pack_plan_create(int device, const uint64_t *q, size_t data_primes, uint32_t log_n, size_t dnum,
                             size_t levels, const uint64_t *keys, size_t max_pairs, praghip_pack_plan **plan);
int praghip_pack_pair(praghip_pack_plan *plan, const uint64_t *left, const uint64_t *right, unsigned level,
                      uint64_t *output);
int praghip_pack_pair_device(praghip_pack_plan *plan, const uint64_t *left, const uint64_t *right, size_t count,
                             unsigned level, uint64_t *output, void *stream);
int praghip_pack_tree_device(praghip_pack_plan *plan, uint64_t *nodes, size_t leaves, size_t slots, void *stream);
int praghip_pack_merges(const praghip_pack_plan *plan, uint64_t *merges);
/* packed_target (bfv_acyclic_pack.hpp:53-56): the coefficient on which
 * coordinate `coordinate` (its low `levels` bits) lands after a packing tree of
 * `levels` levels at N = 2^log_n: those bits reversed, times N >> levels (the
 * reference: levels 9, log_n 14, spacing 32).  E_PACK_KEY_LEVELS unless
 * 1 <= levels <= log_n <= 14.  Host only. */
int praghip_packed_target(size_t coordinate, unsigned levels, uint32_t log_n, uint64_t *target);
int praghip_pack_timing(const praghip_pack_plan *plan, praghip_timing *out);
int praghip_pack_close(praghip_pack_plan *plan, praghip_cleanup *out);
void praghip_pack_destroy(praghip_pack_plan *plan);

/* ------------------------------------------------------------ weight files */
/* The quantized_f12 int32 .npy weights (quantize_weights.py:60-64), read as
 * MappedWeights does (artifacts.hpp:31-49): memory-mapped, version 1/2, '<i4',
 * C order, exactly [rows][cols] ([rows] with vector != 0).  Errors: BAD_SHAPE,
 * E_WEIGHT_FILE, E_WEIGHT_MAP, E_NPY_FORMAT, E_NPY_SHAPE.  at(): the ring word
 * of artifacts.hpp:86-92 (sign-extended, & (2^59-1)).  upload(): copies the
 * int32 [rows][cols] tensor to device memory (praghip_share_gemm, w_bits 32)
 * and waits for the copy. */
typedef struct praghip_weights praghip_weights;
int praghip_weights_open(const char *path, size_t rows, size_t cols, int vector, praghip_weights **out);
int praghip_weights_shape(const praghip_weights *w, size_t *rows, size_t *cols);
const int32_t *praghip_weights_data(const praghip_weights *w);
int praghip_weights_at(const praghip_weights *w, size_t row, size_t col, uint64_t *word);
int praghip_weights_max_abs(const praghip_weights *w, uint64_t *max_abs);
int praghip_weights_upload(const praghip_weights *w, int device, int32_t *dst, void *stream);
/* The file's weights split on the host into the three signed-byte planes of
 * praghip_share_gemm's w_bits 24 and copied to dst (device int8
 * [3][rows][cols]); waits for the copy.  E_WEIGHT_RANGE when a weight lies
 * outside [-0x808080, 0x7F7F7F]. */
int praghip_weights_upload_split(const praghip_weights *w, int device, int8_t *dst, void *stream);
void praghip_weights_close(praghip_weights *w);

/* ------------------------------------------------------------- frames */
/* The 96-byte public frame header of the reference's Channel
 * (native/src/channel.cpp:122-150): "PRGCF001", session[16], config[32], then
 * big-endian u64 sequence, payload bytes, stage, operation and version 1.  A
 * ciphertext frame's payload is the [component][prime][N] little-endian u64
 * layout of every entry point here (2 x 6 x 16384 x 8 = 1,572,864 bytes for
 * a full ciphertext).  encode (send_data): out[96].  decode: the fields of a
 * header with the magic and version 1 (E_FRAME_BINDING otherwise).  check
 * (recv_data): E_FRAME_BINDING unless every field equals `expect`.  Host
 * only. */
typedef struct praghip_frame_header {
  uint8_t session[16];
  uint8_t config[32];
  uint64_t sequence, size, stage, operation;
} praghip_frame_header;
int praghip_frame_encode(const praghip_frame_header *header, uint8_t *out);
int praghip_frame_decode(const uint8_t *in, praghip_frame_header *header);
int praghip_frame_check(const uint8_t *in, const praghip_frame_header *expect);

/* ------------------------------------------------------ synthetic inputs */
/* Seeded counter-based inputs (no counterpart in the reference, whose probes
 * draw from mt19937_64, check_resident.cpp:26): element i of the buffer is
 * splitmix64(seed + (i+1)*0x9E3779B97F4A7C15).  Residues: mulhi(z, q[limb % primes])
 * over device [limbs][2^log_n]; u64: z; int8: mulhi(z, 255) - 127; shifts: mulhi(z, 8). */
int praghip_fill_residues(int device, uint64_t *data, size_t limbs, uint32_t log_n, const uint64_t *q,
                          size_t primes, uint64_t seed, void *stream);
int praghip_fill_u64(int device, uint64_t *data, size_t count, uint64_t seed, void *stream);
int praghip_fill_i8(int device, int8_t *data, size_t count, uint64_t seed, void *stream);
int praghip_fill_shift(int device, int8_t *data, size_t count, uint64_t seed, void *stream);  /* mulhi(z, 8) */

#ifdef __cplusplus
}
#endif
#endif /* PRAGHIP_H */
