/*
 * m3_hip.h - thin C ABI over the HIP runtime and the gfx950 kernels of the
 * m3 HIP execution provider.
 *
 * This is the boundary the C11 host code binds. It takes plain pointers,
 * sizes and POD view blocks; no m3 or torch types cross it. Every function
 * returns an m3_hip_code and, on failure, writes a NUL-terminated message of
 * at most `capacity` bytes into `message` (which may be NULL).
 *
 * Each entry point replaces one piece of the Metal provider of
 * taconotsandwich/m3.c:
 *   m3_hip_device_open/close     <- m3_backend_create_metal and
 *                                   m3_metal_destroy (src/m3_backend_metal.m:
 *                                   234-296, :44-58): device, queue, library
 *   m3_hip_arena_reserve/release <- m3_metal_allocate/m3_metal_free
 *                                   (src/m3_backend_metal.m:60-96); one
 *                                   hipMalloc per session instead of one
 *                                   shared MTLBuffer per slot
 *   m3_hip_copy_h2d/d2h          <- memcpy into shared storage in
 *                                   m3_storage_write/read (src/m3_backend.c:
 *                                   319-366); unified memory does not exist
 *                                   here, so these are the explicit copies
 *   m3_hip_launch_binary         <- m3_metal_encode_binary
 *                                   (src/m3_backend_metal_basic.m:354-395),
 *                                   kernels m3_add/m3_mul (:66-104)
 *   m3_hip_launch_cast/copy      <- m3_metal_encode_unary (:326-352),
 *                                   kernels m3_cast/m3_copy (:29-63)
 *   m3_hip_launch_softmax        <- m3_metal_encode_softmax (:397-433),
 *                                   kernel m3_softmax (:105-147)
 *   m3_hip_launch_snake1d        <- m3_metal_encode_snake1d, kernel
 *                                   m3_snake1d (:150-177)
 *   m3_hip_launch_tanh           <- m3_metal_encode_tanh (:478-511),
 *                                   kernel m3_tanh (:178-...); host
 *                                   semantics src/m3_op_execute_basic.c:
 *                                   217-229
 *   m3_hip_launch_gated_silu     <- m3_metal_encode_gated_silu
 *                                   (src/m3_backend_metal_dense.m:478-533),
 *                                   kernel m3_gated_silu
 *                                   (src/m3_backend_metal_dense_kernels.m:
 *                                   416-...); host semantics
 *                                   src/m3_op_execute_basic.c:104-122
 *   m3_hip_scan_views            <- the host data preflight Metal runs on
 *                                   shared memory before commit
 *                                   (src/m3_backend_metal_basic.m:274-302,
 *                                   src/m3_op_data_preflight.c:8-64)
 *   m3_hip_synchronize           <- commit + waitUntilCompleted
 *                                   (src/m3_backend_metal.m:210-216)
 *   m3_hip_prepare_program       no counterpart: compiles a program's
 *                                   kernel ahead of its first launch
 *   m3_hip_launch_program        no counterpart: runs a run of ADD/SUB/
 *                                   MUL/DIV commands (per-element semantics
 *                                   of src/m3_op_execute_basic.c:61-77) that
 *                                   the session compiler fused into one
 *                                   elementwise program
 *
 * All launches of one device go to that device's single HIP stream, in call
 * order, so a command list executes in order and m3_hip_synchronize waits
 * for all of it. A device handle is not thread-safe.
 */
#ifndef M3_HIP_H
#define M3_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M3_HIP_MAX_RANK 8U

typedef enum {
    M3_HIP_OK = 0,
    M3_HIP_INVALID = 1,      /* malformed argument or view block */
    M3_HIP_NO_DEVICE = 2,    /* no usable HIP device */
    M3_HIP_OUT_OF_MEMORY = 3,
    M3_HIP_RUNTIME = 4,      /* the HIP runtime reported an error */
    M3_HIP_UNSUPPORTED = 5   /* valid request this library cannot run */
} m3_hip_code;

/* Element types; values equal m3_dtype. */
typedef enum {
    M3_HIP_F32 = 0,
    M3_HIP_F16 = 1,
    M3_HIP_BF16 = 2,
    M3_HIP_I32 = 3
} m3_hip_dtype;

typedef enum {
    M3_HIP_ADD = 0,
    M3_HIP_MUL = 1,
    M3_HIP_SUB = 2,
    M3_HIP_DIV = 3
} m3_hip_binary_op;

typedef enum {
    M3_HIP_SCAN_NAN = 0,        /* flag when any element is NaN */
    M3_HIP_SCAN_I32_RANGE = 1   /* flag when any element is non-finite or
                                   outside [-2^31, 2^31) */
} m3_hip_scan_kind;

/* A strided tensor view over device memory. Element (i0, ..., ir-1) lives at
 * base + byte_offset + sum(ik * byte_strides[k]). element_count is the
 * product of shape[0..rank). Output views must be contiguous. The layout
 * matches M3ViewParameters of the reference (src/m3_backend_metal_helpers.h:
 * 12-19) plus the base pointer. */
typedef struct {
    void *base;
    uint64_t byte_offset;
    uint64_t element_count;
    uint64_t shape[M3_HIP_MAX_RANK];
    uint64_t byte_strides[M3_HIP_MAX_RANK];
    uint32_t rank;
    uint32_t dtype;
} m3_hip_view;

typedef struct m3_hip_device m3_hip_device;

/* Per-kernel timing gathered with HIP events on the device stream. */
typedef struct {
    char name[48];
    uint64_t launches;
    double total_ms;
} m3_hip_kernel_time;

int m3_hip_device_count(int *count, char *message, size_t capacity);
int m3_hip_device_open(int ordinal, m3_hip_device **device,
                       char *message, size_t capacity);
void m3_hip_device_close(m3_hip_device *device);
int m3_hip_device_properties(const m3_hip_device *device, char *name,
                             size_t name_capacity, uint64_t *total_bytes,
                             uint32_t *compute_units, char *message,
                             size_t capacity);

/* One hipMalloc of byte_count bytes (256-byte aligned). */
int m3_hip_arena_reserve(m3_hip_device *device, size_t byte_count,
                         void **base, char *message, size_t capacity);
void m3_hip_arena_release(m3_hip_device *device, void *base);

/* Stream-ordered copies. Both return once the host buffer may be reused
 * (h2d) or holds the data (d2h). A host-to-device copy of at most 256
 * bytes (a scalar the host rewrites between commands) travels in a
 * kernel's arguments and does not wait for the stream; a larger one waits
 * for the copy to complete. */
int m3_hip_copy_h2d(m3_hip_device *device, void *device_destination,
                    const void *host_source, size_t byte_count,
                    char *message, size_t capacity);
int m3_hip_copy_d2h(m3_hip_device *device, void *host_destination,
                    const void *device_source, size_t byte_count,
                    char *message, size_t capacity);
/* Fills device memory with zero bytes using a kernel (no memset node). */
int m3_hip_fill_zero(m3_hip_device *device, void *device_destination,
                     size_t byte_count, char *message, size_t capacity);

/* out = left (op) right with right-aligned broadcasting, computed in F32
 * and rounded once to the output dtype. Inputs F32/F16/BF16, any strides;
 * output contiguous; an output may alias an input of the same shape exactly. */
int m3_hip_launch_binary(m3_hip_device *device, uint32_t op,
                         const m3_hip_view *left, const m3_hip_view *right,
                         const m3_hip_view *output, char *message,
                         size_t capacity);
/* Element conversion between any two of F32/F16/BF16/I32 (same dtype is a
 * copy). Float to I32 truncates; callers scan the input first. */
int m3_hip_launch_cast(m3_hip_device *device, const m3_hip_view *input,
                       const m3_hip_view *output, char *message,
                       size_t capacity);
/* Byte copy of a strided input into a contiguous output of the same dtype. */
int m3_hip_launch_copy(m3_hip_device *device, const m3_hip_view *input,
                       const m3_hip_view *output, char *message,
                       size_t capacity);
/* Last-axis softmax of a float tensor without NaN. */
int m3_hip_launch_softmax(m3_hip_device *device, const m3_hip_view *input,
                          const m3_hip_view *output, char *message,
                          size_t capacity);
/* Snake1d on rank-3 F32: y = x + (1/(a+eps)) * sin(a*x)^2, a per channel. */
int m3_hip_launch_snake1d(m3_hip_device *device, const m3_hip_view *input,
                          const m3_hip_view *alpha,
                          const m3_hip_view *output, char *message,
                          size_t capacity);

/* out = tanhf(input) on F32 of rank 1 to 8; any input strides, output
 * contiguous, exact in-place allowed. */
int m3_hip_launch_tanh(m3_hip_device *device, const m3_hip_view *input,
                       const m3_hip_view *output, char *message,
                       size_t capacity);
/* out = round_gate(gate / (1 + expf(-gate))) * up, where round_gate rounds
 * through the gate's dtype; gate, up and output of one shape (no
 * broadcast), each F32/F16/BF16; any input strides, output contiguous,
 * exact aliases allowed. */
int m3_hip_launch_gated_silu(m3_hip_device *device, const m3_hip_view *gate,
                             const m3_hip_view *up,
                             const m3_hip_view *output, char *message,
                             size_t capacity);

/* Elementwise program: a run of ADD/SUB/MUL/DIV and float-to-float CAST
 * (or F32 COPY) operations over one element space of `count` elements,
 * executed per element with the intermediate values in registers as F32.
 * Layout of the 32-bit words:
 *   [0] M3_HIP_PROGRAM_MAGIC
 *   [1] P, operand count (at most M3_HIP_PROGRAM_MAX_OPERANDS)
 *   [2] I, instruction word count (at most M3_HIP_PROGRAM_MAX_WORDS)
 *   [3] count, low 32 bits     [4] count, high 32 bits
 *   [5] K, number of periodic operands (at most P)
 *   [6..7] zero
 *   [8 .. 8+2P) operand p: device address, low word then high word. Bits
 *       30-31 of the high word: the element dtype (M3_HIP_F32, M3_HIP_F16
 *       or M3_HIP_BF16). Bit 0 of the low word set: a scalar, one element
 *       read by every element (aligned to its size). Clear: an array of
 *       `count` elements (16-byte aligned for F32, 8-byte for 16-bit),
 *       element e at address + e * size, unless the operand is periodic.
 *   [8+2P .. 8+2P+2K) periodic operands: pairs (operand index, period
 *       M). Element e of that array operand is at index e mod M: a
 *       trailing-axis broadcast of an M-element tensor. M is a multiple of
 *       4 that divides `count` (so every group of 4 elements lies within
 *       one period); operand indices increase strictly.
 *   [8+2P+2K .. 8+2P+2K+I) instructions.
 * Registers per element: values R0..R3 and fetched operands F0..F3.
 * Instructions (bits 0-1 opcode):
 *   FETCH (two words): bits 2-3 n-1; the second word holds operand
 *       indices f0..f{n-1} in its bytes 0..n-1. Loads array (or periodic)
 *       operand fk, converted to F32, into Fk for k < n; all n loads are
 *       issued together.
 *   OP: bits 2-3 the m3_hip_binary_op; bits 4-5 destination R; bits 8-11
 *       left source, bits 12-15 right source (0-3: R0-R3, 4-7: F0-F3,
 *       8: the scalar operand in bits 16-23); bits 24-25 a rounding dtype.
 *       dst = left (op) right as one F32 operation with the reference's
 *       NaN rules, then rounded through the rounding dtype (F16/BF16: the
 *       value a store to it and a load back give; F32: unchanged).
 *   ROUND: bits 4-5 destination R; bits 8-11 source (as OP's left, scalar
 *       index in bits 16-23); bits 24-25 the dtype. dst = source rounded
 *       through the dtype (a CAST; F32 makes it a move).
 *   STORE: bits 4-5 source R; bits 8-15 array operand (not periodic);
 *       writes the value converted to the operand's dtype.
 * m3_hip_launch_program checks the words on the host (magic, counts,
 * indices, operand kinds, dtypes and alignment) before launching;
 * device_words must hold the same words in device memory. */
#define M3_HIP_PROGRAM_MAGIC 0x4d335031U /* "M3P1" */
#define M3_HIP_PROGRAM_HEADER_WORDS 8U
#define M3_HIP_PROGRAM_MAX_OPERANDS 255U
#define M3_HIP_PROGRAM_MAX_WORDS 4096U

typedef enum {
    M3_HIP_PROGRAM_FETCH = 0,
    M3_HIP_PROGRAM_OP = 1,
    M3_HIP_PROGRAM_STORE = 2,
    M3_HIP_PROGRAM_ROUND = 3
} m3_hip_program_opcode;

/* Checks the words like m3_hip_launch_program and compiles the program's
 * generated kernel into the device's cache without launching anything, so
 * that the first launch does not pay for the compilation (session
 * creation calls it for every program). Returns M3_HIP_OK also when
 * runtime compilation is off or fails: the launch then runs the
 * interpreter. */
int m3_hip_prepare_program(m3_hip_device *device, const uint32_t *words,
                           size_t word_count, char *message,
                           size_t capacity);
int m3_hip_launch_program(m3_hip_device *device, const uint32_t *words,
                          const void *device_words, size_t word_count,
                          char *message, size_t capacity);

/* Scans view i for the condition kinds[i] (an m3_hip_scan_kind), waits, and
 * writes flags[i] = 1 when view i holds an offending element, else 0. */
int m3_hip_scan_views(m3_hip_device *device, const uint32_t *kinds,
                      const m3_hip_view *views, size_t count,
                      uint32_t *flags, char *message, size_t capacity);

/* m3_hip_scan_views in two halves, so that a scan can run while the host
 * does other work: _begin queues the same scan and returns at once with a
 * ticket; _collect waits for the scan with that ticket and writes its
 * flags. Only the last started scan of a device can be collected (another
 * _begin replaces it; blocking scans in between do not). The caller keeps
 * the views unchanged until the scan is collected or discarded. */
int m3_hip_scan_views_begin(m3_hip_device *device, const uint32_t *kinds,
                            const m3_hip_view *views, size_t count,
                            uint32_t *ticket, char *message, size_t capacity);
int m3_hip_scan_views_collect(m3_hip_device *device, uint32_t ticket,
                              size_t count, uint32_t *flags, char *message,
                              size_t capacity);

/* No counterpart in the reference. m3_hip_scan_views for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same scan and results, with the
 * per-view flag words in a static device array of M3_HIP_STATIC_SCAN_VIEWS
 * words (256 bytes on each GPU, held until the process ends) instead of
 * memory the library allocates on first use. It calls no hipMalloc,
 * hipFree or other allocating routine and records no timing events. More
 * than M3_HIP_STATIC_SCAN_VIEWS views is M3_HIP_UNSUPPORTED. Every call on
 * one GPU, from any device handle, shares the array and clears the words
 * it uses first; a host-side flag per GPU admits one call at a time, and a
 * call made while another one on the same GPU has not returned is refused
 * with M3_HIP_UNSUPPORTED ("in use by another call") instead of racing. */
#define M3_HIP_STATIC_SCAN_VIEWS 64U
int m3_hip_scan_views_static(m3_hip_device *device, const uint32_t *kinds,
                             const m3_hip_view *views, size_t count,
                             uint32_t *flags, char *message,
                             size_t capacity);

/* Waits for all work on the device stream and reports any kernel error. */
int m3_hip_synchronize(m3_hip_device *device, char *message,
                       size_t capacity);

/* How many device and pinned host allocations this library has made in
 * the process (every hipMalloc and hipHostMalloc it calls), for tests that
 * show an entry point allocates nothing. No counterpart in the reference. */
int m3_hip_allocation_count(uint64_t *count);

/* How many times the host has waited for the device's stream (stream
 * synchronizations and completion polls, data-scan readbacks, blocking
 * copies) since the device was opened; for tests and measurement. No
 * counterpart in the reference. */
int m3_hip_host_waits(const m3_hip_device *device, uint64_t *waits);

/* Device-side gating of the rest of a command list, so that a list whose
 * checked input (a softmax input, a float-to-I32 cast input) an earlier
 * command of the same list produces runs with one host wait, at its end.
 * The reference's Metal provider rejects such a list
 * (src/m3_backend_metal_basic.m:274-302) and its CPU provider checks the
 * input right before the command (src/m3_op_execute_host.c:5-60); these
 * calls give the CPU provider's order without a mid-list wait:
 *   m3_hip_gate_open   every command kernel launched from here until
 *                      m3_hip_gate_close returns at its start, touching no
 *                      tensor, once a check of this gate has failed;
 *                      idempotent while open;
 *   m3_hip_gate_check  queues, in stream order, the data scan of `view`
 *                      for `kind` (M3_HIP_SCAN_NAN, M3_HIP_SCAN_I32_RANGE)
 *                      and closes the gate when it finds an offending
 *                      element; the first failing check of a gate is the
 *                      one kept;
 *   m3_hip_gate_close  waits for the stream once and ends the gating;
 *                      *failed_kind receives 0 when every check passed,
 *                      else 1 + the kind of the first failing check.
 * A NaN check of a program's output can also be made by the program as it
 * stores it, in place of m3_hip_gate_check's scan:
 *   m3_hip_launch_program_checked  launches the program like
 *                      m3_hip_launch_program; when a gate is open, `kind`
 *                      is M3_HIP_SCAN_NAN and `checked` is the whole of an
 *                      operand that the program stores once (contiguous,
 *                      its address, dtype and element count), the program
 *                      also records whether a value it stores there is NaN
 *                      and *fused receives 1, else 0 (then queue the check
 *                      with m3_hip_gate_check as usual);
 *   m3_hip_gate_pending  with `armed` 1, every command kernel launched
 *                      until the call with 0 returns at its start, closing
 *                      the gate, when the last fused check found a NaN:
 *                      arm it around the launches of the command whose
 *                      input was checked (the command right after the
 *                      program), which gives the order of a failing
 *                      m3_hip_gate_check queued before that command.
 * No counterpart in the reference's backend interface. */
int m3_hip_gate_open(m3_hip_device *device, char *message, size_t capacity);
int m3_hip_gate_check(m3_hip_device *device, uint32_t kind,
                      const m3_hip_view *view, char *message,
                      size_t capacity);
int m3_hip_gate_close(m3_hip_device *device, uint32_t *failed_kind,
                      char *message, size_t capacity);
int m3_hip_launch_program_checked(m3_hip_device *device,
                                  const uint32_t *words,
                                  const void *device_words, size_t word_count,
                                  uint32_t kind, const m3_hip_view *checked,
                                  int *fused, char *message, size_t capacity);
int m3_hip_gate_pending(m3_hip_device *device, int armed, char *message,
                        size_t capacity);

/* Measurement support: with `enabled` 1, every launch is bracketed by HIP
 * events on the device stream and each run waits on the stream (not on the
 * completion word); with 2, runs wait on the stream the same way but no
 * events are attached, for runs under an external kernel profiler; with 0,
 * neither. m3_hip_timing_read synchronizes, folds completed event pairs
 * into per-kernel totals, and copies up to `capacity` entries. */
int m3_hip_timing_enable(m3_hip_device *device, int enabled);
int m3_hip_timing_reset(m3_hip_device *device);
int m3_hip_timing_read(m3_hip_device *device, m3_hip_kernel_time *entries,
                       size_t capacity, size_t *count, char *message,
                       size_t message_capacity);
/* The durations (ms) of the completed launches of kernel `name` since the
 * last reset, in launch order (the first 4,096 are kept): *count receives
 * how many there are, and up to `capacity` are copied. Synchronizes like
 * m3_hip_timing_read. */
int m3_hip_timing_samples(m3_hip_device *device, const char *name,
                          float *durations_ms, size_t capacity,
                          size_t *count, char *message,
                          size_t message_capacity);
/* The device's hipStream_t, for callers that order their own work with it. */
void *m3_hip_stream(m3_hip_device *device);

#ifdef __cplusplus
}
#endif

#endif
