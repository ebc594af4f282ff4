/*
 * einsum_ir_hip.h -- C ABI of the MI355X (gfx950) execution backend for
 * einsum_ir's binary-contraction, permutation and tree hot path.
 *
 * Everything here is plain C: integer codes, int64 sizes/strides, raw device
 * pointers and an opaque plan handle.  The C++ operator classes
 * (BinaryContractionHip, UnaryHip, EinsumNode's device arena) sit on top of
 * these entry points; any other host language binds the same symbols.
 *
 * Conventions
 *   - Strides and sizes are in ELEMENTS, exactly as in the reference's loop IR
 *     `einsum_ir::basic::iter_property` (reference src/basic/constants.h:85-95).
 *   - All tensor pointers are device pointers (HBM).  A `stream` argument is a
 *     hipStream_t passed as void*; NULL means the null stream.
 *   - Every function returns an error code equal to einsum_ir::err_t
 *     (reference src/constants.h:33-46).  A human-readable reason for the last
 *     failure on the calling thread is returned by etir_hip_last_error().
 *   - Plans are immutable after creation; executing one plan concurrently on
 *     different streams is safe.  Execution never allocates memory.
 */
#ifndef EINSUM_IR_HIP_H
#define EINSUM_IR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* error codes: einsum_ir::err_t (reference src/constants.h:33-46) */
#define ETIR_SUCCESS                    0
#define ETIR_COMPILATION_FAILED         1
#define ETIR_DIMENSION_ORDERING_FAILED  2
#define ETIR_TENSOR_BLOCKING_FAILED     3
#define ETIR_NO_DATA_PTR_PROVIDED       4
#define ETIR_CALLED_BEFORE_COMPILATION  5
#define ETIR_INVALID_ID                 6
#define ETIR_INVALID_BACKEND            7
#define ETIR_INVALID_CPX_DIM            8
#define ETIR_INVALID_DTYPE              9
#define ETIR_INVALID_KTYPE             10
#define ETIR_UNDEFINED_ERROR           99

/* data types: einsum_ir::data_t (reference src/constants.h:48-52) plus the
 * additive value BF16 (the reference has no bf16; 2 is unused there). */
#define ETIR_FP32                       0
#define ETIR_FP64                       1
#define ETIR_BF16                       2
#define ETIR_UNDEFINED_DTYPE           99

/* kernel types: einsum_ir::kernel_t (reference src/constants.h:61-77) */
#define ETIR_KTYPE_ZERO                 0
#define ETIR_KTYPE_RELU                 1
#define ETIR_KTYPE_ADD                  2
#define ETIR_KTYPE_COPY                 3
#define ETIR_KTYPE_MADD                 4
#define ETIR_KTYPE_CPX_ZERO             6
#define ETIR_KTYPE_CPX_MADD             8
#define ETIR_KTYPE_UNDEFINED           99

/* dimension types: einsum_ir::dim_t (reference src/constants.h:9-18) */
#define ETIR_DIM_C                      0
#define ETIR_DIM_M                      1
#define ETIR_DIM_N                      2
#define ETIR_DIM_K                      3
#define ETIR_DIM_CPX                    4
#define ETIR_DIM_I                      5
#define ETIR_DIM_J                      6

typedef struct etir_plan_s * etir_plan_t;

/*
 * Creates a contraction plan from the loop IR of one binary contraction.
 *
 * Replaces the compile step of the reference's TPP path:
 *   BinaryContractionTpp::compile      (reference src/backend/BinaryContractionTpp.cpp:4-127)
 *   ContractionOptimizer::optimize     (reference src/basic/binary/ContractionOptimizer.cpp:47-74)
 *   ContractionBackend::compile        (reference src/basic/binary/ContractionBackend.cpp:122-249)
 *   ContractionBackendTpp::compile_kernels (reference src/basic/binary/ContractionBackendTpp.cpp:65-225)
 *
 * num_loops loops, each with a dimension type (ETIR_DIM_C/M/N/K), a size and
 * element strides in the left, right, auxiliary-output and output tensors
 * (the fields of iter_property).  strides_out_aux may be NULL when neither
 * touch kernel reads the auxiliary tensor.  Loops of type I/J are accepted and,
 * as in the reference lowering (BinaryContractionTpp.cpp:46-66 only emits
 * C/M/N/K loops), are not iterated.
 *
 * Supported dtypes: (left,right,comp,out) = (FP32,FP32,FP32,FP32),
 * (BF16,BF16,FP32,FP32), (BF16,BF16,FP32,BF16), (FP64,FP64,FP64,FP64).
 * Touch kernels: first in {ZERO, COPY, ADD, UNDEFINED}, main MADD,
 * last in {RELU, ADD, UNDEFINED} -- the set ContractionBackendTpp accepts
 * (ContractionBackendTpp.cpp:127-163).
 *
 * Complex contractions (the reference's CPX kernels, which it runs on its
 * BLAS backend: BinaryContractionBlas.cpp:68-85): main CPX_MADD, exactly one
 * loop of type ETIR_DIM_CPX with size 2 whose strides locate the imaginary
 * parts (0 = real, 1 = imaginary in every tensor), first touch ZERO, CPX_ZERO
 * or UNDEFINED (accumulate into the output), last touch UNDEFINED; FP32 or
 * FP64 throughout.
 *
 * The plan owns small device-resident offset tables (allocated here, never
 * during execution).
 */
int etir_hip_contraction_create( int64_t         num_loops,
                                 int32_t const * dim_types,
                                 int64_t const * sizes,
                                 int64_t const * strides_left,
                                 int64_t const * strides_right,
                                 int64_t const * strides_out_aux,
                                 int64_t const * strides_out,
                                 int32_t         dtype_left,
                                 int32_t         dtype_right,
                                 int32_t         dtype_comp,
                                 int32_t         dtype_out,
                                 int32_t         ktype_first_touch,
                                 int32_t         ktype_main,
                                 int32_t         ktype_last_touch,
                                 etir_plan_t   * plan );

/*
 * Enqueues one contraction on `stream`.  Replaces
 *   BinaryContractionTpp::contract     (reference src/backend/BinaryContractionTpp.cpp:129-146)
 *   ContractionBackend::contract       (reference src/basic/binary/ContractionBackend.cpp:251-294)
 * out_aux may be NULL unless a touch kernel reads it.  Asynchronous: errors of
 * the device work surface at the next synchronisation.
 */
int etir_hip_contraction_execute( etir_plan_t  plan,
                                  void const * left,
                                  void const * right,
                                  void const * out_aux,
                                  void       * out,
                                  void       * stream );

/*
 * Plans and executes one contraction without allocating device memory: the
 * arguments of etir_hip_contraction_create followed by those of
 * etir_hip_contraction_execute, with the same results.  No counterpart in
 * the reference: it is for callers that cannot allocate (code under stream
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * offset tables and any split-K workspace live in a fixed 64 MiB device
 * array per GPU (held until the process ends); a contraction that needs more
 * fails with an error naming both sizes.  All calls on one GPU share that
 * array: calls that overlap on one GPU (other streams, other host threads)
 * race.  Enqueued on `stream`; no host synchronisation.
 */
int etir_hip_contraction_execute_noalloc( int64_t         num_loops,
                                          int32_t const * dim_types,
                                          int64_t const * sizes,
                                          int64_t const * strides_left,
                                          int64_t const * strides_right,
                                          int64_t const * strides_out_aux,
                                          int64_t const * strides_out,
                                          int32_t         dtype_left,
                                          int32_t         dtype_right,
                                          int32_t         dtype_comp,
                                          int32_t         dtype_out,
                                          int32_t         ktype_first_touch,
                                          int32_t         ktype_main,
                                          int32_t         ktype_last_touch,
                                          void const    * left,
                                          void const    * right,
                                          void const    * out_aux,
                                          void          * out,
                                          void          * stream );

/*
 * Creates a permutation plan (the unary COPY/ZERO/ADD operator).
 * Replaces
 *   UnaryTpp::compile                  (reference src/backend/UnaryTpp.cpp:4-50)
 *   UnaryOptimizer::optimize           (reference src/basic/unary/UnaryOptimizer.cpp:12-67)
 *   UnaryBackend::compile              (reference src/basic/unary/UnaryBackend.cpp:59-104)
 *   UnaryBackendTpp::compile_kernels   (reference src/basic/unary/UnaryBackendTpp.cpp:31-103)
 * Dimensions are given in OUTPUT order with input strides already reordered
 * to that order, i.e. the state after Unary::compile_base
 * (reference src/backend/Unary.cpp:82-113).  ktype: COPY (out = in),
 * ZERO (out = 0) or ADD (out += in).  dtype_in must equal dtype_out.
 */
int etir_hip_permute_create( int64_t         num_dims,
                             int64_t const * sizes,
                             int64_t const * strides_in,
                             int64_t const * strides_out,
                             int32_t         dtype_in,
                             int32_t         dtype_comp,
                             int32_t         dtype_out,
                             int32_t         ktype_main,
                             etir_plan_t   * plan );

/*
 * Enqueues one permutation on `stream`.  Replaces
 *   UnaryTpp::eval                     (reference src/backend/UnaryTpp.cpp:52-54)
 *   UnaryBackend::eval                 (reference src/basic/unary/UnaryBackend.cpp:106-146)
 */
int etir_hip_permute_execute( etir_plan_t  plan,
                              void const * in,
                              void       * out,
                              void       * stream );

/* Releases a contraction or permutation plan and its device tables. */
int etir_hip_plan_destroy( etir_plan_t plan );

/*
 * Writes a one-line description of the plan's kernel choice (kernel name,
 * tile shape, fused sizes, operand load modes) into buf (NUL-terminated,
 * truncated to len bytes).  Diagnostic only.
 */
int etir_hip_plan_describe( etir_plan_t plan,
                            char      * buf,
                            int64_t     len );

/* Number of floating point operations of one execution of a contraction plan
 * (2*C*M*N*K; same definition as the bench harness, reference
 * src/bench_binary.cpp:46-50), 0 for permutation plans. */
int64_t etir_hip_plan_flops( etir_plan_t plan );

/* Algorithmic HBM bytes of one execution (every input element read once, every
 * output element written once, plus a read of the output where the touch
 * kernels need it). */
int64_t etir_hip_plan_bytes( etir_plan_t plan );

/* Reason for the last failure of an etir_hip_* call on this thread. */
char const * etir_hip_last_error( void );

/* Device memory helpers used by MemoryManager's arena and the harnesses.
 * Only these -- never the execute calls -- allocate. */
int etir_hip_malloc( void ** ptr, int64_t num_bytes );
int etir_hip_free( void * ptr );
int etir_hip_memcpy_h2d( void * dst, void const * src, int64_t num_bytes );
int etir_hip_memcpy_d2h( void * dst, void const * src, int64_t num_bytes );
int etir_hip_memcpy_d2d( void * dst, void const * src, int64_t num_bytes, void * stream );
int etir_hip_memset( void * dst, int32_t value, int64_t num_bytes );
int etir_hip_synchronize( void * stream );

/* Number of visible HIP devices (0 on a machine without a GPU). */
int etir_hip_device_count( void );

/* 1 if the GPU can access ptr directly (device, managed, or mapped pinned
 * host memory), 0 if it cannot (pageable host memory, NULL).  No counterpart
 * in the reference, whose tensors are host memory: the synchronous operator
 * calls (BinaryContractionHip::contract, UnaryHip::eval, EinsumNode::eval,
 * store_and_lock_data) use it to stage host tensors through device copies. */
int etir_hip_pointer_is_device( void const * ptr );

/* Streams and graphs for repeated tree evaluation.  These have no
 * counterpart in the reference (its EinsumNode::eval, reference
 * src/backend/EinsumNode.cpp:496-540, calls the backends directly each
 * time); EinsumExpression::eval_graph records one evaluation of the tree with
 * them and replays it.
 *   etir_hip_stream_create   a stream of default priority (non-blocking)
 *   etir_hip_graph_begin     starts recording the work enqueued on `stream`
 *                            (thread-local capture; not the null stream)
 *   etir_hip_graph_end       stops the recording and instantiates it
 *   etir_hip_graph_abort     stops a recording and discards it
 *   etir_hip_graph_launch    enqueues one replay on `stream`
 * A recorded graph holds the kernels' arguments, pointers included, as they
 * were when it was recorded. */
typedef struct etir_graph_s * etir_graph_t;
int etir_hip_stream_create( void ** stream );
int etir_hip_stream_destroy( void * stream );
int etir_hip_graph_begin( void * stream );
int etir_hip_graph_end( void * stream, etir_graph_t * graph );
int etir_hip_graph_abort( void * stream );
int etir_hip_graph_launch( etir_graph_t graph, void * stream );
int etir_hip_graph_destroy( etir_graph_t graph );

/* Events for concurrent tree evaluation.  No counterpart in the reference,
 * whose tree evaluates node after node (reference
 * src/backend/EinsumNode.cpp:496-540): EinsumNode runs an independent subtree
 * on a stream of its own, started after an event recorded on its parent's
 * stream and joined back through an event recorded at its end.
 *   etir_hip_event_create       an event without timing data
 *   etir_hip_event_record       records it on `stream` (NULL: the null stream)
 *   etir_hip_stream_wait_event  makes work enqueued later on `stream` wait
 *                               for the event's last recording */
int etir_hip_event_create( void ** event );
int etir_hip_event_destroy( void * event );
int etir_hip_event_record( void * event, void * stream );
int etir_hip_stream_wait_event( void * stream, void * event );

#ifdef __cplusplus
}
#endif

#endif
