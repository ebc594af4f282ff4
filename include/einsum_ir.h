/*
 * einsum_ir.h -- C ABI of the operator layer of libeinsum_ir.so.
 *
 * The C++ classes (einsum_ir::backend::BinaryContractionHip, UnaryHip,
 * EinsumNode, einsum_ir::frontend::EinsumExpression, EinsumTree) are the
 * drop-in for the reference's operator API.  These functions expose the same
 * operators to callers that can only bind C (ctypes, other languages): each
 * one builds the objects the reference's bench harnesses build from the same
 * string inputs (reference src/bench_binary.cpp:212-402,
 * src/bench_unary.cpp:55-216, src/bench_expression.cpp:8-291,
 * src/bench_tree.cpp:8-140) and forwards to their init/compile/eval calls.
 *
 * Dimension ids are the positions of the sorted dimension names
 * (EinsumExpressionAscii::parse_dim_ids, reference
 * src/frontend/EinsumExpressionAscii.cpp:267-303); `dim_sizes` lists the sizes
 * in ascending id order, as the reference harnesses expect.  Tensor pointers
 * are device pointers.  Return values are einsum_ir::err_t codes.
 */
#ifndef EINSUM_IR_H
#define EINSUM_IR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct etir_binary_s     * etir_binary_t;
typedef struct etir_unary_s      * etir_unary_t;
typedef struct etir_expression_s * etir_expression_t;
typedef struct etir_tree_s       * etir_tree_t;
typedef struct etir_nodes_s      * etir_nodes_t;

/* BinaryContraction (reference src/backend/BinaryContraction.h:279-391)
 * through BinaryContractionHip: `expr` is "abkl,cdkl->abcd" or the bracketed
 * form; outer sizes (NULL = inner sizes) describe views into larger tensors;
 * aux_outer_sizes (NULL allowed) is the auxiliary tensor's outer size per id. */
int etir_binary_create( char const    * expr,
                        int64_t const * dim_sizes,
                        int64_t         num_dim_sizes,
                        int64_t const * aux_outer_sizes,
                        int32_t         dtype_left,
                        int32_t         dtype_right,
                        int32_t         dtype_comp,
                        int32_t         dtype_out,
                        int32_t         ktype_first_touch,
                        int32_t         ktype_main,
                        int32_t         ktype_last_touch,
                        etir_binary_t * handle );
/* BinaryContraction::contract with auxiliary tensor (synchronous). */
int etir_binary_contract( etir_binary_t handle, void const * left, void const * right,
                          void const * out_aux, void * out );
/* BinaryContraction::num_ops */
int64_t etir_binary_num_ops( etir_binary_t handle );
/* m_num_dims_{c,m,n,k} and the products of m_sizes_{c,m,n,k} (read by the harnesses) */
int etir_binary_sizes( etir_binary_t handle, int64_t * num_dims_cmnk, int64_t * sizes_cmnk );
int etir_binary_destroy( etir_binary_t handle );

/* Unary (reference src/backend/Unary.h:98-157) through UnaryHip:
 * `expr` is "abcd->dbca"; ktype COPY, ZERO or ADD. */
int etir_unary_create( char const * expr, int64_t const * dim_sizes, int64_t num_dim_sizes,
                       int32_t dtype, int32_t ktype, etir_unary_t * handle );
int etir_unary_eval( etir_unary_t handle, void const * in, void * out );
int etir_unary_destroy( etir_unary_t handle );

/* EinsumExpression (reference src/frontend/EinsumExpression.h:148-201):
 * `expr` with n inputs, `path` the 2*(n-1) ids of opt_einsum's standard
 * contraction path, data_ptrs the n inputs followed by the output.
 * stream: hipStream_t as void* (NULL = null stream). */
int etir_expression_create( char const        * expr,
                            int64_t const     * dim_sizes,
                            int64_t             num_dim_sizes,
                            int64_t const     * path,
                            int64_t             path_len,
                            int32_t             dtype,
                            void * const      * data_ptrs,
                            void              * stream,
                            etir_expression_t * handle );
/* The same for complex tensors (reference EinsumExpression::init with a
 * complex_t, src/frontend/EinsumExpression.h:160-170): ctype 0 REAL_ONLY,
 * 1 BATCH_INNER (every tensor gets an innermost dim of size 2: real and
 * imaginary parts interleaved, the layout of complex64/complex128 arrays;
 * bench_expression's CPX_FP32/CPX_FP64), 2 BATCH_OUTER (an outermost dim of
 * size 2: all real parts, then all imaginary parts).  `expr` and `dim_sizes`
 * describe the tensors without that dim; dtype FP32 or FP64. */
int etir_expression_create_ctype( char const        * expr,
                                  int64_t const     * dim_sizes,
                                  int64_t             num_dim_sizes,
                                  int64_t const     * path,
                                  int64_t             path_len,
                                  int32_t             ctype,
                                  int32_t             dtype,
                                  void * const      * data_ptrs,
                                  void              * stream,
                                  etir_expression_t * handle );
/* EinsumExpression::eval: enqueues the tree and waits for it. */
int etir_expression_eval( etir_expression_t handle );
/* Enqueues the tree on the stream without waiting. */
int etir_expression_eval_async( etir_expression_t handle );
/* The tree's evaluation as a replay of a recorded HIP graph (recorded on the
 * first call and again after store_and_lock_data / unlock_data); the stream
 * given at creation must not be NULL.  No counterpart in the reference: it
 * replaces EinsumNode::eval's per-call launches (reference
 * src/backend/EinsumNode.cpp:496-540) for repeated evaluations.
 * _eval_graph waits for the replay, _eval_graph_async does not. */
int etir_expression_eval_graph( etir_expression_t handle );
int etir_expression_eval_graph_async( etir_expression_t handle );
int64_t etir_expression_num_ops( etir_expression_t handle );
/* EinsumExpression::store_and_lock_data / unlock_data for input tensor `tensor_id`. */
int etir_expression_store_and_lock_data( etir_expression_t handle, int64_t tensor_id );
int etir_expression_unlock_data( etir_expression_t handle, int64_t tensor_id );
/* Bytes of the device arena planned for the intermediates. */
int64_t etir_expression_arena_bytes( etir_expression_t handle );
int etir_expression_destroy( etir_expression_t handle );

/* EinsumTree (reference src/frontend/EinsumTree.h:46-60) from the bracketed
 * tree format of bench_tree; `data_ptrs` holds one pointer per node in
 * post-order (leaves' inputs, NULL for intermediates, the root's output). */
int64_t etir_tree_count_nodes( char const * tree );
int etir_tree_create( char const * tree, char const * dim_sizes, int32_t dtype,
                      void * const * data_ptrs, void * stream, etir_tree_t * handle );
int etir_tree_eval( etir_tree_t handle );
int64_t etir_tree_num_ops( etir_tree_t handle );
int etir_tree_destroy( etir_tree_t handle );

/* EinsumNode trees built node by node, as the reference's bench_mlp does
 * (reference src/bench_mlp.cpp:85-307 with EinsumNode's init overloads,
 * src/backend/EinsumNode.h:141-216).  One handle owns the dim-size map
 * (`ids[i]` has size `sizes[i]`), the auxiliary tensors' outer sizes
 * (`aux_ids`/`aux_sizes`, e.g. 1 for the batch dims a bias broadcasts over),
 * the nodes, their MemoryManager and the stream (NULL = null stream).
 * Nodes are numbered in the order they are added. */
int etir_nodes_create( int64_t num_ids, int64_t const * ids, int64_t const * sizes,
                       int64_t num_aux_ids, int64_t const * aux_ids, int64_t const * aux_sizes,
                       void * stream, etir_nodes_t * handle );
/* leaf: EinsumNode::init( num_dims, dim_ids, sizes, NULL, dtype, data, memory ) */
int etir_nodes_add_leaf( etir_nodes_t handle, int64_t num_dims, int64_t const * dim_ids,
                         int32_t dtype, void * data, int64_t * node );
/* binary contraction node: EinsumNode::init( num_dims, dim_ids, sizes,
 * aux ? aux sizes : NULL, NULL, NULL, NULL, dtype, aux, data, first, main,
 * last, left, right, memory, 1 ); data NULL = intermediate in the arena. */
int etir_nodes_add_binary( etir_nodes_t handle, int64_t num_dims, int64_t const * dim_ids,
                           int32_t dtype, void * aux, void * data,
                           int32_t ktype_first_touch, int32_t ktype_main, int32_t ktype_last_touch,
                           int64_t left, int64_t right, int64_t * node );
/* EinsumNode::compile of the root (the whole tree below it). */
int etir_nodes_compile( etir_nodes_t handle, int64_t root );
int etir_nodes_store_and_lock_data( etir_nodes_t handle, int64_t node );
int etir_nodes_unlock_data( etir_nodes_t handle, int64_t node );
/* EinsumNode::eval of the compiled root: _eval waits, _eval_async does not. */
int etir_nodes_eval( etir_nodes_t handle );
int etir_nodes_eval_async( etir_nodes_t handle );
/* The root's evaluation as a replay of a recorded HIP graph, recorded on the
 * first call and again after compile, store_and_lock_data or unlock_data;
 * the stream given at creation must not be NULL.  No counterpart in the
 * reference (the same as etir_expression_eval_graph, for trees built node by
 * node): one replay instead of EinsumNode::eval's per-call launches.
 * _eval_graph waits for the replay, _eval_graph_async does not. */
int etir_nodes_eval_graph( etir_nodes_t handle );
int etir_nodes_eval_graph_async( etir_nodes_t handle );
int64_t etir_nodes_num_ops( etir_nodes_t handle );
int etir_nodes_destroy( etir_nodes_t handle );

#ifdef __cplusplus
}
#endif

#endif
