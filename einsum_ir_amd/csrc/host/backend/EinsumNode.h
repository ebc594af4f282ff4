// Node of an einsum tree, executed device-resident on one HIP stream.
//
// Drop-in for the reference's einsum_ir::backend::EinsumNode
// (reference src/backend/EinsumNode.h:16-270): same three init overloads,
// compile / store_and_lock_data / unlock_data / eval / num_ops.  Differences:
//   - all data pointers are device pointers; intermediates live in the
//     MemoryManager's single HBM arena; locked data is a device copy;
//   - eval() enqueues the whole tree (permutes and contractions, post-order)
//     on one stream and synchronises once, at the end;
//   - the backend is HIP (EINSUM_IR_BACKEND unset, AUTO or HIP).
#ifndef EINSUM_IR_BACKEND_EINSUM_NODE
#define EINSUM_IR_BACKEND_EINSUM_NODE

#include <vector>
#include "BinaryContraction.h"
#include "MemoryManager.h"
#include "Unary.h"
#include "../constants.h"

namespace einsum_ir {
  namespace backend {
    class EinsumNode;
    class BinaryContractionHip;
    class HostStaging;
    class UnaryHip;
  }
}

class einsum_ir::backend::EinsumNode {
  public:
    data_t m_dtype = data_t::UNDEFINED_DTYPE;

    kernel_t m_ktype_first_touch = kernel_t::UNDEFINED_KTYPE;
    kernel_t m_ktype_main = kernel_t::UNDEFINED_KTYPE;
    kernel_t m_ktype_last_touch = kernel_t::UNDEFINED_KTYPE;

    //! bytes of the node's tensor
    int64_t m_size = 0;

    int64_t m_num_dims = 0;
    int64_t const * m_dim_ids_ext = nullptr;
    std::vector< int64_t > m_dim_ids_int;

    std::map< int64_t, int64_t > const * m_dim_sizes_inner = nullptr;
    std::map< int64_t, int64_t > const * m_dim_sizes_aux_outer = nullptr;
    std::map< int64_t, int64_t > const * m_dim_sizes_outer = nullptr;

    std::vector< EinsumNode * > m_children;

    void * m_data_ptr_int = nullptr;
    void * m_data_ptr_ext = nullptr;
    void * m_data_ptr_active = nullptr;
    void * m_data_ptr_aux_int = nullptr;
    void * m_data_ptr_aux_ext = nullptr;

    std::map< int64_t, int64_t > const * m_offsets_aux_ext = nullptr;
    std::map< int64_t, int64_t > const * m_offsets_ext = nullptr;
    int64_t m_offset_aux_bytes = 0;
    int64_t m_offset_bytes = 0;

    bool m_reorder_dims = false;
    bool m_pack_inputs = false;

    backend_t m_btype_unary  = backend_t::UNDEFINED_BACKEND;
    backend_t m_btype_binary = backend_t::UNDEFINED_BACKEND;

    Unary * m_unary = nullptr;
    BinaryContraction * m_cont = nullptr;

    MemoryManager * m_memory = nullptr;
    int64_t m_mem_id = 0;
    int64_t m_count_mem_users = 0;
    int64_t m_active_mem_users = 0;
    int64_t m_req_mem = 0;
    int64_t m_mem_subtree = 0;

    std::vector< int64_t > m_exec_order;

    int64_t m_num_ops_node = 0;
    int64_t m_num_ops_children = 0;

    int64_t m_num_tasks_intra_op = 1;

    bool m_compiled = false;
    bool m_data_locked = false;

    int64_t m_num_threads = 1;

    //! HIP stream of the whole tree (hipStream_t as void*, nullptr = null stream)
    void * m_stream = nullptr;

    //! Concurrent evaluation of independent subtrees, set up by compile() on
    //! the node it is called on (the root).  A forked node's subtree runs on
    //! its own stream (m_stream, one of the root's pool) from m_ev_fork,
    //! recorded on the parent's stream, to m_ev_done, which the parent's
    //! stream waits for before the parent's kernels; its intermediates live
    //! in an arena of their own (m_fork_memory), as the subtree runs while
    //! its sibling's does.
    bool m_forked = false;
    void * m_ev_fork = nullptr;
    void * m_ev_done = nullptr;
    MemoryManager * m_fork_memory = nullptr;
    //! the root's pool of streams for forked subtrees (owned by the root)
    std::vector< void * > m_pool;

    //! complex trees: id of the complex dim of this node's contraction (-1:
    //! the contraction's default, the first C dim of the output)
    int64_t m_cpx_dim_id = -1;

    ~EinsumNode();

    /** Leaf node (reference EinsumNode.h:141-157). **/
    void init( int64_t                              i_num_dims,
               int64_t                      const * i_dim_ids,
               std::map< int64_t, int64_t > const * i_dim_sizes_inner,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer,
               data_t                               i_dtype,
               void                               * i_data_ptr,
               MemoryManager                      * i_memory );

    /** Node with one child: a permutation of the child's tensor. **/
    void init( int64_t                              i_num_dims,
               int64_t                      const * i_dim_ids,
               std::map< int64_t, int64_t > const * i_dim_sizes_inner,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer,
               data_t                               i_dtype,
               void                               * i_data_ptr,
               EinsumNode                         * i_child,
               MemoryManager                      * i_memory,
               int64_t                              i_num_threads );

    /** Node with two children: a binary contraction. **/
    void init( int64_t                              i_num_dims,
               int64_t                      const * i_dim_ids,
               std::map< int64_t, int64_t > const * i_dim_sizes_inner,
               std::map< int64_t, int64_t > const * i_dim_sizes_aux_outer,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer,
               std::map< int64_t, int64_t > const * i_offsets_aux,
               std::map< int64_t, int64_t > const * i_offsets,
               data_t                               i_dtype,
               void                               * i_data_ptr_aux,
               void                               * i_data_ptr,
               kernel_t                             i_ktype_first_touch,
               kernel_t                             i_ktype_main,
               kernel_t                             i_ktype_last_touch,
               EinsumNode                         * i_left,
               EinsumNode                         * i_right,
               MemoryManager                      * i_memory,
               int64_t                              i_num_threads );

    /** Compiles the tree below this node, plans and allocates the arena. **/
    err_t compile();

    err_t compile_recursive();

    /** Copies (and permutes) the external input once into device memory owned by the node. **/
    err_t store_and_lock_data();

    err_t unlock_data();

    /** Evaluates the tree and waits for the result. **/
    void eval();

    /**
     * eval() with its error: stages host tensors through device copies,
     * enqueues the tree, waits for it and copies computed host tensors back.
     **/
    err_t eval_sync();

    /**
     * Replaces the external pointers of this subtree that point to host
     * memory by device copies from io_staging (inputs copied in, computed
     * tensors copied back by io_staging.finish()); the replaced pointers are
     * appended to io_saved for restore_ext().
     **/
    void stage_ext( HostStaging & io_staging,
                    std::vector< std::pair< void **, void * > > & io_saved );

    //! restores the external pointers saved by stage_ext
    static void restore_ext( std::vector< std::pair< void **, void * > > const & i_saved );

    //! true if an external pointer of this subtree is host memory the GPU cannot reach
    bool has_host_ext() const;

    /** Enqueues the evaluation of the tree on the stream without waiting. **/
    err_t eval_async();

    /** eval_async() with every kernel on this node's stream, in the order of
        the one-stream evaluation (forked subtrees keep their arenas); for
        recording the tree as a graph. **/
    err_t eval_one_stream_async();

    /** Enqueues the subtree; i_forks: forked subtrees on their streams. **/
    err_t eval_tree( bool i_forks );

    /** Kernels of the subtree on i_stream (nullptr: each node's own stream). **/
    void kernels_on( void * i_stream );

    /** Sets the stream of this node and its subtree (before compile()). **/
    void set_stream( void * i_stream );

    /** Puts this node's subtree on a stream and an arena (its kernels included). **/
    void assign( void * i_stream, MemoryManager * i_memory );

    /** Chooses the subtrees that run concurrently and sets up their streams,
        events and arenas (root only, after compile_recursive). **/
    err_t schedule_streams();

    /** Frees what schedule_streams() set up in this subtree. **/
    void release_schedule();

    /** Allocates the arenas of the forked subtrees below this node. **/
    err_t alloc_fork_memory();

    /** True if evaluating this node enqueues work on the GPU. **/
    bool has_work() const;

    /** Rough run time of this node's own kernel (us), to place subtrees. **/
    double est_node_us() const;

    /** Rough run time of the subtree on one stream (us). **/
    double est_subtree_us() const;

    int64_t num_ops( bool i_children = true );

    void cancel_memory_reservation();

    void compile_memory_usage();

    bool requires_permutation();
};

#endif
