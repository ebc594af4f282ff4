// Einsum expression: an einsum string plus a contraction path turned into an
// EinsumNode tree (drop-in for reference src/frontend/EinsumExpression.h:18-201).
// Data pointers are device pointers; the tree runs on one HIP stream.
#ifndef EINSUM_IR_FRONTEND_EINSUM_EXPRESSION
#define EINSUM_IR_FRONTEND_EINSUM_EXPRESSION

#include <cstdint>
#include <string>
#include "../backend/EinsumNode.h"

namespace einsum_ir {
  namespace frontend {
    class EinsumExpression;
  }
}

class einsum_ir::frontend::EinsumExpression {
  public:
    int64_t m_num_dims = 0;
    int64_t const * m_dim_sizes = nullptr;
    int64_t m_num_conts = 0;
    //! dim ids of the einsum string, tensor after tensor, output last
    int64_t const * m_string_dim_ids_ext = nullptr;
    //! number of dims of every tensor in the einsum string
    int64_t const * m_string_num_dims_ext = nullptr;
    data_t m_dtype = data_t::UNDEFINED_DTYPE;
    complex_t m_ctype_ext = complex_t::UNDEFINED_CTYPE;
    void * const * m_data_ptrs = nullptr;
    //! contraction path in opt_einsum's "standard" form (operands removed after use)
    int64_t const * m_path_ext = nullptr;
    //! contraction path with unique tensor ids
    std::vector< int64_t > m_path_int;
    std::vector< int64_t > m_string_dim_ids_int;
    std::vector< int64_t > m_string_num_dims_int;
    std::map< int64_t, int64_t > m_map_dim_sizes;
    std::vector< backend::EinsumNode > m_nodes;
    backend::MemoryManager m_memory;
    bool m_compiled = false;
    void * m_stream = nullptr;
    //! recorded evaluation of the tree (etir_graph_t as void*), replayed by eval_graph()
    void * m_graph = nullptr;

    EinsumExpression() = default;
    EinsumExpression( EinsumExpression const & ) = delete;
    EinsumExpression & operator=( EinsumExpression const & ) = delete;
    ~EinsumExpression();

    /** Number of occurrences of each dim id (reference EinsumExpression.cpp:9-23). **/
    static void histogram( int64_t         i_num_dims,
                           int64_t         i_string_size,
                           int64_t const * i_string_dim_ids,
                           int64_t       * o_histogram );

    /** Dims of an intermediate: those still needed later, ascending ids (:25-70). **/
    static void substring_out( int64_t                        i_num_dims_left,
                               int64_t                        i_num_dims_right,
                               int64_t                const * i_dim_ids_left,
                               int64_t                const * i_dim_ids_right,
                               int64_t                      * io_histogram,
                               std::vector< int64_t >       & o_substring_out );

    /** Path with unique tensor ids: outputs get new ids (:72-99). **/
    static void unique_tensor_ids( int64_t         i_num_conts,
                                   int64_t const * i_path,
                                   int64_t       * o_path );

    void init( int64_t                 i_num_dims,
               int64_t const         * i_dim_sizes,
               int64_t                 i_num_conts,
               int64_t const         * i_string_num_dims,
               int64_t const         * i_string_dim_ids,
               int64_t const         * i_path,
               complex_t               i_ctype,
               data_t                  i_dtype,
               void          * const * i_data_ptrs );

    void init( int64_t                 i_num_dims,
               int64_t const         * i_dim_sizes,
               int64_t                 i_num_conts,
               int64_t const         * i_string_num_dims,
               int64_t const         * i_string_dim_ids,
               int64_t const         * i_path,
               data_t                  i_dtype,
               void          * const * i_data_ptrs );

    /** HIP stream of the tree (set before compile()). **/
    void set_stream( void * i_stream ) { m_stream = i_stream; }

    err_t compile();

    err_t store_and_lock_data( int64_t i_tensor_id );

    err_t unlock_data( int64_t i_tensor_id );

    void eval();

    /**
     * Enqueues one evaluation of the tree as a replay of a HIP graph recorded
     * from eval's launches (recorded on the first call, and again after
     * store_and_lock_data / unlock_data changed what eval launches).  The
     * stream must not be the null stream.  Does not wait.  The results are
     * those of eval(): the same kernels on the same data in the same order.
     **/
    err_t eval_graph_async();

    //! drops the recorded graph (the next eval_graph_async records a new one)
    void reset_graph();

    int64_t num_ops();

    /**
     * The compiled tree in the einsum tree exchange format, the format that
     * EinsumTreeAscii::parse_tree reads (reference EinsumExpression.h:218-235):
     * a leaf is its dim ids "3,2,4"; a node is "[child],[child]->[ids]" or
     * "[child]->[ids]"; a leaf whose internal dim order differs from its
     * tensor's is the unary node "[ext ids]->[internal ids]".  For example
     * "[0,3],[[3,2,4],[4,2]->[1,2,3]]->[0,1,2]".
     *
     * @param i_node subtree to write, nullptr: the whole tree.
     * @return the string, or an error text before compile().
     **/
    std::string to_string_exchange_format( backend::EinsumNode const * i_node = nullptr ) const;

    /**
     * The compiled tree drawn for reading (reference EinsumExpression.h:
     * 210-216): one line per level, root first, each node's dim ids
     * separated by spaces in a cell of the widest node's width, and every
     * node placed centred over the cells its children can take.  Trees of
     * more than 16 levels (whose drawing would be 2^levels cells wide) give
     * an error text instead.
     **/
    std::string to_string_render() const;
};

#endif
