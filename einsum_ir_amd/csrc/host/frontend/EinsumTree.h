// Einsum tree given node by node (drop-in for reference
// src/frontend/EinsumTree.{h,cpp}:18-94): leaves, unary (permutation) nodes
// and binary contraction nodes; the last node is the root.
#ifndef EINSUM_IR_FRONTEND_EINSUM_TREE
#define EINSUM_IR_FRONTEND_EINSUM_TREE

#include <map>
#include <string>
#include <vector>
#include "../backend/EinsumNode.h"

namespace einsum_ir {
  namespace frontend {
    class EinsumTree;
  }
}

class einsum_ir::frontend::EinsumTree {
  public:
    std::vector< backend::EinsumNode > m_nodes;
    std::vector< std::vector< int64_t > > * m_dim_ids = nullptr;
    std::vector< std::vector< int64_t > > * m_children = nullptr;
    void * const * m_data_ptrs = nullptr;
    backend::MemoryManager m_memory;
    data_t m_dtype = data_t::UNDEFINED_DTYPE;
    std::map< int64_t, int64_t > * m_map_dim_sizes = nullptr;
    void * m_stream = nullptr;

    void init( std::vector< std::vector< int64_t > > * i_dim_ids,
               std::vector< std::vector< int64_t > > * i_children,
               std::map< int64_t, int64_t >          * i_map_dim_sizes,
               data_t                                  i_dtype,
               void                          * const * i_data_ptrs );

    void set_stream( void * i_stream ) { m_stream = i_stream; }

    err_t compile();

    void eval();

    int64_t num_ops();
};

#endif
