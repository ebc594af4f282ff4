// Behaviour follows reference src/frontend/EinsumTree.cpp:5-102.
#include "EinsumTree.h"

void einsum_ir::frontend::EinsumTree::init( std::vector< std::vector< int64_t > > * i_dim_ids,
                                            std::vector< std::vector< int64_t > > * i_children,
                                            std::map< int64_t, int64_t >          * i_map_dim_sizes,
                                            data_t                                  i_dtype,
                                            void                          * const * i_data_ptrs ) {
  m_dim_ids = i_dim_ids;
  m_children = i_children;
  m_map_dim_sizes = i_map_dim_sizes;
  m_dtype = i_dtype;
  m_data_ptrs = i_data_ptrs;
}

einsum_ir::err_t einsum_ir::frontend::EinsumTree::compile() {
  if( m_children == nullptr || m_dim_ids == nullptr || m_children->empty()
      || m_children->size() != m_dim_ids->size() ) {
    return err_t::COMPILATION_FAILED;
  }
  std::size_t const l_n = m_children->size();
  m_nodes.clear();
  m_nodes.resize( l_n );
  for( std::size_t l_no = 0; l_no < l_n; l_no++ ) {
    std::vector< int64_t > const & l_ch = m_children->at( l_no );
    std::vector< int64_t > & l_ids = m_dim_ids->at( l_no );
    for( int64_t l_c : l_ch ) {
      if( l_c < 0 || (std::size_t) l_c >= l_no ) return err_t::INVALID_ID;
    }
    if( l_ch.empty() ) {
      m_nodes[l_no].init( l_ids.size(), l_ids.data(), m_map_dim_sizes, nullptr, m_dtype,
                          m_data_ptrs[l_no], &m_memory );
    }
    else if( l_ch.size() == 1 ) {
      m_nodes[l_no].init( l_ids.size(), l_ids.data(), m_map_dim_sizes, nullptr, m_dtype,
                          m_data_ptrs[l_no], &m_nodes[ l_ch[0] ], &m_memory, 1 );
    }
    else {
      m_nodes[l_no].init( l_ids.size(), l_ids.data(), m_map_dim_sizes, nullptr, nullptr, nullptr, nullptr,
                          m_dtype, nullptr, m_data_ptrs[l_no],
                          kernel_t::ZERO, kernel_t::MADD, kernel_t::UNDEFINED_KTYPE,
                          &m_nodes[ l_ch[0] ], &m_nodes[ l_ch[1] ], &m_memory, 1 );
    }
  }
  m_nodes.back().set_stream( m_stream );
  return m_nodes.back().compile();
}

void einsum_ir::frontend::EinsumTree::eval() {
  m_nodes.back().eval();
}

int64_t einsum_ir::frontend::EinsumTree::num_ops() {
  return m_nodes.empty() ? 0 : m_nodes.back().num_ops( true );
}
