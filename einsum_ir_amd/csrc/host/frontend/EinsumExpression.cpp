// Behaviour follows reference src/frontend/EinsumExpression.cpp:9-367.
#include "EinsumExpression.h"
#include "einsum_ir_hip.h"
#include <algorithm>
#include <deque>
#include <set>

void einsum_ir::frontend::EinsumExpression::histogram( int64_t         i_num_dims,
                                                       int64_t         i_string_size,
                                                       int64_t const * i_string_dim_ids,
                                                       int64_t       * o_histogram ) {
  std::fill( o_histogram, o_histogram + i_num_dims, 0 );
  for( int64_t l_en = 0; l_en < i_string_size; l_en++ ) {
    o_histogram[ i_string_dim_ids[l_en] ]++;
  }
}

void einsum_ir::frontend::EinsumExpression::substring_out( int64_t                        i_num_dims_left,
                                                           int64_t                        i_num_dims_right,
                                                           int64_t                const * i_dim_ids_left,
                                                           int64_t                const * i_dim_ids_right,
                                                           int64_t                      * io_histogram,
                                                           std::vector< int64_t >       & o_substring_out ) {
  // the operands are consumed ...
  for( int64_t l_i = 0; l_i < i_num_dims_left;  l_i++ ) io_histogram[ i_dim_ids_left[l_i]  ]--;
  for( int64_t l_i = 0; l_i < i_num_dims_right; l_i++ ) io_histogram[ i_dim_ids_right[l_i] ]--;
  // ... every dim still referenced elsewhere survives, in ascending id order
  std::set< int64_t > l_keep;
  for( int64_t l_i = 0; l_i < i_num_dims_left;  l_i++ ) if( io_histogram[ i_dim_ids_left[l_i]  ] > 0 ) l_keep.insert( i_dim_ids_left[l_i] );
  for( int64_t l_i = 0; l_i < i_num_dims_right; l_i++ ) if( io_histogram[ i_dim_ids_right[l_i] ] > 0 ) l_keep.insert( i_dim_ids_right[l_i] );
  o_substring_out.assign( l_keep.begin(), l_keep.end() );
  // ... and the intermediate adds one reference to each of its dims
  for( int64_t l_id : o_substring_out ) io_histogram[l_id]++;
}

void einsum_ir::frontend::EinsumExpression::unique_tensor_ids( int64_t         i_num_conts,
                                                               int64_t const * i_path,
                                                               int64_t       * o_path ) {
  int64_t l_next = i_num_conts + 1;
  std::deque< int64_t > l_live;
  for( int64_t l_te = 0; l_te < l_next; l_te++ ) l_live.push_back( l_te );

  for( int64_t l_co = 0; l_co < i_num_conts; l_co++ ) {
    int64_t const l_p0 = i_path[2 * l_co];
    int64_t const l_p1 = i_path[2 * l_co + 1];
    o_path[2 * l_co]     = l_live[l_p0];
    o_path[2 * l_co + 1] = l_live[l_p1];
    l_live.erase( l_live.begin() + std::max( l_p0, l_p1 ) );
    l_live.erase( l_live.begin() + std::min( l_p0, l_p1 ) );
    l_live.push_back( l_next++ );
  }
}

void einsum_ir::frontend::EinsumExpression::init( int64_t                 i_num_dims,
                                                  int64_t const         * i_dim_sizes,
                                                  int64_t                 i_num_conts,
                                                  int64_t const         * i_string_num_dims,
                                                  int64_t const         * i_string_dim_ids,
                                                  int64_t const         * i_path,
                                                  complex_t               i_ctype,
                                                  data_t                  i_dtype,
                                                  void          * const * i_data_ptrs ) {
  m_num_dims = i_num_dims;
  m_dim_sizes = i_dim_sizes;
  m_num_conts = i_num_conts;
  m_string_num_dims_ext = i_string_num_dims;
  m_string_dim_ids_ext = i_string_dim_ids;
  m_path_ext = i_path;
  m_ctype_ext = i_ctype;
  m_dtype = i_dtype;
  m_data_ptrs = i_data_ptrs;
  m_compiled = false;
}

void einsum_ir::frontend::EinsumExpression::init( int64_t                 i_num_dims,
                                                  int64_t const         * i_dim_sizes,
                                                  int64_t                 i_num_conts,
                                                  int64_t const         * i_string_num_dims,
                                                  int64_t const         * i_string_dim_ids,
                                                  int64_t const         * i_path,
                                                  data_t                  i_dtype,
                                                  void          * const * i_data_ptrs ) {
  init( i_num_dims, i_dim_sizes, i_num_conts, i_string_num_dims, i_string_dim_ids, i_path,
        complex_t::REAL_ONLY, i_dtype, i_data_ptrs );
}

einsum_ir::err_t einsum_ir::frontend::EinsumExpression::compile() {
  reset_graph();
  if( m_num_conts < 1 ) {
    return err_t::COMPILATION_FAILED;
  }

  m_path_int.resize( 2 * m_num_conts );
  unique_tensor_ids( m_num_conts, m_path_ext, m_path_int.data() );

  m_map_dim_sizes.clear();
  for( int64_t l_di = 0; l_di < m_num_dims; l_di++ ) m_map_dim_sizes.insert( { l_di, m_dim_sizes[l_di] } );

  int64_t const l_num_in  = m_num_conts + 1;
  int64_t const l_num_all = l_num_in + 1;     // inputs + output of the einsum string

  int64_t l_size_in = 0;
  for( int64_t l_te = 0; l_te < l_num_in; l_te++ ) l_size_in += m_string_num_dims_ext[l_te];
  int64_t const l_size_all = l_size_in + m_string_num_dims_ext[l_num_all - 1];

  // internal string: the inputs followed by every intermediate
  m_string_dim_ids_int.assign( m_string_dim_ids_ext, m_string_dim_ids_ext + l_size_in );
  m_string_num_dims_int.assign( m_string_num_dims_ext, m_string_num_dims_ext + l_num_in );
  std::vector< int64_t > l_offsets( 1, 0 );
  for( int64_t l_te = 1; l_te < l_num_all; l_te++ ) {
    l_offsets.push_back( l_offsets.back() + m_string_num_dims_int[l_te - 1] );
  }

  std::vector< int64_t > l_hist( m_num_dims );
  histogram( m_num_dims, l_size_all, m_string_dim_ids_ext, l_hist.data() );

  // intermediates of every contraction except the last
  for( int64_t l_co = 0; l_co < m_num_conts - 1; l_co++ ) {
    int64_t const l_l = m_path_int[2 * l_co];
    int64_t const l_r = m_path_int[2 * l_co + 1];
    std::vector< int64_t > l_sub;
    substring_out( m_string_num_dims_int[l_l], m_string_num_dims_int[l_r],
                   m_string_dim_ids_int.data() + l_offsets[l_l],
                   m_string_dim_ids_int.data() + l_offsets[l_r],
                   l_hist.data(), l_sub );
    m_string_dim_ids_int.insert( m_string_dim_ids_int.end(), l_sub.begin(), l_sub.end() );
    m_string_num_dims_int.push_back( (int64_t) l_sub.size() );
    l_offsets.push_back( (int64_t) m_string_dim_ids_int.size() );
  }

  // root: the external output's dims
  int64_t const * l_root_ids = m_string_dim_ids_ext + l_size_in;
  int64_t const l_root_nd = m_string_num_dims_ext[l_num_all - 1];

  // complex tensors: the complex dim (size 2) is the output's innermost
  // (BATCH_INNER) or outermost (BATCH_OUTER) dim and appears in every tensor;
  // every contraction runs the complex kernels.  BATCH_INNER contracts into a
  // complex-outermost root and converts it with one more (unary) node
  // (reference EinsumExpression.cpp:214-224, 316-330).
  bool const l_cpx = ( m_ctype_ext != complex_t::REAL_ONLY );
  bool const l_cpx_inner = ( m_ctype_ext == complex_t::BATCH_INNER );
  int64_t l_cpx_id = -1;
  if( l_cpx ) {
    if( l_root_nd < 1 || m_dtype == data_t::BF16 ) return err_t::INVALID_CPX_DIM;
    l_cpx_id = l_cpx_inner ? l_root_ids[l_root_nd - 1] : l_root_ids[0];
    if( m_map_dim_sizes.at( l_cpx_id ) != 2 ) return err_t::INVALID_CPX_DIM;
  }
  if( l_cpx_inner ) {
    m_string_num_dims_int.push_back( l_root_nd );
    m_string_dim_ids_int.push_back( l_cpx_id );
    m_string_dim_ids_int.insert( m_string_dim_ids_int.end(), l_root_ids, l_root_ids + l_root_nd - 1 );
    l_offsets.push_back( (int64_t) m_string_dim_ids_int.size() );
  }
  m_string_num_dims_int.push_back( l_root_nd );
  m_string_dim_ids_int.insert( m_string_dim_ids_int.end(), l_root_ids, l_root_ids + l_root_nd );

  kernel_t const l_first = l_cpx ? kernel_t::CPX_ZERO : kernel_t::ZERO;
  kernel_t const l_main  = l_cpx ? kernel_t::CPX_MADD : kernel_t::MADD;

  // nodes: inputs first, then one node per contraction, then (BATCH_INNER)
  // the conversion; the last node is the root
  int64_t const l_num_nodes = l_num_in + m_num_conts + ( l_cpx_inner ? 1 : 0 );
  m_nodes.clear();
  m_nodes.resize( l_num_nodes );
  for( int64_t l_te = 0; l_te < l_num_in; l_te++ ) {
    m_nodes[l_te].init( m_string_num_dims_int[l_te], m_string_dim_ids_int.data() + l_offsets[l_te],
                        &m_map_dim_sizes, nullptr, m_dtype, m_data_ptrs[l_te], &m_memory );
  }
  for( int64_t l_co = 0; l_co < m_num_conts; l_co++ ) {
    int64_t const l_id_out = l_num_in + l_co;
    bool const l_root = ( l_co == m_num_conts - 1 ) && !l_cpx_inner;
    m_nodes[l_id_out].init( m_string_num_dims_int[l_id_out],
                            m_string_dim_ids_int.data() + l_offsets[l_id_out],
                            &m_map_dim_sizes, nullptr, nullptr, nullptr, nullptr,
                            m_dtype, nullptr,
                            l_root ? m_data_ptrs[l_num_all - 1] : nullptr,
                            l_first, l_main, kernel_t::UNDEFINED_KTYPE,
                            &m_nodes[ m_path_int[2 * l_co] ], &m_nodes[ m_path_int[2 * l_co + 1] ],
                            &m_memory, 1 );
    m_nodes[l_id_out].m_cpx_dim_id = l_cpx_id;
  }
  if( l_cpx_inner ) {
    int64_t const l_id = l_num_in + m_num_conts;
    m_nodes[l_id].init( l_root_nd, m_string_dim_ids_int.data() + l_offsets[l_id], &m_map_dim_sizes, nullptr,
                        m_dtype, m_data_ptrs[l_num_all - 1], &m_nodes[l_id - 1], &m_memory, 1 );
  }
  m_nodes.back().set_stream( m_stream );
  err_t l_err = m_nodes.back().compile();
  m_compiled = ( l_err == err_t::SUCCESS );
  return l_err;
}

einsum_ir::err_t einsum_ir::frontend::EinsumExpression::store_and_lock_data( int64_t i_tensor_id ) {
  if( !m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  if( i_tensor_id < 0 || i_tensor_id >= m_num_conts + 1 ) return err_t::INVALID_ID;
  reset_graph();
  return m_nodes[i_tensor_id].store_and_lock_data();
}

einsum_ir::err_t einsum_ir::frontend::EinsumExpression::unlock_data( int64_t i_tensor_id ) {
  if( !m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  if( i_tensor_id < 0 || i_tensor_id >= m_num_conts + 1 ) return err_t::INVALID_ID;
  reset_graph();
  return m_nodes[i_tensor_id].unlock_data();
}

void einsum_ir::frontend::EinsumExpression::eval() {
  m_nodes.back().eval();
}

einsum_ir::frontend::EinsumExpression::~EinsumExpression() {
  reset_graph();
}

void einsum_ir::frontend::EinsumExpression::reset_graph() {
  if( m_graph != nullptr ) {
    etir_hip_graph_destroy( static_cast< etir_graph_t >( m_graph ) );
    m_graph = nullptr;
  }
}

einsum_ir::err_t einsum_ir::frontend::EinsumExpression::eval_graph_async() {
  if( !m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  if( m_stream == nullptr ) return err_t::UNDEFINED_ERROR;
  if( m_graph == nullptr ) {
    // a recording keeps the pointers it saw: host tensors (which eval() stages
    // through temporary device copies) cannot take part
    if( m_nodes.back().has_host_ext() ) return err_t::NO_DATA_PTR_PROVIDED;
    if( etir_hip_graph_begin( m_stream ) != ETIR_SUCCESS ) return err_t::UNDEFINED_ERROR;
    // recorded on the one stream: a recording that followed the forked
    // subtrees onto their streams ended in a crash of the host process
    err_t l_err = m_nodes.back().eval_one_stream_async();
    if( l_err != err_t::SUCCESS ) {
      etir_hip_graph_abort( m_stream );
      return l_err;
    }
    etir_graph_t l_graph = nullptr;
    if( etir_hip_graph_end( m_stream, &l_graph ) != ETIR_SUCCESS ) return err_t::UNDEFINED_ERROR;
    m_graph = l_graph;
  }
  return etir_hip_graph_launch( static_cast< etir_graph_t >( m_graph ), m_stream ) == ETIR_SUCCESS
           ? err_t::SUCCESS : err_t::UNDEFINED_ERROR;
}

int64_t einsum_ir::frontend::EinsumExpression::num_ops() {
  return m_nodes.empty() ? 0 : m_nodes.back().num_ops( true );
}

namespace {
  std::string join_ids( int64_t const * i_ids, int64_t i_n, char i_sep ) {
    std::string l_s;
    for( int64_t l_i = 0; l_i < i_n; l_i++ ) {
      if( l_i > 0 ) l_s += i_sep;
      l_s += std::to_string( i_ids[l_i] );
    }
    return l_s;
  }
}

std::string einsum_ir::frontend::EinsumExpression::to_string_exchange_format( backend::EinsumNode const * i_node ) const {
  if( !m_compiled || m_nodes.empty() ) return "Error: Expression not compiled.";
  backend::EinsumNode const & l_node = ( i_node != nullptr ) ? *i_node : m_nodes.back();
  std::string const l_ids = join_ids( l_node.m_dim_ids_int.data(), l_node.m_num_dims, ',' );
  if( l_node.m_children.size() == 2 ) {
    return "[" + to_string_exchange_format( l_node.m_children[0] ) + "],["
         + to_string_exchange_format( l_node.m_children[1] ) + "]->[" + l_ids + "]";
  }
  // a one-child node (the complex BATCH_INNER root's conversion) is written
  // as its own ids only, its subtree left out, as the reference writes it
  // (src/frontend/EinsumExpression.cpp:504-563)
  if( l_node.m_children.size() == 1 ) return l_ids;
  if(    l_node.m_dim_ids_ext != nullptr
      && !std::equal( l_node.m_dim_ids_ext, l_node.m_dim_ids_ext + l_node.m_num_dims, l_node.m_dim_ids_int.begin() ) ) {
    return "[" + join_ids( l_node.m_dim_ids_ext, l_node.m_num_dims, ',' ) + "]->[" + l_ids + "]";
  }
  return l_ids;
}

std::string einsum_ir::frontend::EinsumExpression::to_string_render() const {
  if( !m_compiled || m_nodes.empty() ) return "Error: Expression not compiled.";
  // levels of (node, slot): a node in slot s has its children in slots 2s, 2s+1
  std::vector< std::vector< std::pair< backend::EinsumNode const *, int64_t > > > l_levels;
  l_levels.push_back( { { &m_nodes.back(), 0 } } );
  while( true ) {
    std::vector< std::pair< backend::EinsumNode const *, int64_t > > l_next;
    for( auto const & l_e : l_levels.back() ) {
      for( std::size_t l_ch = 0; l_ch < l_e.first->m_children.size(); l_ch++ ) {
        l_next.push_back( { l_e.first->m_children[l_ch], 2 * l_e.second + (int64_t) l_ch } );
      }
    }
    if( l_next.empty() ) break;
    l_levels.push_back( l_next );
  }
  // the drawing doubles in width with every level
  if( l_levels.size() > 16 ) {
    return "Error: tree too deep to draw (" + std::to_string( l_levels.size() ) + " levels).";
  }
  std::size_t l_width = 0;
  for( auto const & l_lvl : l_levels ) {
    for( auto const & l_e : l_lvl ) {
      l_width = std::max( l_width, join_ids( l_e.first->m_dim_ids_int.data(), l_e.first->m_num_dims, ' ' ).size() );
    }
  }
  // the deepest level has 2^(L-1) slots of two cells each; a slot on level l
  // spans 2^(L-l) cells and its node sits in the cell left of the middle
  int64_t const l_num_lvls = (int64_t) l_levels.size();
  std::string l_out;
  for( int64_t l_lv = 0; l_lv < l_num_lvls; l_lv++ ) {
    int64_t const l_span = int64_t( 1 ) << ( l_num_lvls - l_lv );
    int64_t l_cell = 0;
    std::string l_line;
    for( auto const & l_e : l_levels[l_lv] ) {
      int64_t const l_at = l_e.second * l_span + l_span / 2 - 1;
      for( ; l_cell < l_at; l_cell++ ) l_line += std::string( l_width, ' ' );
      std::string l_label = join_ids( l_e.first->m_dim_ids_int.data(), l_e.first->m_num_dims, ' ' );
      l_label.resize( l_width, ' ' );
      l_line += l_label;
      l_cell++;
    }
    if( l_lv > 0 ) l_out += '\n';
    l_out += l_line;
  }
  return l_out;
}
