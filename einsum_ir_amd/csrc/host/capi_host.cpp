// extern "C" functions of include/einsum_ir.h: the operator classes built from
// the same string inputs as the reference's bench harnesses.
#include "einsum_ir.h"
#include "backend/BinaryContractionHip.h"
#include "backend/UnaryHip.h"
#include "frontend/EinsumExpression.h"
#include "frontend/EinsumExpressionAscii.h"
#include "frontend/EinsumTree.h"
#include "frontend/EinsumTreeAscii.h"
#include <deque>
#include <memory>
#include <string>

using namespace einsum_ir;

namespace {

// an expression string parsed into dim-id vectors (bench_binary.cpp:238-402)
struct ParsedExpr {
  std::vector< std::vector< int64_t > > tensors;   // inputs..., output
  std::map< int64_t, int64_t > sizes;
};

err_t parse_expr( char const * i_expr, int64_t const * i_sizes, int64_t i_num_sizes, ParsedExpr & o ) {
  if( i_expr == nullptr || ( i_num_sizes > 0 && i_sizes == nullptr ) ) return err_t::COMPILATION_FAILED;
  std::string l_arg( i_expr ), l_std;
  if( !l_arg.empty() && l_arg[0] == '[' ) l_std = l_arg;
  else frontend::EinsumExpressionAscii::schar_to_standard( l_arg, l_std );

  std::vector< std::string > l_tensors;
  frontend::EinsumExpressionAscii::parse_tensors( l_std, l_tensors );
  std::map< std::string, int64_t > l_ids;
  frontend::EinsumExpressionAscii::parse_dim_ids( l_std, l_ids );
  if( (int64_t) l_ids.size() != i_num_sizes ) return err_t::COMPILATION_FAILED;

  o.tensors.clear();
  for( std::string const & l_t : l_tensors ) {
    std::vector< std::string > l_names;
    frontend::EinsumExpressionAscii::split_string( l_t, ",", l_names );
    std::vector< int64_t > l_v;
    for( std::string const & l_n : l_names ) l_v.push_back( l_ids.at( l_n ) );
    o.tensors.push_back( l_v );
  }
  o.sizes.clear();
  for( int64_t l_i = 0; l_i < i_num_sizes; l_i++ ) o.sizes.insert( { l_i, i_sizes[l_i] } );
  return err_t::SUCCESS;
}

}  // namespace

struct etir_binary_s {
  ParsedExpr expr;
  std::map< int64_t, int64_t > aux_outer;
  bool has_aux_outer = false;
  backend::BinaryContractionHip cont;
};

struct etir_unary_s {
  ParsedExpr expr;
  backend::UnaryHip unary;
};

struct etir_expression_s {
  std::vector< int64_t > sizes;
  std::vector< int64_t > string_num_dims;
  std::vector< int64_t > string_dim_ids;
  std::vector< int64_t > path;
  std::vector< void * > ptrs;
  frontend::EinsumExpression expr;
};

struct etir_tree_s {
  std::vector< std::vector< int64_t > > dim_ids;
  std::vector< std::vector< int64_t > > children;
  std::map< int64_t, int64_t > sizes;
  std::vector< void * > ptrs;
  frontend::EinsumTree tree;
};

// EinsumNodes built one by one (reference src/bench_mlp.cpp:85-307): the
// handle owns the size maps, the dim-id arrays the nodes borrow, the nodes and
// their memory manager; deque storage keeps every borrowed address stable
struct etir_nodes_s {
  std::map< int64_t, int64_t > sizes;
  std::map< int64_t, int64_t > aux_sizes;
  std::deque< std::vector< int64_t > > dim_ids;
  std::deque< backend::EinsumNode > nodes;
  backend::MemoryManager memory;
  void * stream = nullptr;
  int64_t root = -1;
  // recorded evaluation of the root (etir_nodes_eval_graph*), dropped when
  // the tree is compiled again or its locked data changes
  etir_graph_t graph = nullptr;

  void reset_graph() {
    if( graph != nullptr ) etir_hip_graph_destroy( graph );
    graph = nullptr;
  }
  ~etir_nodes_s() { reset_graph(); }
};

extern "C" {

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
                        etir_binary_t * handle ) {
  if( handle == nullptr ) return err_t::UNDEFINED_ERROR;
  *handle = nullptr;
  std::unique_ptr< etir_binary_s > l_h( new etir_binary_s() );
  try {
    err_t l_err = parse_expr( expr, dim_sizes, num_dim_sizes, l_h->expr );
    if( l_err != err_t::SUCCESS ) return l_err;
    if( l_h->expr.tensors.size() != 3 ) return err_t::COMPILATION_FAILED;
    if( aux_outer_sizes != nullptr ) {
      for( int64_t l_i = 0; l_i < num_dim_sizes; l_i++ ) l_h->aux_outer.insert( { l_i, aux_outer_sizes[l_i] } );
      l_h->has_aux_outer = true;
    }
    auto & l_t = l_h->expr.tensors;
    l_h->cont.init( l_t[0].size(), l_t[1].size(), l_t[2].size(),
                    &l_h->expr.sizes, &l_h->expr.sizes, &l_h->expr.sizes,
                    l_h->has_aux_outer ? &l_h->aux_outer : nullptr, &l_h->expr.sizes,
                    l_t[0].data(), l_t[1].data(), l_t[2].data(),
                    (data_t) dtype_left, (data_t) dtype_right, (data_t) dtype_comp, (data_t) dtype_out,
                    (kernel_t) ktype_first_touch, (kernel_t) ktype_main, (kernel_t) ktype_last_touch, 1 );
    l_err = l_h->cont.compile();
    if( l_err != err_t::SUCCESS ) return l_err;
  }
  catch( std::exception const & ) {
    return err_t::COMPILATION_FAILED;
  }
  *handle = l_h.release();
  return err_t::SUCCESS;
}

int etir_binary_contract( etir_binary_t handle, void const * left, void const * right,
                          void const * out_aux, void * out ) {
  if( handle == nullptr ) return err_t::CALLED_BEFORE_COMPILATION;
  handle->cont.contract( left, right, out_aux, out );
  return handle->cont.last_error();
}

int64_t etir_binary_num_ops( etir_binary_t handle ) {
  return handle == nullptr ? 0 : handle->cont.num_ops();
}

int etir_binary_sizes( etir_binary_t handle, int64_t * num_dims_cmnk, int64_t * sizes_cmnk ) {
  if( handle == nullptr || num_dims_cmnk == nullptr || sizes_cmnk == nullptr ) return err_t::UNDEFINED_ERROR;
  backend::BinaryContraction & l_c = handle->cont;
  std::vector< int64_t > const * l_sz[4] = { &l_c.m_sizes_c, &l_c.m_sizes_m, &l_c.m_sizes_n, &l_c.m_sizes_k };
  int64_t const l_nd[4] = { l_c.m_num_dims_c, l_c.m_num_dims_m, l_c.m_num_dims_n, l_c.m_num_dims_k };
  for( int l_i = 0; l_i < 4; l_i++ ) {
    num_dims_cmnk[l_i] = l_nd[l_i];
    sizes_cmnk[l_i] = 1;
    for( int64_t l_s : *l_sz[l_i] ) sizes_cmnk[l_i] *= l_s;
  }
  return err_t::SUCCESS;
}

int etir_binary_destroy( etir_binary_t handle ) {
  delete handle;
  return err_t::SUCCESS;
}

int etir_unary_create( char const * expr, int64_t const * dim_sizes, int64_t num_dim_sizes,
                       int32_t dtype, int32_t ktype, etir_unary_t * handle ) {
  if( handle == nullptr ) return err_t::UNDEFINED_ERROR;
  *handle = nullptr;
  std::unique_ptr< etir_unary_s > l_h( new etir_unary_s() );
  try {
    err_t l_err = parse_expr( expr, dim_sizes, num_dim_sizes, l_h->expr );
    if( l_err != err_t::SUCCESS ) return l_err;
    auto & l_t = l_h->expr.tensors;
    if( l_t.size() != 2 || l_t[0].size() != l_t[1].size() ) return err_t::COMPILATION_FAILED;
    l_h->unary.init( l_t[0].size(), &l_h->expr.sizes, l_t[0].data(), l_t[1].data(),
                     (data_t) dtype, (data_t) dtype, (data_t) dtype, (kernel_t) ktype, 1 );
    l_err = l_h->unary.compile();
    if( l_err != err_t::SUCCESS ) return l_err;
  }
  catch( std::exception const & ) {
    return err_t::COMPILATION_FAILED;
  }
  *handle = l_h.release();
  return err_t::SUCCESS;
}

int etir_unary_eval( etir_unary_t handle, void const * in, void * out ) {
  if( handle == nullptr ) return err_t::CALLED_BEFORE_COMPILATION;
  handle->unary.eval( in, out );
  return handle->unary.last_error();
}

int etir_unary_destroy( etir_unary_t handle ) {
  delete handle;
  return err_t::SUCCESS;
}

int etir_expression_create( char const        * expr,
                            int64_t const     * dim_sizes,
                            int64_t             num_dim_sizes,
                            int64_t const     * path,
                            int64_t             path_len,
                            int32_t             dtype,
                            void * const      * data_ptrs,
                            void              * stream,
                            etir_expression_t * handle ) {
  return etir_expression_create_ctype( expr, dim_sizes, num_dim_sizes, path, path_len, (int32_t) REAL_ONLY,
                                       dtype, data_ptrs, stream, handle );
}

int etir_expression_create_ctype( char const        * expr,
                                  int64_t const     * dim_sizes,
                                  int64_t             num_dim_sizes,
                                  int64_t const     * path,
                                  int64_t             path_len,
                                  int32_t             ctype,
                                  int32_t             dtype,
                                  void * const      * data_ptrs,
                                  void              * stream,
                                  etir_expression_t * handle ) {
  if( handle == nullptr ) return err_t::UNDEFINED_ERROR;
  *handle = nullptr;
  if( ctype != REAL_ONLY && ctype != BATCH_INNER && ctype != BATCH_OUTER ) return err_t::COMPILATION_FAILED;
  std::unique_ptr< etir_expression_s > l_h( new etir_expression_s() );
  try {
    ParsedExpr l_p;
    err_t l_err = parse_expr( expr, dim_sizes, num_dim_sizes, l_p );
    if( l_err != err_t::SUCCESS ) return l_err;
    int64_t const l_num_tensors = (int64_t) l_p.tensors.size();
    int64_t const l_num_conts = l_num_tensors - 2;
    if( l_num_conts < 1 || path_len != 2 * l_num_conts || path == nullptr || data_ptrs == nullptr ) {
      return err_t::COMPILATION_FAILED;
    }
    l_h->sizes.assign( dim_sizes, dim_sizes + num_dim_sizes );
    // complex tensors: one more dim of size 2 with the next free id, innermost
    // (BATCH_INNER, as bench_expression.cpp:110,196-222 appends it) or
    // outermost (BATCH_OUTER) in every tensor
    int64_t l_num_ids = num_dim_sizes;
    if( ctype != REAL_ONLY ) {
      l_h->sizes.push_back( 2 );
      for( auto & l_t : l_p.tensors ) {
        if( ctype == BATCH_INNER ) l_t.push_back( num_dim_sizes );
        else                       l_t.insert( l_t.begin(), num_dim_sizes );
      }
      l_num_ids++;
    }
    for( auto const & l_t : l_p.tensors ) {
      l_h->string_num_dims.push_back( (int64_t) l_t.size() );
      l_h->string_dim_ids.insert( l_h->string_dim_ids.end(), l_t.begin(), l_t.end() );
    }
    l_h->path.assign( path, path + path_len );
    l_h->ptrs.assign( data_ptrs, data_ptrs + l_num_tensors );
    l_h->expr.init( l_num_ids, l_h->sizes.data(), l_num_conts,
                    l_h->string_num_dims.data(), l_h->string_dim_ids.data(), l_h->path.data(),
                    (complex_t) ctype, (data_t) dtype, l_h->ptrs.data() );
    l_h->expr.set_stream( stream );
    l_err = l_h->expr.compile();
    if( l_err != err_t::SUCCESS ) return l_err;
  }
  catch( std::exception const & ) {
    return err_t::COMPILATION_FAILED;
  }
  *handle = l_h.release();
  return err_t::SUCCESS;
}

int etir_expression_eval( etir_expression_t handle ) {
  if( handle == nullptr || !handle->expr.m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  return handle->expr.m_nodes.back().eval_sync();
}

int etir_expression_eval_async( etir_expression_t handle ) {
  if( handle == nullptr || !handle->expr.m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  return handle->expr.m_nodes.back().eval_async();
}

int etir_expression_eval_graph( etir_expression_t handle ) {
  if( handle == nullptr || !handle->expr.m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  err_t l_err = handle->expr.eval_graph_async();
  if( l_err != err_t::SUCCESS ) return l_err;
  return etir_hip_synchronize( handle->expr.m_stream ) == ETIR_SUCCESS ? err_t::SUCCESS : err_t::UNDEFINED_ERROR;
}

int etir_expression_eval_graph_async( etir_expression_t handle ) {
  if( handle == nullptr || !handle->expr.m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  return handle->expr.eval_graph_async();
}

int64_t etir_expression_num_ops( etir_expression_t handle ) {
  return handle == nullptr ? 0 : handle->expr.num_ops();
}

int etir_expression_store_and_lock_data( etir_expression_t handle, int64_t tensor_id ) {
  if( handle == nullptr ) return err_t::CALLED_BEFORE_COMPILATION;
  return handle->expr.store_and_lock_data( tensor_id );
}

int etir_expression_unlock_data( etir_expression_t handle, int64_t tensor_id ) {
  if( handle == nullptr ) return err_t::CALLED_BEFORE_COMPILATION;
  return handle->expr.unlock_data( tensor_id );
}

int64_t etir_expression_arena_bytes( etir_expression_t handle ) {
  return handle == nullptr ? 0 : handle->expr.m_memory.get_required_memory();
}

int etir_expression_destroy( etir_expression_t handle ) {
  delete handle;
  return err_t::SUCCESS;
}

int64_t etir_tree_count_nodes( char const * tree ) {
  return tree == nullptr ? 0 : frontend::EinsumTreeAscii::count_nodes( tree );
}

int etir_tree_create( char const * tree, char const * dim_sizes, int32_t dtype,
                      void * const * data_ptrs, void * stream, etir_tree_t * handle ) {
  if( handle == nullptr ) return err_t::UNDEFINED_ERROR;
  *handle = nullptr;
  if( tree == nullptr || dim_sizes == nullptr || data_ptrs == nullptr ) return err_t::COMPILATION_FAILED;
  std::unique_ptr< etir_tree_s > l_h( new etir_tree_s() );
  try {
    int64_t const l_n = frontend::EinsumTreeAscii::count_nodes( tree );
    l_h->dim_ids.resize( l_n );
    l_h->children.resize( l_n );
    int64_t l_parsed = 0;
    err_t l_err = frontend::EinsumTreeAscii::parse_tree( tree, l_h->dim_ids, l_h->children, l_parsed );
    if( l_err != err_t::SUCCESS || l_parsed != l_n ) return err_t::COMPILATION_FAILED;
    frontend::EinsumTreeAscii::parse_dim_size( dim_sizes, l_h->dim_ids, l_h->sizes );
    l_h->ptrs.assign( data_ptrs, data_ptrs + l_n );
    l_h->tree.init( &l_h->dim_ids, &l_h->children, &l_h->sizes, (data_t) dtype, l_h->ptrs.data() );
    l_h->tree.set_stream( stream );
    l_err = l_h->tree.compile();
    if( l_err != err_t::SUCCESS ) return l_err;
  }
  catch( std::exception const & ) {
    return err_t::COMPILATION_FAILED;
  }
  *handle = l_h.release();
  return err_t::SUCCESS;
}

int etir_tree_eval( etir_tree_t handle ) {
  if( handle == nullptr || handle->tree.m_nodes.empty() ) return err_t::CALLED_BEFORE_COMPILATION;
  return handle->tree.m_nodes.back().eval_sync();
}

int64_t etir_tree_num_ops( etir_tree_t handle ) {
  return handle == nullptr ? 0 : handle->tree.num_ops();
}

int etir_tree_destroy( etir_tree_t handle ) {
  delete handle;
  return err_t::SUCCESS;
}

int etir_nodes_create( int64_t         num_ids,
                       int64_t const * ids,
                       int64_t const * sizes,
                       int64_t         num_aux_ids,
                       int64_t const * aux_ids,
                       int64_t const * aux_sizes,
                       void          * stream,
                       etir_nodes_t  * handle ) {
  if( handle == nullptr ) return err_t::UNDEFINED_ERROR;
  *handle = nullptr;
  if( num_ids < 0 || num_aux_ids < 0 || ( num_ids > 0 && ( ids == nullptr || sizes == nullptr ) )
      || ( num_aux_ids > 0 && ( aux_ids == nullptr || aux_sizes == nullptr ) ) ) {
    return err_t::COMPILATION_FAILED;
  }
  std::unique_ptr< etir_nodes_s > l_h( new etir_nodes_s() );
  for( int64_t l_i = 0; l_i < num_ids; l_i++ ) l_h->sizes[ ids[l_i] ] = sizes[l_i];
  for( int64_t l_i = 0; l_i < num_aux_ids; l_i++ ) l_h->aux_sizes[ aux_ids[l_i] ] = aux_sizes[l_i];
  l_h->stream = stream;
  *handle = l_h.release();
  return err_t::SUCCESS;
}

int etir_nodes_add_leaf( etir_nodes_t    handle,
                         int64_t         num_dims,
                         int64_t const * dim_ids,
                         int32_t         dtype,
                         void          * data,
                         int64_t       * node ) {
  if( handle == nullptr || node == nullptr || num_dims < 0 || ( num_dims > 0 && dim_ids == nullptr ) ) {
    return err_t::COMPILATION_FAILED;
  }
  handle->dim_ids.emplace_back( dim_ids, dim_ids + num_dims );
  handle->nodes.emplace_back();
  handle->nodes.back().init( num_dims, handle->dim_ids.back().data(), &handle->sizes, nullptr,
                             (data_t) dtype, data, &handle->memory );
  *node = (int64_t) handle->nodes.size() - 1;
  return err_t::SUCCESS;
}

int etir_nodes_add_binary( etir_nodes_t    handle,
                           int64_t         num_dims,
                           int64_t const * dim_ids,
                           int32_t         dtype,
                           void          * aux,
                           void          * data,
                           int32_t         ktype_first_touch,
                           int32_t         ktype_main,
                           int32_t         ktype_last_touch,
                           int64_t         left,
                           int64_t         right,
                           int64_t       * node ) {
  if( handle == nullptr || node == nullptr || num_dims < 0 || ( num_dims > 0 && dim_ids == nullptr ) ) {
    return err_t::COMPILATION_FAILED;
  }
  int64_t const l_n = (int64_t) handle->nodes.size();
  if( left < 0 || left >= l_n || right < 0 || right >= l_n || left == right ) return err_t::INVALID_ID;
  handle->dim_ids.emplace_back( dim_ids, dim_ids + num_dims );
  handle->nodes.emplace_back();
  std::map< int64_t, int64_t > const * l_aux_sizes = ( aux != nullptr && !handle->aux_sizes.empty() )
                                                       ? &handle->aux_sizes : nullptr;
  handle->nodes.back().init( num_dims, handle->dim_ids.back().data(), &handle->sizes, l_aux_sizes, nullptr,
                             nullptr, nullptr, (data_t) dtype, aux, data,
                             (kernel_t) ktype_first_touch, (kernel_t) ktype_main, (kernel_t) ktype_last_touch,
                             &handle->nodes[left], &handle->nodes[right], &handle->memory, 1 );
  *node = l_n;
  return err_t::SUCCESS;
}

int etir_nodes_compile( etir_nodes_t handle, int64_t root ) {
  if( handle == nullptr ) return err_t::CALLED_BEFORE_COMPILATION;
  if( root < 0 || root >= (int64_t) handle->nodes.size() ) return err_t::INVALID_ID;
  handle->reset_graph();
  try {
    handle->nodes[root].set_stream( handle->stream );
    err_t l_err = handle->nodes[root].compile();
    if( l_err != err_t::SUCCESS ) return l_err;
  }
  catch( std::exception const & ) {
    return err_t::COMPILATION_FAILED;
  }
  handle->root = root;
  return err_t::SUCCESS;
}

int etir_nodes_store_and_lock_data( etir_nodes_t handle, int64_t node ) {
  if( handle == nullptr || handle->root < 0 ) return err_t::CALLED_BEFORE_COMPILATION;
  if( node < 0 || node >= (int64_t) handle->nodes.size() ) return err_t::INVALID_ID;
  handle->reset_graph();
  return handle->nodes[node].store_and_lock_data();
}

int etir_nodes_unlock_data( etir_nodes_t handle, int64_t node ) {
  if( handle == nullptr || handle->root < 0 ) return err_t::CALLED_BEFORE_COMPILATION;
  if( node < 0 || node >= (int64_t) handle->nodes.size() ) return err_t::INVALID_ID;
  handle->reset_graph();
  return handle->nodes[node].unlock_data();
}

int etir_nodes_eval_async( etir_nodes_t handle ) {
  if( handle == nullptr || handle->root < 0 ) return err_t::CALLED_BEFORE_COMPILATION;
  return handle->nodes[ handle->root ].eval_async();
}

int etir_nodes_eval( etir_nodes_t handle ) {
  if( handle == nullptr || handle->root < 0 ) return err_t::CALLED_BEFORE_COMPILATION;
  return handle->nodes[ handle->root ].eval_sync();
}

int etir_nodes_eval_graph_async( etir_nodes_t handle ) {
  if( handle == nullptr || handle->root < 0 ) return err_t::CALLED_BEFORE_COMPILATION;
  if( handle->stream == nullptr ) return err_t::UNDEFINED_ERROR;
  backend::EinsumNode & l_root = handle->nodes[ handle->root ];
  if( handle->graph == nullptr ) {
    // a recording keeps the pointers it saw: host tensors, staged through
    // temporary device copies per evaluation, cannot take part
    if( l_root.has_host_ext() ) return err_t::NO_DATA_PTR_PROVIDED;
    if( etir_hip_graph_begin( handle->stream ) != ETIR_SUCCESS ) return err_t::UNDEFINED_ERROR;
    err_t l_err = l_root.eval_one_stream_async();
    if( l_err != err_t::SUCCESS ) {
      etir_hip_graph_abort( handle->stream );
      return l_err;
    }
    if( etir_hip_graph_end( handle->stream, &handle->graph ) != ETIR_SUCCESS ) {
      handle->graph = nullptr;
      return err_t::UNDEFINED_ERROR;
    }
  }
  return etir_hip_graph_launch( handle->graph, handle->stream ) == ETIR_SUCCESS
           ? err_t::SUCCESS : err_t::UNDEFINED_ERROR;
}

int etir_nodes_eval_graph( etir_nodes_t handle ) {
  int l_err = etir_nodes_eval_graph_async( handle );
  if( l_err != err_t::SUCCESS ) return l_err;
  return etir_hip_synchronize( handle->stream ) == ETIR_SUCCESS ? err_t::SUCCESS : err_t::UNDEFINED_ERROR;
}

int64_t etir_nodes_num_ops( etir_nodes_t handle ) {
  if( handle == nullptr || handle->root < 0 ) return 0;
  return handle->nodes[ handle->root ].num_ops( true );
}

int etir_nodes_destroy( etir_nodes_t handle ) {
  delete handle;
  return err_t::SUCCESS;
}

}  // extern "C"
