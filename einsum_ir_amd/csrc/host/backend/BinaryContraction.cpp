#include <stdexcept>
#include "BinaryContraction.h"
#include <algorithm>

void einsum_ir::backend::BinaryContraction::dim_types( int64_t         i_num_dims_t0,
                                                       int64_t         i_num_dims_t1,
                                                       int64_t         i_num_dims_t2,
                                                       int64_t const * i_dim_ids_t0,
                                                       int64_t const * i_dim_ids_t1,
                                                       int64_t const * i_dim_ids_t2,
                                                       dim_t           i_dim_type_t2,
                                                       dim_t           i_dim_type_t2_t0,
                                                       dim_t           i_dim_type_t2_t1,
                                                       dim_t           i_dim_type_t2_t0_t1,
                                                       dim_t         * o_dim_types_t2 ) {
  // occurrences still available for matching in t0 and t1
  std::vector< bool > l_used_t0( i_num_dims_t0, false );
  std::vector< bool > l_used_t1( i_num_dims_t1, false );
  auto match = []( int64_t i_id, int64_t i_n, int64_t const * i_ids, std::vector< bool > & io_used ) {
    for( int64_t l_i = 0; l_i < i_n; l_i++ ) {
      if( !io_used[l_i] && i_ids[l_i] == i_id ) {
        io_used[l_i] = true;
        return true;
      }
    }
    return false;
  };

  for( int64_t l_di = 0; l_di < i_num_dims_t2; l_di++ ) {
    int64_t const l_id = i_dim_ids_t2[l_di];
    bool const l_in_t0 = match( l_id, i_num_dims_t0, i_dim_ids_t0, l_used_t0 );
    bool const l_in_t1 = match( l_id, i_num_dims_t1, i_dim_ids_t1, l_used_t1 );
    if(      l_in_t0 && l_in_t1 ) o_dim_types_t2[l_di] = i_dim_type_t2_t0_t1;
    else if( l_in_t0 )            o_dim_types_t2[l_di] = i_dim_type_t2_t0;
    else if( l_in_t1 )            o_dim_types_t2[l_di] = i_dim_type_t2_t1;
    else                          o_dim_types_t2[l_di] = i_dim_type_t2;
  }
}

void einsum_ir::backend::BinaryContraction::dim_types( int64_t                      i_num_dims_left,
                                                       int64_t                      i_num_dims_right,
                                                       int64_t                      i_num_dims_out,
                                                       int64_t              const * i_dim_ids_left,
                                                       int64_t              const * i_dim_ids_right,
                                                       int64_t              const * i_dim_ids_out,
                                                       std::vector< dim_t >       * o_dim_types_left,
                                                       std::vector< dim_t >       * o_dim_types_right,
                                                       std::vector< dim_t >       * o_dim_types_out ) {
  o_dim_types_left->resize( i_num_dims_left );
  o_dim_types_right->resize( i_num_dims_right );
  o_dim_types_out->resize( i_num_dims_out );

  // left relative to (right, out): I / K / M / C
  dim_types( i_num_dims_right, i_num_dims_out, i_num_dims_left,
             i_dim_ids_right, i_dim_ids_out, i_dim_ids_left,
             I, K, M, C, o_dim_types_left->data() );
  // right relative to (left, out): J / K / N / C
  dim_types( i_num_dims_left, i_num_dims_out, i_num_dims_right,
             i_dim_ids_left, i_dim_ids_out, i_dim_ids_right,
             J, K, N, C, o_dim_types_right->data() );
  // out relative to (left, right): - / M / N / C
  dim_types( i_num_dims_left, i_num_dims_right, i_num_dims_out,
             i_dim_ids_left, i_dim_ids_right, i_dim_ids_out,
             UNDEFINED_DIM, M, N, C, o_dim_types_out->data() );
}

int64_t einsum_ir::backend::BinaryContraction::filter_dim_ids( int64_t         i_num_dims_tensor,
                                                               dim_t           i_dim_type_filter,
                                                               dim_t   const * i_dim_types_tensor,
                                                               int64_t const * i_dim_ids_tensor,
                                                               int64_t       * o_dim_ids_filtered ) {
  int64_t l_count = 0;
  for( int64_t l_di = 0; l_di < i_num_dims_tensor; l_di++ ) {
    if( i_dim_types_tensor[l_di] == i_dim_type_filter ) {
      o_dim_ids_filtered[l_count++] = i_dim_ids_tensor[l_di];
    }
  }
  return l_count;
}

void einsum_ir::backend::BinaryContraction::dim_types_ids( int64_t                        i_num_dims_left,
                                                           int64_t                        i_num_dims_right,
                                                           int64_t                        i_num_dims_out,
                                                           int64_t                const * i_dim_ids_left,
                                                           int64_t                const * i_dim_ids_right,
                                                           int64_t                const * i_dim_ids_out,
                                                           std::vector< dim_t >         * o_dim_types_out,
                                                           std::vector< int64_t >       * o_dim_ids_c,
                                                           std::vector< int64_t >       * o_dim_ids_m,
                                                           std::vector< int64_t >       * o_dim_ids_n,
                                                           std::vector< int64_t >       * o_dim_ids_k,
                                                           std::vector< int64_t >       * o_dim_ids_i,
                                                           std::vector< int64_t >       * o_dim_ids_j ) {
  std::vector< dim_t > l_types_left;
  std::vector< dim_t > l_types_right;
  dim_types( i_num_dims_left, i_num_dims_right, i_num_dims_out,
             i_dim_ids_left, i_dim_ids_right, i_dim_ids_out,
             &l_types_left, &l_types_right, o_dim_types_out );

  auto collect = []( int64_t i_n, dim_t i_type, std::vector< dim_t > const & i_types,
                     int64_t const * i_ids, std::vector< int64_t > * o_ids ) {
    o_ids->resize( i_n );
    int64_t l_count = filter_dim_ids( i_n, i_type, i_types.data(), i_ids, o_ids->data() );
    o_ids->resize( l_count );
  };
  collect( i_num_dims_out,   C, *o_dim_types_out, i_dim_ids_out,   o_dim_ids_c );
  collect( i_num_dims_out,   M, *o_dim_types_out, i_dim_ids_out,   o_dim_ids_m );
  collect( i_num_dims_out,   N, *o_dim_types_out, i_dim_ids_out,   o_dim_ids_n );
  collect( i_num_dims_left,  K, l_types_left,     i_dim_ids_left,  o_dim_ids_k );
  collect( i_num_dims_left,  I, l_types_left,     i_dim_ids_left,  o_dim_ids_i );
  collect( i_num_dims_right, J, l_types_right,    i_dim_ids_right, o_dim_ids_j );
}

void einsum_ir::backend::BinaryContraction::strides( int64_t                              i_num_dims,
                                                     int64_t                      const * i_dim_ids,
                                                     std::map< int64_t, int64_t > const * i_dim_sizes,
                                                     std::map< int64_t, int64_t >       * o_strides ) {
  o_strides->clear();
  int64_t l_stride = 1;
  for( int64_t l_di = i_num_dims - 1; l_di >= 0; l_di-- ) {
    int64_t const l_id   = i_dim_ids[l_di];
    int64_t const l_size = i_dim_sizes->at( l_id );
    o_strides->insert( { l_id, l_size < 2 ? 0 : l_stride } );
    l_stride *= l_size;
  }
}

void einsum_ir::backend::BinaryContraction::init( int64_t                              i_num_dims_left,
                                                  int64_t                              i_num_dims_right,
                                                  int64_t                              i_num_dims_out,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_inner,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_outer_left,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_outer_right,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_outer_out_aux,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_outer_out,
                                                  int64_t                      const * i_dim_ids_left,
                                                  int64_t                      const * i_dim_ids_right,
                                                  int64_t                      const * i_dim_ids_out,
                                                  data_t                               i_dtype_left,
                                                  data_t                               i_dtype_right,
                                                  data_t                               i_dtype_comp,
                                                  data_t                               i_dtype_out,
                                                  kernel_t                             i_ktype_first_touch,
                                                  kernel_t                             i_ktype_main,
                                                  kernel_t                             i_ktype_last_touch,
                                                  int64_t                              i_num_threads ) {
  init( i_num_dims_left, i_num_dims_right, i_num_dims_out,
        i_dim_sizes_inner, i_dim_sizes_outer_left, i_dim_sizes_outer_right,
        i_dim_sizes_outer_out_aux, i_dim_sizes_outer_out,
        nullptr,
        i_dim_ids_left, i_dim_ids_right, i_dim_ids_out,
        nullptr, nullptr, nullptr,
        i_dtype_left, i_dtype_right, i_dtype_comp, i_dtype_out,
        i_ktype_first_touch, i_ktype_main, i_ktype_last_touch,
        i_num_threads );
}

void einsum_ir::backend::BinaryContraction::init( int64_t                              i_num_dims_left,
                                                  int64_t                              i_num_dims_right,
                                                  int64_t                              i_num_dims_out,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_inner,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_outer_left,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_outer_right,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_outer_out_aux,
                                                  std::map< int64_t, int64_t > const * i_dim_sizes_outer_out,
                                                  std::vector< int64_t >       const * i_loop_ids_ext,
                                                  int64_t                      const * i_dim_ids_left,
                                                  int64_t                      const * i_dim_ids_right,
                                                  int64_t                      const * i_dim_ids_out,
                                                  int64_t                      const * i_dim_ids_permute_left,
                                                  int64_t                      const * i_dim_ids_permute_right,
                                                  MemoryManager                      * i_memory,
                                                  data_t                               i_dtype_left,
                                                  data_t                               i_dtype_right,
                                                  data_t                               i_dtype_comp,
                                                  data_t                               i_dtype_out,
                                                  kernel_t                             i_ktype_first_touch,
                                                  kernel_t                             i_ktype_main,
                                                  kernel_t                             i_ktype_last_touch,
                                                  int64_t                              i_num_threads ) {
  m_num_dims_left  = i_num_dims_left;
  m_num_dims_right = i_num_dims_right;
  m_num_dims_out   = i_num_dims_out;
  m_dim_sizes_inner         = i_dim_sizes_inner;
  m_dim_sizes_outer_left    = i_dim_sizes_outer_left;
  m_dim_sizes_outer_right   = i_dim_sizes_outer_right;
  m_dim_sizes_outer_out_aux = i_dim_sizes_outer_out_aux;
  m_dim_sizes_outer_out     = i_dim_sizes_outer_out;
  m_loop_ids_ext = i_loop_ids_ext;
  m_dim_ids_left  = i_dim_ids_left;
  m_dim_ids_right = i_dim_ids_right;
  m_dim_ids_out   = i_dim_ids_out;
  m_dim_ids_permute_left  = i_dim_ids_permute_left;
  m_dim_ids_permute_right = i_dim_ids_permute_right;
  m_memory = i_memory;
  m_dtype_left  = i_dtype_left;
  m_dtype_right = i_dtype_right;
  m_dtype_comp  = i_dtype_comp;
  m_dtype_out   = i_dtype_out;
  m_ktype_first_touch = i_ktype_first_touch;
  m_ktype_main        = i_ktype_main;
  m_ktype_last_touch  = i_ktype_last_touch;
  m_num_threads = i_num_threads;
  m_compiled = false;
}

einsum_ir::err_t einsum_ir::backend::BinaryContraction::compile_base() {
  if(    m_dim_sizes_inner == nullptr
      || ( m_num_dims_left  > 0 && m_dim_ids_left  == nullptr )
      || ( m_num_dims_right > 0 && m_dim_ids_right == nullptr )
      || ( m_num_dims_out   > 0 && m_dim_ids_out   == nullptr ) ) {
    return err_t::COMPILATION_FAILED;
  }

  dim_types_ids( m_num_dims_left, m_num_dims_right, m_num_dims_out,
                 m_dim_ids_left, m_dim_ids_right, m_dim_ids_out,
                 &m_dim_types_out,
                 &m_dim_ids_c, &m_dim_ids_m, &m_dim_ids_n,
                 &m_dim_ids_k, &m_dim_ids_i, &m_dim_ids_j );

  m_num_dims_c = m_dim_ids_c.size();
  m_num_dims_m = m_dim_ids_m.size();
  m_num_dims_n = m_dim_ids_n.size();
  m_num_dims_k = m_dim_ids_k.size();
  m_num_dims_i = m_dim_ids_i.size();
  m_num_dims_j = m_dim_ids_j.size();

  auto sizes_of = [this]( std::vector< int64_t > const & i_ids, std::vector< int64_t > & o_sizes ) {
    o_sizes.resize( i_ids.size() );
    for( std::size_t l_i = 0; l_i < i_ids.size(); l_i++ ) {
      o_sizes[l_i] = m_dim_sizes_inner->at( i_ids[l_i] );
    }
  };
  try {
    sizes_of( m_dim_ids_c, m_sizes_c );
    sizes_of( m_dim_ids_m, m_sizes_m );
    sizes_of( m_dim_ids_n, m_sizes_n );
    sizes_of( m_dim_ids_k, m_sizes_k );
    sizes_of( m_dim_ids_i, m_sizes_i );
    sizes_of( m_dim_ids_j, m_sizes_j );
  }
  catch( std::out_of_range const & ) {
    return err_t::COMPILATION_FAILED;
  }

  m_dim_types.clear();
  for( int64_t l_id : m_dim_ids_c ) m_dim_types.insert( { l_id, C } );
  for( int64_t l_id : m_dim_ids_m ) m_dim_types.insert( { l_id, M } );
  for( int64_t l_id : m_dim_ids_n ) m_dim_types.insert( { l_id, N } );
  for( int64_t l_id : m_dim_ids_k ) m_dim_types.insert( { l_id, K } );

  // the external loop order is recorded but, as in the reference, not used
  if( m_loop_ids_ext != nullptr ) {
    m_loop_ids_int.assign( m_loop_ids_ext->begin(), m_loop_ids_ext->end() );
  }
  return err_t::SUCCESS;
}

int64_t einsum_ir::backend::BinaryContraction::num_ops() {
  int64_t l_c = 1, l_m = 1, l_n = 1, l_k = 1;
  for( int64_t l_s : m_sizes_c ) l_c *= l_s;
  for( int64_t l_s : m_sizes_m ) l_m *= l_s;
  for( int64_t l_s : m_sizes_n ) l_n *= l_s;
  for( int64_t l_s : m_sizes_k ) l_k *= l_s;

  int64_t l_ops = 2 * l_c * l_m * l_n * l_k;
  if( m_ktype_main == kernel_t::CPX_MADD ) {
    l_ops *= 2;
  }
  if( m_ktype_first_touch == ZERO || m_ktype_first_touch == CPX_ZERO ) {
    l_ops -= l_c * l_m * l_n;
  }
  return l_ops;
}
