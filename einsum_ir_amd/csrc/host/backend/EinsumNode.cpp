// Behaviour follows the reference's EinsumNode (reference src/backend/EinsumNode.cpp):
//   init overloads          :21-190  (environment switches EINSUM_IR_BACKEND,
//                                     EINSUM_IR_REORDER_DIMS, EINSUM_IR_PACK_INPUTS)
//   compile_recursive       :204-454 (swap_inputs, reorder, contraction, unary
//                                     copy, offsets, memory need, child order)
//   store_and_lock_data     :458-479
//   eval                    :496-540
//   compile_memory_usage    :560-578, requires_permutation :580-593
// Device-specific: one stream for the tree, device arena and device copies.
#include <stdexcept>
#include "EinsumNode.h"
#include "BinaryContractionFactory.h"
#include "BinaryContractionHip.h"
#include "BinaryPrimitives.h"
#include "HostStaging.h"
#include "Tensor.h"
#include "UnaryHip.h"
#include "einsum_ir_hip.h"
#include <algorithm>
#include <cstdio>
#include <functional>
#include <cstdlib>
#include <cstring>

namespace {
  bool env_flag( char const * i_name, bool i_default ) {
    char const * l_v = std::getenv( i_name );
    if( l_v == nullptr ) return i_default;
    return std::strcmp( l_v, "1" ) == 0 || std::strcmp( l_v, "true" ) == 0;
  }
}

einsum_ir::backend::EinsumNode::~EinsumNode() {
  // this node's own share of the schedule (the subtree's nodes free theirs)
  for( void * l_s : m_pool ) etir_hip_synchronize( l_s );
  etir_hip_event_destroy( m_ev_fork );
  etir_hip_event_destroy( m_ev_done );
  delete m_fork_memory;
  for( void * l_s : m_pool ) etir_hip_stream_destroy( l_s );
  delete m_unary;
  delete m_cont;
  if( m_data_ptr_int != nullptr ) {
    etir_hip_free( m_data_ptr_int );
  }
}

void einsum_ir::backend::EinsumNode::init( int64_t                              i_num_dims,
                                           int64_t                      const * i_dim_ids,
                                           std::map< int64_t, int64_t > const * i_dim_sizes_inner,
                                           std::map< int64_t, int64_t > const * i_dim_sizes_outer,
                                           data_t                               i_dtype,
                                           void                               * i_data_ptr,
                                           MemoryManager                      * i_memory ) {
  m_dtype = i_dtype;
  m_ktype_first_touch = kernel_t::UNDEFINED_KTYPE;
  m_ktype_main        = kernel_t::UNDEFINED_KTYPE;
  m_ktype_last_touch  = kernel_t::UNDEFINED_KTYPE;
  m_size = 0;
  m_num_dims = i_num_dims;
  m_dim_ids_ext = i_dim_ids;
  m_dim_ids_int.assign( i_dim_ids, i_dim_ids + i_num_dims );
  m_dim_sizes_inner = i_dim_sizes_inner;
  m_dim_sizes_outer = ( i_dim_sizes_outer != nullptr ) ? i_dim_sizes_outer : i_dim_sizes_inner;
  m_dim_sizes_aux_outer = nullptr;
  m_offsets_aux_ext = nullptr;
  m_offsets_ext = nullptr;
  m_children.clear();
  m_data_ptr_int = nullptr;
  m_data_ptr_active = nullptr;
  m_data_ptr_ext = i_data_ptr;
  m_data_ptr_aux_ext = nullptr;

  // backend selection: the reference's variable, with HIP as this library's backend
  m_btype_unary  = backend_t::HIP;
  m_btype_binary = backend_t::AUTO;
  if( char const * l_bt = std::getenv( "EINSUM_IR_BACKEND" ) ) {
    if(      std::strcmp( l_bt, "AUTO" )   == 0 ) m_btype_binary = backend_t::AUTO;
    else if( std::strcmp( l_bt, "HIP" )    == 0 ) m_btype_binary = backend_t::HIP;
    else if( std::strcmp( l_bt, "TPP" )    == 0 ) m_btype_binary = backend_t::TPP;
    else if( std::strcmp( l_bt, "BLAS" )   == 0 ) m_btype_binary = backend_t::BLAS;
    else if( std::strcmp( l_bt, "TBLIS" )  == 0 ) m_btype_binary = backend_t::TBLIS;
    else if( std::strcmp( l_bt, "SCALAR" ) == 0 ) m_btype_binary = backend_t::SCALAR;
  }
  m_reorder_dims = env_flag( "EINSUM_IR_REORDER_DIMS", true );
  m_pack_inputs  = env_flag( "EINSUM_IR_PACK_INPUTS", false );

  m_unary = nullptr;
  m_cont = nullptr;
  m_num_ops_node = 0;
  m_num_ops_children = 0;
  m_num_tasks_intra_op = 1;
  m_memory = i_memory;
  m_mem_id = 0;
  m_count_mem_users = 1;
  m_active_mem_users = 0;
  m_req_mem = 0;
  m_mem_subtree = 0;
  m_compiled = false;
  m_data_locked = false;
}

void einsum_ir::backend::EinsumNode::init( int64_t                              i_num_dims,
                                           int64_t                      const * i_dim_ids,
                                           std::map< int64_t, int64_t > const * i_dim_sizes_inner,
                                           std::map< int64_t, int64_t > const * i_dim_sizes_outer,
                                           data_t                               i_dtype,
                                           void                               * i_data_ptr,
                                           EinsumNode                         * i_child,
                                           MemoryManager                      * i_memory,
                                           int64_t                              i_num_threads ) {
  init( i_num_dims, i_dim_ids, i_dim_sizes_inner, i_dim_sizes_outer, i_dtype, i_data_ptr, i_memory );
  m_children.assign( 1, i_child );
  m_num_threads = i_num_threads;
}

void einsum_ir::backend::EinsumNode::init( int64_t                              i_num_dims,
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
                                           int64_t                              i_num_threads ) {
  init( i_num_dims, i_dim_ids, i_dim_sizes_inner, i_dim_sizes_outer, i_dtype, i_data_ptr, i_memory );
  m_dim_sizes_aux_outer = i_dim_sizes_aux_outer;
  m_offsets_aux_ext     = i_offsets_aux;
  m_offsets_ext         = i_offsets;
  m_data_ptr_aux_ext    = i_data_ptr_aux;
  m_ktype_first_touch   = i_ktype_first_touch;
  m_ktype_main          = i_ktype_main;
  m_ktype_last_touch    = i_ktype_last_touch;
  m_children = { i_left, i_right };
  m_num_threads = i_num_threads;
}

void einsum_ir::backend::EinsumNode::set_stream( void * i_stream ) {
  m_stream = i_stream;
  for( EinsumNode * l_ch : m_children ) l_ch->set_stream( i_stream );
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::compile() {
  err_t l_err = compile_recursive();
  if( l_err != err_t::SUCCESS ) return l_err;
  if( m_memory == nullptr ) return err_t::UNDEFINED_ERROR;
  release_schedule();
  l_err = schedule_streams();
  if( l_err != err_t::SUCCESS ) return l_err;
  compile_memory_usage();
  l_err = m_memory->alloc_all_memory();
  if( l_err != err_t::SUCCESS ) return l_err;
  return alloc_fork_memory();
}

void einsum_ir::backend::EinsumNode::assign( void * i_stream, MemoryManager * i_memory ) {
  m_stream = i_stream;
  m_memory = i_memory;
  if( m_cont != nullptr ) static_cast< BinaryContractionHip * >( m_cont )->set_stream( i_stream );
  if( m_unary != nullptr ) static_cast< UnaryHip * >( m_unary )->set_stream( i_stream );
  for( EinsumNode * l_ch : m_children ) l_ch->assign( i_stream, i_memory );
}

double einsum_ir::backend::EinsumNode::est_node_us() const {
  // per kernel: 5 us of launch and latency, then the longer of its flops at
  // 60 TFLOP/s and its tensors' bytes at 3 TB/s (a rough order, used only to
  // place subtrees)
  if( m_children.size() == 2 ) {
    double const l_bytes = double( m_size + m_children[0]->m_size + m_children[1]->m_size );
    return 5.0 + std::max( double( m_num_ops_node ) / 60.0e6, l_bytes / 3.0e6 );
  }
  return has_work() ? 5.0 + 2.0 * double( m_size ) / 3.0e6 : 0.0;
}

double einsum_ir::backend::EinsumNode::est_subtree_us() const {
  double l_t = est_node_us();
  for( EinsumNode const * l_ch : m_children ) l_t += l_ch->est_subtree_us();
  return l_t;
}

bool einsum_ir::backend::EinsumNode::has_work() const {
  if( !m_children.empty() ) return true;
  // a leaf: the copy into its internal layout (see eval_async)
  return !m_data_locked && m_data_ptr_ext != nullptr && m_req_mem != 0;
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::schedule_streams() {
  assign( m_stream, m_memory );
  // streams in the pool: at most this many forked subtrees run at once
  // (three: with the tree's stream, the four hardware queues a process gets
  // by default; more streams share queues and serialise behind each other's
  // waits -- einsum_benchmark MERA 0.53 ms/eval with 3 or 4, 0.56 with 5 or 6)
  int64_t l_max = 3;
  if( char const * l_env = std::getenv( "ETIR_TREE_STREAMS" ) ) l_max = std::max( 0, std::atoi( l_env ) );
  // a forked subtree's arena is its own: no fork above this peak
  int64_t const l_mem_max = int64_t( 1 ) << 30;

  // Depth first, in enqueue order, with estimated times (est_node_us): at a
  // binary node whose children both enqueue work, the child whose subtree
  // takes less time is forked onto the pool stream whose enqueued work ends
  // first (a new one while the pool has room), unless waiting for that
  // stream would take as long as running the other child first.  A stream is
  // not taken while a subtree enqueued on it is being scheduled; once that
  // subtree is placed, later forks may queue behind it.
  std::vector< void * > l_str = { m_stream };   // slot 0: the tree's stream
  std::vector< double > l_end = { 0.0 };        // estimated end of each slot's work
  std::vector< char >   l_busy = { 1 };
  err_t l_err = err_t::SUCCESS;
  std::function< double( EinsumNode *, std::size_t, double ) > l_sched =
    [&]( EinsumNode * i_n, std::size_t i_slot, double i_t ) -> double {
    double const l_own = i_n->est_node_us();
    int64_t l_p = -1;
    EinsumNode * l_f = nullptr;
    EinsumNode * l_o = nullptr;
    if( i_n->m_children.size() == 2 ) {
      EinsumNode * l_a = i_n->m_children[0];
      EinsumNode * l_b = i_n->m_children[1];
      bool const l_a_light = l_a->est_subtree_us() <= l_b->est_subtree_us();
      l_f = l_a_light ? l_a : l_b;
      l_o = l_a_light ? l_b : l_a;
      // a fork costs two event records and two waits: only subtrees that run
      // long enough to hide them (synthetic einsum_benchmark tree, one 6 us
      // node forked: 95.5 -> 98.5 us/eval)
      if(    l_f->has_work() && l_o->has_work() && l_f->m_mem_subtree <= l_mem_max
          && l_f->est_subtree_us() >= 10.0 ) {
        double l_best = 0.0;
        for( std::size_t l_k = 1; l_k < l_str.size(); l_k++ ) {
          if( !l_busy[l_k] && ( l_p < 0 || l_end[l_k] < l_best ) ) {
            l_p = (int64_t) l_k;
            l_best = l_end[l_k];
          }
        }
        if( ( l_p < 0 || l_best > i_t ) && (int64_t) l_str.size() - 1 < l_max ) {
          void * l_new = nullptr;
          if( etir_hip_stream_create( &l_new ) != ETIR_SUCCESS ) {
            l_err = err_t::UNDEFINED_ERROR;
            return i_t;
          }
          m_pool.push_back( l_new );
          l_str.push_back( l_new );
          l_end.push_back( 0.0 );
          l_busy.push_back( 0 );
          l_p = (int64_t) l_str.size() - 1;
          l_best = 0.0;
        }
        if( l_p >= 0 && std::max( i_t, l_best ) - i_t >= l_o->est_subtree_us() ) l_p = -1;
      }
    }
    if( l_p < 0 ) {
      double l_t = i_t;
      for( std::size_t l_c = 0; l_c < i_n->m_children.size(); l_c++ ) {
        l_t = l_sched( i_n->m_children[ i_n->m_exec_order[l_c] ], i_slot, l_t );
      }
      return l_t + l_own;
    }
    if(    etir_hip_event_create( &l_f->m_ev_fork ) != ETIR_SUCCESS
        || etir_hip_event_create( &l_f->m_ev_done ) != ETIR_SUCCESS ) {
      l_err = err_t::UNDEFINED_ERROR;
      return i_t;
    }
    l_f->m_forked = true;
    l_f->m_fork_memory = new MemoryManager();
    l_f->m_fork_memory->share_allocator( *m_memory );
    l_f->assign( l_str[l_p], l_f->m_fork_memory );
    l_busy[l_p] = 1;
    double const l_tf = l_sched( l_f, (std::size_t) l_p, std::max( i_t, l_end[l_p] ) );
    l_busy[l_p] = 0;
    l_end[l_p] = l_tf;
    double const l_to = l_sched( l_o, i_slot, i_t );
    return std::max( l_tf, l_to ) + l_own;
  };
  l_sched( this, 0, 0.0 );
  return l_err;
}

void einsum_ir::backend::EinsumNode::release_schedule() {
  // nothing may still run on the pool when the arenas go
  for( void * l_s : m_pool ) etir_hip_synchronize( l_s );
  for( EinsumNode * l_ch : m_children ) l_ch->release_schedule();
  etir_hip_event_destroy( m_ev_fork );
  etir_hip_event_destroy( m_ev_done );
  m_ev_fork = nullptr;
  m_ev_done = nullptr;
  delete m_fork_memory;
  m_fork_memory = nullptr;
  m_forked = false;
  for( void * l_s : m_pool ) etir_hip_stream_destroy( l_s );
  m_pool.clear();
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::alloc_fork_memory() {
  if( m_fork_memory != nullptr ) {
    err_t l_err = m_fork_memory->alloc_all_memory();
    if( l_err != err_t::SUCCESS ) return l_err;
  }
  for( EinsumNode * l_ch : m_children ) {
    err_t l_err = l_ch->alloc_fork_memory();
    if( l_err != err_t::SUCCESS ) return l_err;
  }
  return err_t::SUCCESS;
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::compile_recursive() {
  err_t l_err = err_t::UNDEFINED_ERROR;

  // backend of the contraction: AUTO resolves to HIP, complex kernels
  // included (the reference sends those to its BLAS backend,
  // EinsumNode.cpp:207-213; the HIP backend runs them natively)
  if( m_btype_binary == backend_t::AUTO ) {
    m_btype_binary = backend_t::HIP;
  }
  if( !BinaryContractionFactory::supports( m_btype_binary ) ) {
    return err_t::INVALID_BACKEND;
  }

  try {
    m_size = Tensor::size( ce_n_bytes( m_dtype ), m_num_dims, m_dim_ids_ext, *m_dim_sizes_outer );
  }
  catch( std::out_of_range const & ) {
    return err_t::COMPILATION_FAILED;
  }

  if( m_children.size() == 2 ) {
    // the left operand must provide the output's fastest non-C dim
    if( BinaryPrimitives::swap_inputs( m_children[0]->m_num_dims, m_children[1]->m_num_dims, m_num_dims,
                                       m_children[0]->m_dim_ids_ext, m_children[1]->m_dim_ids_ext,
                                       m_dim_ids_int.data() ) ) {
      std::swap( m_children[0], m_children[1] );
    }

    // internal dim orders of the children: the GPU kernel's layouts for the
    // HIP backend (leaves keep theirs when the kernel reads them well as they
    // are), the backend's tensor ordering otherwise
    if( m_reorder_dims && m_btype_binary == backend_t::HIP ) {
      int64_t const l_esz = ce_n_bytes( m_children[0]->m_dtype );
      l_err = BinaryPrimitives::reorder_gpu( m_children[0]->m_children.empty(),
                                             m_children[1]->m_children.empty(),
                                             16 / l_esz, l_esz, int64_t( 2 ) << 20,
                                             m_children[0]->m_num_dims, m_children[1]->m_num_dims, m_num_dims,
                                             m_dim_sizes_inner,
                                             m_children[0]->m_dim_ids_int.data(),
                                             m_children[1]->m_dim_ids_int.data(),
                                             m_dim_ids_int.data() );
      if( l_err != err_t::SUCCESS ) return l_err;
    }
    else if( m_reorder_dims ) {
      BinaryPrimitives l_prims;
      l_prims.init( m_dtype, m_btype_binary );
      l_err = l_prims.reorder( m_btype_binary,
                               m_children[0]->m_num_dims, m_children[1]->m_num_dims, m_num_dims,
                               m_dim_sizes_inner,
                               m_children[0]->m_dim_ids_int.data(),
                               m_children[1]->m_dim_ids_int.data(),
                               m_dim_ids_int.data() );
      if( l_err != err_t::SUCCESS ) return l_err;
    }

    delete m_cont;
    m_cont = BinaryContractionFactory::create( m_btype_binary );
    m_cont->init( m_children[0]->m_num_dims, m_children[1]->m_num_dims, m_num_dims,
                  m_dim_sizes_inner,
                  m_children[0]->m_dim_sizes_outer, m_children[1]->m_dim_sizes_outer,
                  m_dim_sizes_aux_outer, m_dim_sizes_outer,
                  nullptr,
                  m_children[0]->m_dim_ids_int.data(), m_children[1]->m_dim_ids_int.data(),
                  m_dim_ids_int.data(),
                  nullptr, nullptr,
                  m_memory,
                  m_children[0]->m_dtype, m_children[1]->m_dtype,
                  ( m_dtype == data_t::BF16 ) ? data_t::FP32 : m_dtype,
                  m_dtype,
                  m_ktype_first_touch, m_ktype_main, m_ktype_last_touch,
                  m_num_threads );
    static_cast< BinaryContractionHip * >( m_cont )->set_stream( m_stream );
    static_cast< BinaryContractionHip * >( m_cont )->m_cpx_dim_id = m_cpx_dim_id;
    l_err = m_cont->compile();
    if( l_err != err_t::SUCCESS ) return l_err;
  }

  // unary copy: external layout -> internal layout (leaves), or the child's
  // layout -> this node's layout (one child)
  delete m_unary;
  UnaryHip * l_unary = new UnaryHip();
  m_unary = l_unary;
  l_unary->set_stream( m_stream );
  if( m_children.size() != 1 ) {
    m_unary->init( m_num_dims, m_dim_sizes_outer, m_dim_ids_ext, m_dim_ids_int.data(),
                   m_dtype, m_dtype, m_dtype, kernel_t::COPY, 1 );
  }
  else {
    // the child's data is in its internal layout; the parent reads this node's
    // data in this node's internal layout (both equal the external ones unless
    // a binary parent reordered them)
    m_unary->init( m_num_dims, m_dim_sizes_outer, m_children[0]->m_dim_ids_int.data(), m_dim_ids_int.data(),
                   m_dtype, m_dtype, m_dtype, kernel_t::COPY, 1 );
  }
  l_err = m_unary->compile();
  if( l_err != err_t::SUCCESS ) return l_err;

  // byte offsets of the node's data inside larger (outer) tensors
  auto offset_bytes = [this]( std::map< int64_t, int64_t > const * i_offsets,
                              std::map< int64_t, int64_t > const * i_outer ) -> int64_t {
    int64_t l_off = 0;
    int64_t l_stride = 1;
    for( int64_t l_di = m_num_dims - 1; l_di >= 0; l_di-- ) {
      int64_t const l_id = m_dim_ids_int[l_di];
      auto l_it = i_offsets->find( l_id );
      if( l_it != i_offsets->end() ) l_off += l_stride * l_it->second;
      l_stride *= i_outer->at( l_id );
    }
    return l_off * ce_n_bytes( m_dtype );
  };
  if( m_offsets_aux_ext != nullptr && m_dim_sizes_aux_outer != nullptr ) {
    m_offset_aux_bytes = offset_bytes( m_offsets_aux_ext, m_dim_sizes_aux_outer );
  }
  if( m_offsets_ext != nullptr ) {
    m_offset_bytes = offset_bytes( m_offsets_ext, m_dim_sizes_outer );
  }

  // memory need: intermediates and permuted inputs live in the arena
  m_req_mem = ( m_data_ptr_ext == nullptr || requires_permutation() ) ? m_size : 0;

  // children, and the order that minimises the peak memory of the subtree
  if( m_children.size() > 1 ) {
    for( EinsumNode * l_ch : m_children ) {
      l_err = l_ch->compile_recursive();
      if( l_err != err_t::SUCCESS ) return l_err;
    }
    int64_t const l_m0 = m_children[0]->m_mem_subtree;
    int64_t const l_m1 = m_children[1]->m_mem_subtree;
    int64_t const l_first0 = std::max( l_m0, l_m1 + m_children[0]->m_req_mem );
    int64_t const l_first1 = std::max( l_m1, l_m0 + m_children[1]->m_req_mem );
    if( l_first0 <= l_first1 ) {
      m_mem_subtree = l_first0;
      m_exec_order = { 0, 1 };
    }
    else {
      m_mem_subtree = l_first1;
      m_exec_order = { 1, 0 };
    }
    m_mem_subtree = std::max( m_mem_subtree,
                              m_req_mem + m_children[0]->m_req_mem + m_children[1]->m_req_mem );
  }
  else if( m_children.size() == 1 ) {
    l_err = m_children[0]->compile_recursive();
    if( l_err != err_t::SUCCESS ) return l_err;
    m_exec_order = { 0 };
    m_mem_subtree = std::max( m_children[0]->m_mem_subtree, m_req_mem + m_children[0]->m_req_mem );
  }
  else {
    m_mem_subtree = m_req_mem;
  }

  m_num_ops_node = ( m_children.size() > 1 ) ? m_cont->num_ops() : 0;
  m_num_ops_children = 0;
  for( EinsumNode * l_ch : m_children ) {
    m_num_ops_children += l_ch->m_num_ops_node + l_ch->m_num_ops_children;
  }

  m_compiled = true;
  return err_t::SUCCESS;
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::store_and_lock_data() {
  if( !m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  if( m_data_ptr_ext == nullptr ) return err_t::NO_DATA_PTR_PROVIDED;
  if( m_data_ptr_int == nullptr ) {
    if( etir_hip_malloc( &m_data_ptr_int, m_size ) != ETIR_SUCCESS ) return err_t::UNDEFINED_ERROR;
  }
  UnaryHip * l_unary = static_cast< UnaryHip * >( m_unary );
  HostStaging l_st;   // a host tensor is read through a device copy
  void const * l_src = l_st.stage( m_data_ptr_ext, m_size, true, false );
  if( l_st.error() != err_t::SUCCESS ) return l_st.error();
  err_t l_err = l_unary->eval_async( l_src, m_data_ptr_int );
  if( l_err != err_t::SUCCESS ) return l_err;
  if( etir_hip_synchronize( m_stream ) != ETIR_SUCCESS ) return err_t::UNDEFINED_ERROR;
  m_data_locked = true;
  return err_t::SUCCESS;
}

void einsum_ir::backend::EinsumNode::stage_ext( HostStaging & io_staging,
                                                std::vector< std::pair< void **, void * > > & io_saved ) {
  for( EinsumNode * l_ch : m_children ) l_ch->stage_ext( io_staging, io_saved );
  // a locked node reads its device copy, not the external tensor
  if( m_data_ptr_ext != nullptr && !m_data_locked ) {
    // inputs are read; a computed tensor is written, and copied in as well
    // (accumulating touches read it, elements outside the node's view keep
    // their values)
    bool const l_written = !m_children.empty();
    void * l_dev = io_staging.stage( m_data_ptr_ext, m_size, true, l_written );
    if( l_dev != m_data_ptr_ext ) {
      io_saved.emplace_back( &m_data_ptr_ext, m_data_ptr_ext );
      m_data_ptr_ext = l_dev;
    }
  }
  if( m_data_ptr_aux_ext != nullptr ) {
    int64_t l_bytes = m_size;
    if( m_dim_sizes_aux_outer != nullptr ) {
      try {
        l_bytes = Tensor::size( ce_n_bytes( m_dtype ), m_num_dims, m_dim_ids_ext, *m_dim_sizes_aux_outer );
      }
      catch( std::out_of_range const & ) {
        l_bytes = m_size;
      }
    }
    void * l_dev = io_staging.stage( m_data_ptr_aux_ext, l_bytes, true, false );
    if( l_dev != m_data_ptr_aux_ext ) {
      io_saved.emplace_back( &m_data_ptr_aux_ext, m_data_ptr_aux_ext );
      m_data_ptr_aux_ext = l_dev;
    }
  }
}

void einsum_ir::backend::EinsumNode::restore_ext( std::vector< std::pair< void **, void * > > const & i_saved ) {
  for( auto const & l_s : i_saved ) *l_s.first = l_s.second;
}

bool einsum_ir::backend::EinsumNode::has_host_ext() const {
  for( EinsumNode const * l_ch : m_children ) {
    if( l_ch->has_host_ext() ) return true;
  }
  if( m_data_ptr_ext != nullptr && !m_data_locked && etir_hip_pointer_is_device( m_data_ptr_ext ) != 1 ) {
    return true;
  }
  return m_data_ptr_aux_ext != nullptr && etir_hip_pointer_is_device( m_data_ptr_aux_ext ) != 1;
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::unlock_data() {
  if( m_data_ptr_ext == nullptr ) return err_t::NO_DATA_PTR_PROVIDED;
  if( m_data_ptr_int != nullptr ) {
    etir_hip_free( m_data_ptr_int );
    m_data_ptr_int = nullptr;
  }
  m_data_locked = false;
  return err_t::SUCCESS;
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::eval_async() {
  return eval_tree( true );
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::eval_one_stream_async() {
  kernels_on( m_stream );
  err_t const l_err = eval_tree( false );
  kernels_on( nullptr );
  return l_err;
}

void einsum_ir::backend::EinsumNode::kernels_on( void * i_stream ) {
  void * l_s = ( i_stream != nullptr ) ? i_stream : m_stream;
  if( m_cont != nullptr ) static_cast< BinaryContractionHip * >( m_cont )->set_stream( l_s );
  if( m_unary != nullptr ) static_cast< UnaryHip * >( m_unary )->set_stream( l_s );
  for( EinsumNode * l_ch : m_children ) l_ch->kernels_on( i_stream );
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::eval_tree( bool i_forks ) {
  if( !m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  // forked children first, each on its own stream from this point of this
  // node's stream on; then the others on this stream; then this stream waits
  // for the forked ones
  auto forked = [i_forks]( EinsumNode const * i_c ) { return i_forks && i_c->m_forked && i_c->has_work(); };
  bool l_joins = false;
  for( std::size_t l_ch = 0; l_ch < m_children.size(); l_ch++ ) {
    EinsumNode * l_c = m_children[ m_exec_order[l_ch] ];
    if( !forked( l_c ) ) continue;
    if(    etir_hip_event_record( l_c->m_ev_fork, m_stream ) != ETIR_SUCCESS
        || etir_hip_stream_wait_event( l_c->m_stream, l_c->m_ev_fork ) != ETIR_SUCCESS ) {
      return err_t::UNDEFINED_ERROR;
    }
    err_t l_err = l_c->eval_tree( i_forks );
    if( l_err != err_t::SUCCESS ) return l_err;
    if( etir_hip_event_record( l_c->m_ev_done, l_c->m_stream ) != ETIR_SUCCESS ) return err_t::UNDEFINED_ERROR;
    l_joins = true;
  }
  for( std::size_t l_ch = 0; l_ch < m_children.size(); l_ch++ ) {
    EinsumNode * l_c = m_children[ m_exec_order[l_ch] ];
    if( forked( l_c ) ) continue;
    err_t l_err = l_c->eval_tree( i_forks );
    if( l_err != err_t::SUCCESS ) return l_err;
  }
  if( l_joins ) {
    for( EinsumNode * l_c : m_children ) {
      if( !forked( l_c ) ) continue;
      if( etir_hip_stream_wait_event( m_stream, l_c->m_ev_done ) != ETIR_SUCCESS ) return err_t::UNDEFINED_ERROR;
    }
  }

  if( m_data_locked ) {
    m_data_ptr_active = m_data_ptr_int;
  }
  else if( m_mem_id ) {
    m_data_ptr_active = m_memory->get_mem_ptr( m_mem_id );
    m_active_mem_users = m_count_mem_users;
  }
  else {
    m_data_ptr_active = m_data_ptr_ext;
  }

  UnaryHip * l_unary = static_cast< UnaryHip * >( m_unary );
  if( m_children.size() != 1 ) {
    if( !m_data_locked && m_data_ptr_ext != nullptr && m_req_mem != 0 ) {
      err_t l_err = l_unary->eval_async( m_data_ptr_ext, m_data_ptr_active );
      if( l_err != err_t::SUCCESS ) return l_err;
    }
  }
  else {
    err_t l_err = l_unary->eval_async( m_children[0]->m_data_ptr_active, m_data_ptr_active );
    if( l_err != err_t::SUCCESS ) return l_err;
  }

  if( m_children.size() == 2 ) {
    void const * l_aux = ( m_data_ptr_aux_int != nullptr ) ? m_data_ptr_aux_int : m_data_ptr_aux_ext;
    if( l_aux != nullptr ) l_aux = static_cast< char const * >( l_aux ) + m_offset_aux_bytes;
    void * l_out = static_cast< char * >( m_data_ptr_active ) + m_offset_bytes;
    err_t l_err = static_cast< BinaryContractionHip * >( m_cont )->contract_async( m_children[0]->m_data_ptr_active,
                                                                                   m_children[1]->m_data_ptr_active,
                                                                                   l_aux, l_out );
    if( l_err != err_t::SUCCESS ) return l_err;
  }
  return err_t::SUCCESS;
}

einsum_ir::err_t einsum_ir::backend::EinsumNode::eval_sync() {
  if( !m_compiled ) return err_t::CALLED_BEFORE_COMPILATION;
  // host tensors (the reference's callers pass them) take part through device
  // copies made for this evaluation
  HostStaging l_st;
  std::vector< std::pair< void **, void * > > l_saved;
  stage_ext( l_st, l_saved );
  err_t l_err = l_st.error();
  if( l_err == err_t::SUCCESS ) l_err = eval_async();
  if( l_err == err_t::SUCCESS && etir_hip_synchronize( m_stream ) != ETIR_SUCCESS ) {
    l_err = err_t::UNDEFINED_ERROR;
  }
  if( l_err == err_t::SUCCESS && l_st.active() ) l_err = l_st.finish();
  restore_ext( l_saved );
  return l_err;
}

void einsum_ir::backend::EinsumNode::eval() {
  err_t const l_err = eval_sync();
  if( l_err != err_t::SUCCESS ) {
    std::fprintf( stderr, "einsum_ir: tree evaluation failed (%d): %s\n", (int) l_err, etir_hip_last_error() );
  }
}

int64_t einsum_ir::backend::EinsumNode::num_ops( bool i_children ) {
  return m_num_ops_node + ( i_children ? m_num_ops_children : 0 );
}

void einsum_ir::backend::EinsumNode::cancel_memory_reservation() {
  m_active_mem_users--;
  if( m_active_mem_users <= 0 && m_mem_id ) {
    m_memory->remove_reservation( m_mem_id );
  }
}

void einsum_ir::backend::EinsumNode::compile_memory_usage() {
  m_memory->m_layer_id++;
  for( std::size_t l_ch = 0; l_ch < m_children.size(); l_ch++ ) {
    m_children[ m_exec_order[l_ch] ]->compile_memory_usage();
  }
  m_memory->m_layer_id--;

  if( m_req_mem ) {
    m_mem_id = m_memory->reserve_memory( m_req_mem );
  }
  // planning walk: the children's data is released once this node is planned
  for( EinsumNode * l_ch : m_children ) {
    l_ch->m_active_mem_users = l_ch->m_count_mem_users;
    l_ch->cancel_memory_reservation();
  }
}

bool einsum_ir::backend::EinsumNode::requires_permutation() {
  if( m_dim_ids_ext == m_dim_ids_int.data() || m_data_ptr_ext == nullptr ) return false;
  for( int64_t l_di = 0; l_di < m_num_dims; l_di++ ) {
    if( m_dim_ids_ext[l_di] != m_dim_ids_int[l_di] ) return true;
  }
  return false;
}
