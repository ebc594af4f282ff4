// extern "C" entry points of libeinsum_ir_hip.so (declared in
// include/einsum_ir_hip.h).  Thin: argument checks, plan ownership, error
// strings; planning and kernels live in contract_plan.cpp / permute.hip.
#include "etir_internal.h"
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace etir {

namespace {
thread_local std::string t_last_error;
}

void set_error( std::string const & msg ) {
  t_last_error = msg;
}

int fail( int code, std::string const & msg ) {
  t_last_error = msg;
  return code;
}

}  // namespace etir

using etir::fail;

extern "C" {

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
                                 etir_plan_t   * plan ) {
  if( plan == nullptr ) return fail( ETIR_UNDEFINED_ERROR, "plan output pointer is null" );
  *plan = nullptr;
  int l_device = 0;
  ETIR_HIP_CHECK( hipGetDevice( &l_device ) );
  etir_plan_s * l_plan = new etir_plan_s();
  l_plan->kind = 1;
  l_plan->device = l_device;
  int l_err = etir::plan_contraction( num_loops, dim_types, sizes,
                                      strides_left, strides_right, strides_out_aux, strides_out,
                                      dtype_left, dtype_right, dtype_comp, dtype_out,
                                      ktype_first_touch, ktype_main, ktype_last_touch,
                                      l_plan->cont );
  if( l_err != ETIR_SUCCESS ) {
    etir::release_contraction( l_plan->cont );
    delete l_plan;
    return l_err;
  }
  *plan = l_plan;
  return ETIR_SUCCESS;
}

int etir_hip_contraction_execute( etir_plan_t  plan,
                                  void const * left,
                                  void const * right,
                                  void const * out_aux,
                                  void       * out,
                                  void       * stream ) {
  if( plan == nullptr || plan->kind != 1 ) {
    return fail( ETIR_CALLED_BEFORE_COMPILATION, "not a contraction plan" );
  }
  return etir::launch_contraction( plan->cont, left, right, out_aux, out,
                                   reinterpret_cast< hipStream_t >( stream ) );
}

int etir_hip_permute_create( int64_t         num_dims,
                             int64_t const * sizes,
                             int64_t const * strides_in,
                             int64_t const * strides_out,
                             int32_t         dtype_in,
                             int32_t         dtype_comp,
                             int32_t         dtype_out,
                             int32_t         ktype_main,
                             etir_plan_t   * plan ) {
  if( plan == nullptr ) return fail( ETIR_UNDEFINED_ERROR, "plan output pointer is null" );
  *plan = nullptr;
  if( dtype_in != dtype_out || ( dtype_comp != dtype_in && dtype_comp != ETIR_UNDEFINED_DTYPE ) ) {
    return fail( ETIR_INVALID_DTYPE, "permute: input, compute and output dtypes must match" );
  }
  int l_device = 0;
  ETIR_HIP_CHECK( hipGetDevice( &l_device ) );
  etir_plan_s * l_plan = new etir_plan_s();
  l_plan->kind = 2;
  l_plan->device = l_device;
  int l_err = etir::plan_permute( num_dims, sizes, strides_in, strides_out,
                                  dtype_in, ktype_main, l_plan->perm );
  if( l_err != ETIR_SUCCESS ) {
    delete l_plan;
    return l_err;
  }
  *plan = l_plan;
  return ETIR_SUCCESS;
}

int etir_hip_permute_execute( etir_plan_t  plan,
                              void const * in,
                              void       * out,
                              void       * stream ) {
  if( plan == nullptr || plan->kind != 2 ) {
    return fail( ETIR_CALLED_BEFORE_COMPILATION, "not a permutation plan" );
  }
  return etir::launch_permute( plan->perm, in, out, reinterpret_cast< hipStream_t >( stream ) );
}

int etir_hip_plan_destroy( etir_plan_t plan ) {
  if( plan == nullptr ) return ETIR_SUCCESS;
  if( plan->kind == 1 ) etir::release_contraction( plan->cont );
  if( plan->kind == 2 ) etir::release_permute( plan->perm );
  delete plan;
  return ETIR_SUCCESS;
}

int etir_hip_plan_describe( etir_plan_t plan, char * buf, int64_t len ) {
  if( plan == nullptr || buf == nullptr || len <= 0 ) {
    return fail( ETIR_UNDEFINED_ERROR, "describe: invalid arguments" );
  }
  std::string l_s;
  if( plan->kind == 1 ) {
    l_s = plan->cont.desc;
  }
  else {
    static char const * l_modes[] = { "fill", "transpose", "copy_vec", "gather", "tiled", "reg4", "rows" };
    etir::PermutePlan const & p = plan->perm;
    char l_tmp[256];
    std::snprintf( l_tmp, sizeof( l_tmp ), "permute %s dims=%d elems=%lld vec=%d",
                   l_modes[ (int) p.mode ], p.num_dims, (long long) p.num_elements, p.args.vec_ok );
    l_s = l_tmp;
    if( p.mode == etir::PermMode::TILED ) {
      l_s += " tile=[";
      for( int l_k = 0; l_k < p.args.tile_nd; l_k++ ) {
        l_s += ( l_k ? "," : "" ) + std::to_string( p.args.tile_ext[l_k] );
      }
      l_s += "] pad=" + std::to_string( p.args.tile_pad );
    }
    if( p.mode == etir::PermMode::TRANSPOSE && p.tr_shape != 0 ) {
      l_s += p.tr_shape == 1 ? " tile=128x32" : p.tr_shape == 2 ? " tile=32x128"
           : p.tr_shape == 3 ? " tile=128x64 v16" : " tile=128x32 v16";
      if( p.args.o1_size > 0 ) l_s += " fold=" + std::to_string( p.args.o1_size ) + "x" + std::to_string( p.args.size_o / p.args.o1_size );
    }
    if( p.mode == etir::PermMode::ROWS ) {
      l_s += " row=" + std::to_string( p.rows_len ) + "/" + std::to_string( p.rows_vw )
           + " tile=" + std::to_string( p.args.rows_ex ) + "x" + std::to_string( p.args.rows_ey )
           + " pitch=" + std::to_string( p.args.rows_pitch );
    }
    if( p.mode == etir::PermMode::REG4 ) {
      l_s += " i=" + std::to_string( p.args.size_i ) + " o=" + std::to_string( p.args.size_o )
           + " c=" + std::to_string( p.args.c_size ) + "/" + std::to_string( p.args.c_chunk )
           + " b=" + std::to_string( p.reg4_vb )
           + " t=" + std::to_string( p.reg4_threads ) + "x" + std::to_string( p.reg4_cpt )
           + ( p.reg4_direct ? " direct" : "" );
    }
  }
  std::strncpy( buf, l_s.c_str(), (std::size_t) len - 1 );
  buf[len - 1] = '\0';
  return ETIR_SUCCESS;
}

int64_t etir_hip_plan_flops( etir_plan_t plan ) {
  if( plan == nullptr || plan->kind != 1 ) return 0;
  return plan->cont.flops;
}

int64_t etir_hip_plan_bytes( etir_plan_t plan ) {
  if( plan == nullptr ) return 0;
  if( plan->kind == 1 ) return plan->cont.bytes;
  etir::PermutePlan const & p = plan->perm;
  int64_t l_rw = ( p.ktype == ETIR_KTYPE_ZERO ) ? 1 : ( p.ktype == ETIR_KTYPE_ADD ? 3 : 2 );
  return l_rw * p.elem_bytes * p.num_elements;
}

char const * etir_hip_last_error( void ) {
  return etir::t_last_error.c_str();
}

int etir_hip_malloc( void ** ptr, int64_t num_bytes ) {
  if( ptr == nullptr || num_bytes < 0 ) return fail( ETIR_UNDEFINED_ERROR, "malloc: invalid arguments" );
  *ptr = nullptr;
  if( num_bytes == 0 ) return ETIR_SUCCESS;
  ETIR_HIP_CHECK( hipMalloc( ptr, (std::size_t) num_bytes ) );
  return ETIR_SUCCESS;
}

int etir_hip_free( void * ptr ) {
  if( ptr == nullptr ) return ETIR_SUCCESS;
  ETIR_HIP_CHECK( hipFree( ptr ) );
  return ETIR_SUCCESS;
}

int etir_hip_memcpy_h2d( void * dst, void const * src, int64_t num_bytes ) {
  if( num_bytes <= 0 ) return ETIR_SUCCESS;
  ETIR_HIP_CHECK( hipMemcpy( dst, src, (std::size_t) num_bytes, hipMemcpyHostToDevice ) );
  return ETIR_SUCCESS;
}

int etir_hip_memcpy_d2h( void * dst, void const * src, int64_t num_bytes ) {
  if( num_bytes <= 0 ) return ETIR_SUCCESS;
  ETIR_HIP_CHECK( hipMemcpy( dst, src, (std::size_t) num_bytes, hipMemcpyDeviceToHost ) );
  return ETIR_SUCCESS;
}

int etir_hip_memcpy_d2d( void * dst, void const * src, int64_t num_bytes, void * stream ) {
  if( num_bytes <= 0 ) return ETIR_SUCCESS;
  ETIR_HIP_CHECK( hipMemcpyAsync( dst, src, (std::size_t) num_bytes, hipMemcpyDeviceToDevice,
                                  reinterpret_cast< hipStream_t >( stream ) ) );
  return ETIR_SUCCESS;
}

int etir_hip_memset( void * dst, int32_t value, int64_t num_bytes ) {
  if( num_bytes <= 0 ) return ETIR_SUCCESS;
  ETIR_HIP_CHECK( hipMemset( dst, value, (std::size_t) num_bytes ) );
  return ETIR_SUCCESS;
}

int etir_hip_synchronize( void * stream ) {
  if( stream == nullptr ) {
    ETIR_HIP_CHECK( hipDeviceSynchronize() );
  }
  else {
    ETIR_HIP_CHECK( hipStreamSynchronize( reinterpret_cast< hipStream_t >( stream ) ) );
  }
  return ETIR_SUCCESS;
}

int etir_hip_device_count( void ) {
  int l_n = 0;
  if( hipGetDeviceCount( &l_n ) != hipSuccess ) return 0;
  return l_n;
}

int etir_hip_pointer_is_device( void const * ptr ) {
  if( ptr == nullptr ) return 0;
  hipPointerAttribute_t l_a;
  if( hipPointerGetAttributes( &l_a, ptr ) != hipSuccess ) {
    // unknown to the runtime: pageable host memory
    (void) hipGetLastError();
    return 0;
  }
  if( l_a.type == hipMemoryTypeDevice || l_a.type == hipMemoryTypeManaged ) return 1;
  // pinned host memory the GPU reaches at the same address
  if( l_a.type == hipMemoryTypeHost && l_a.devicePointer == ptr ) return 1;
  return 0;
}

int etir_hip_stream_create( void ** stream ) {
  if( stream == nullptr ) return fail( ETIR_UNDEFINED_ERROR, "stream_create: invalid arguments" );
  *stream = nullptr;
  hipStream_t l_s = nullptr;
  ETIR_HIP_CHECK( hipStreamCreateWithFlags( &l_s, hipStreamNonBlocking ) );
  *stream = l_s;
  return ETIR_SUCCESS;
}

int etir_hip_stream_destroy( void * stream ) {
  if( stream == nullptr ) return ETIR_SUCCESS;
  ETIR_HIP_CHECK( hipStreamDestroy( reinterpret_cast< hipStream_t >( stream ) ) );
  return ETIR_SUCCESS;
}

int etir_hip_event_create( void ** event ) {
  if( event == nullptr ) return fail( ETIR_UNDEFINED_ERROR, "event_create: invalid arguments" );
  *event = nullptr;
  hipEvent_t l_ev = nullptr;
  ETIR_HIP_CHECK( hipEventCreateWithFlags( &l_ev, hipEventDisableTiming ) );
  *event = l_ev;
  return ETIR_SUCCESS;
}

int etir_hip_event_destroy( void * event ) {
  if( event == nullptr ) return ETIR_SUCCESS;
  ETIR_HIP_CHECK( hipEventDestroy( reinterpret_cast< hipEvent_t >( event ) ) );
  return ETIR_SUCCESS;
}

int etir_hip_event_record( void * event, void * stream ) {
  if( event == nullptr ) return fail( ETIR_UNDEFINED_ERROR, "event_record: invalid arguments" );
  ETIR_HIP_CHECK( hipEventRecord( reinterpret_cast< hipEvent_t >( event ), reinterpret_cast< hipStream_t >( stream ) ) );
  return ETIR_SUCCESS;
}

int etir_hip_stream_wait_event( void * stream, void * event ) {
  if( event == nullptr ) return fail( ETIR_UNDEFINED_ERROR, "stream_wait_event: invalid arguments" );
  ETIR_HIP_CHECK( hipStreamWaitEvent( reinterpret_cast< hipStream_t >( stream ), reinterpret_cast< hipEvent_t >( event ), 0 ) );
  return ETIR_SUCCESS;
}

int etir_hip_graph_begin( void * stream ) {
  if( stream == nullptr ) return fail( ETIR_UNDEFINED_ERROR, "graph_begin: the null stream cannot be recorded" );
  ETIR_HIP_CHECK( hipStreamBeginCapture( reinterpret_cast< hipStream_t >( stream ),
                                         hipStreamCaptureModeThreadLocal ) );
  return ETIR_SUCCESS;
}

int etir_hip_graph_end( void * stream, etir_graph_t * graph ) {
  if( stream == nullptr || graph == nullptr ) return fail( ETIR_UNDEFINED_ERROR, "graph_end: invalid arguments" );
  *graph = nullptr;
  hipGraph_t l_g = nullptr;
  ETIR_HIP_CHECK( hipStreamEndCapture( reinterpret_cast< hipStream_t >( stream ), &l_g ) );
  hipGraphExec_t l_exec = nullptr;
  hipError_t l_e = hipGraphInstantiate( &l_exec, l_g, nullptr, nullptr, 0 );
  (void) hipGraphDestroy( l_g );
  if( l_e != hipSuccess ) {
    return fail( ETIR_UNDEFINED_ERROR, std::string( "hipGraphInstantiate failed: " ) + hipGetErrorString( l_e ) );
  }
  *graph = reinterpret_cast< etir_graph_t >( l_exec );
  return ETIR_SUCCESS;
}

int etir_hip_graph_abort( void * stream ) {
  if( stream == nullptr ) return ETIR_SUCCESS;
  hipGraph_t l_g = nullptr;
  hipError_t l_e = hipStreamEndCapture( reinterpret_cast< hipStream_t >( stream ), &l_g );
  if( l_g != nullptr ) (void) hipGraphDestroy( l_g );
  (void) hipGetLastError();
  return l_e == hipSuccess ? ETIR_SUCCESS
                           : fail( ETIR_UNDEFINED_ERROR, std::string( "graph_abort: " ) + hipGetErrorString( l_e ) );
}

int etir_hip_graph_launch( etir_graph_t graph, void * stream ) {
  if( graph == nullptr ) return fail( ETIR_CALLED_BEFORE_COMPILATION, "graph_launch: no graph" );
  ETIR_HIP_CHECK( hipGraphLaunch( reinterpret_cast< hipGraphExec_t >( graph ),
                                  reinterpret_cast< hipStream_t >( stream ) ) );
  return ETIR_SUCCESS;
}

int etir_hip_graph_destroy( etir_graph_t graph ) {
  if( graph == nullptr ) return ETIR_SUCCESS;
  ETIR_HIP_CHECK( hipGraphExecDestroy( reinterpret_cast< hipGraphExec_t >( graph ) ) );
  return ETIR_SUCCESS;
}

}  // extern "C"
