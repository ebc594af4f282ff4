// bench_binary: one binary contraction through BinaryContractionHip.
//
//   bench_binary einsum_string dimension_sizes [dtype [loop_order]]
//
// Arguments and report follow reference src/bench_binary.cpp:212-408: the
// expression in single-character or standard format, sizes in ascending
// order of the dimension ids, dtype FP32 or FP64 (BF16 is additive: bf16
// inputs, fp32 accumulation and output), a loop order (accepted and handed to
// init; one kernel grid runs every loop).  Data as the reference makes it:
// left uniform [0,1), right ones.  Tensors live on the GPU; times are per
// call of contract_async over a run of calls (one warm-up).  The result is
// checked against a float64 host evaluation (relative Frobenius error: fp32
// 1e-5, fp64 1e-12, bf16 2e-3); the exit status is 1 when it is not met.
#include <cstdlib>

#include "bench_util.h"
#include "backend/BinaryContractionHip.h"
#include "backend/MemoryManager.h"
#include "frontend/EinsumExpressionAscii.h"

using namespace etir_bench;
using einsum_ir::frontend::EinsumExpressionAscii;

namespace {

int usage() {
  std::cerr << "usage: bench_binary einsum_string dimension_sizes [dtype [loop_order]]\n"
               "  einsum_string    a binary contraction, e.g. \"abc,acdb->abd\" or \"[a,b,c],[a,c,d,b]->[a,b,d]\"\n"
               "  dimension_sizes  sizes in ascending order of the dimension ids, e.g. \"32,8,4,2\"\n"
               "  dtype            FP32 (default), FP64 or BF16\n"
               "  loop_order       dimension names, e.g. \"a,b,c,d\" (the GPU plan runs all loops in one grid)"
            << std::endl;
  return EXIT_FAILURE;
}

int run( int i_argc, char * i_argv[] ) {
  std::string const l_arg( i_argv[1] );
  std::string l_std, l_schar;
  if( !l_arg.empty() && l_arg[0] == '[' ) {
    l_std = l_arg;
    EinsumExpressionAscii::standard_to_schar( l_std, l_schar );
  }
  else {
    l_schar = l_arg;
    EinsumExpressionAscii::schar_to_standard( l_schar, l_std );
  }
  std::vector< std::string > l_tensors;
  EinsumExpressionAscii::parse_tensors( l_std, l_tensors );
  if( l_tensors.size() != 3 ) {
    std::cerr << "Einsum string is not a binary contraction" << std::endl;
    return EXIT_FAILURE;
  }
  std::cout << "parsed tensors:" << std::endl;
  for( auto const & l_t : l_tensors ) std::cout << "  " << l_t << std::endl;

  std::map< std::string, int64_t > l_ids;
  EinsumExpressionAscii::parse_dim_ids( l_std, l_ids );
  std::cout << "parsed dimension ids:" << std::endl;
  for( auto const & l_e : l_ids ) std::cout << "  " << l_e.first << ": " << l_e.second << std::endl;

  std::vector< int64_t > l_size_vec;
  EinsumExpressionAscii::parse_dim_sizes( i_argv[2], l_size_vec );
  if( l_size_vec.size() != l_ids.size() ) {
    std::cerr << "error: " << l_ids.size() << " dimension sizes expected, got " << l_size_vec.size() << std::endl;
    return EXIT_FAILURE;
  }
  SizeMap l_sizes;
  std::map< int64_t, std::string > l_names;
  std::cout << "parsed dimension sizes:" << std::endl;
  for( auto const & l_e : l_ids ) {
    l_sizes[l_e.second] = l_size_vec[l_e.second];
    l_names[l_e.second] = l_e.first;
    std::cout << "  " << l_e.first << ": " << l_size_vec[l_e.second] << std::endl;
  }

  std::string const l_dtype_arg = ( i_argc > 3 ) ? i_argv[3] : "FP32";
  Elem l_in, l_out_elem;
  einsum_ir::data_t l_dt_in, l_dt_comp;
  if( l_dtype_arg == "FP32" )      { l_in = Elem::F32;  l_out_elem = Elem::F32; l_dt_in = einsum_ir::FP32; l_dt_comp = einsum_ir::FP32; }
  else if( l_dtype_arg == "FP64" ) { l_in = Elem::F64;  l_out_elem = Elem::F64; l_dt_in = einsum_ir::FP64; l_dt_comp = einsum_ir::FP64; }
  else if( l_dtype_arg == "BF16" ) { l_in = Elem::BF16; l_out_elem = Elem::F32; l_dt_in = einsum_ir::BF16; l_dt_comp = einsum_ir::FP32; }
  else {
    std::cerr << "failed to determine dtype" << std::endl;
    return EXIT_FAILURE;
  }
  std::cout << "dtype: " << l_dtype_arg << std::endl;

  std::vector< int64_t > l_loop_order;
  std::vector< int64_t > * l_loop_order_ptr = nullptr;
  if( i_argc > 4 ) {
    EinsumExpressionAscii::parse_loop_order( i_argv[4], l_ids, l_loop_order );
    std::cout << "loop order: " << i_argv[4] << std::endl;
    l_loop_order_ptr = &l_loop_order;
  }

  // dim ids of the three tensors
  std::vector< int64_t > l_dims[3];
  for( int l_te = 0; l_te < 3; l_te++ ) {
    std::vector< std::string > l_nm;
    EinsumExpressionAscii::split_string( l_tensors[l_te], ",", l_nm );
    for( auto const & l_n : l_nm ) l_dims[l_te].push_back( l_ids.at( l_n ) );
  }
  auto numel = [&]( std::vector< int64_t > const & i_d ) {
    int64_t l_n = 1;
    for( int64_t l_id : i_d ) l_n *= l_sizes.at( l_id );
    return l_n;
  };
  int64_t l_flops = 2;
  for( auto const & l_e : l_sizes ) l_flops *= l_e.second;

  Rng l_rng( 1 );
  HostData l_left  = make_data( l_in, numel( l_dims[0] ), Fill::UNIFORM, l_rng );
  HostData l_right = make_data( l_in, numel( l_dims[1] ), Fill::ONES, l_rng );
  HostData l_out   = make_data( l_out_elem, numel( l_dims[2] ), Fill::UNIFORM, l_rng );
  DeviceBuffer l_d_left( l_left.bytes() ), l_d_right( l_right.bytes() ), l_d_out( l_out.bytes() );
  l_d_left.upload( l_left );
  l_d_right.upload( l_right );
  l_d_out.upload( l_out );

  void * l_stream = nullptr;
  check_hip( etir_hip_stream_create( &l_stream ), "etir_hip_stream_create" );

  std::cout << "einsum_ir:" << std::endl;
  einsum_ir::backend::MemoryManager l_memory;
  einsum_ir::backend::BinaryContractionHip l_bin;
  std::vector< int64_t > l_no_permute;
  auto l_t0 = std::chrono::steady_clock::now();
  l_bin.init( (int64_t) l_dims[0].size(), (int64_t) l_dims[1].size(), (int64_t) l_dims[2].size(),
              &l_sizes, &l_sizes, &l_sizes, nullptr, &l_sizes,
              l_loop_order_ptr,
              l_dims[0].data(), l_dims[1].data(), l_dims[2].data(),
              l_no_permute.data(), l_no_permute.data(),
              &l_memory,
              l_dt_in, l_dt_in, l_dt_comp, l_dt_comp,
              einsum_ir::ZERO, einsum_ir::MADD, einsum_ir::UNDEFINED_KTYPE,
              1 );
  l_bin.set_stream( l_stream );
  einsum_ir::err_t l_err = l_bin.compile();
  if( l_err == einsum_ir::SUCCESS ) l_err = l_memory.alloc_all_memory();
  double const l_time_compile = seconds_since( l_t0 );
  if( l_err != einsum_ir::SUCCESS ) {
    std::cerr << "error: compile failed (" << (int) l_err << "): " << etir_hip_last_error() << std::endl;
    return EXIT_FAILURE;
  }

  double const l_time = time_per_call(
      [&]() {
        if( l_bin.contract_async( l_d_left.ptr(), l_d_right.ptr(), nullptr, l_d_out.ptr() ) != einsum_ir::SUCCESS ) {
          throw std::runtime_error( std::string( "contract_async failed: " ) + etir_hip_last_error() );
        }
      },
      [&]() { check_hip( etir_hip_synchronize( l_stream ), "etir_hip_synchronize" ); } );
  double const l_gflops = 1.0e-9 * double( l_flops ) / l_time;
  std::cout << "  time (compile): " << l_time_compile << std::endl;
  std::cout << "  time (contract): " << l_time << std::endl;
  std::cout << "  gflops: " << l_gflops << std::endl;
  char l_desc[512] = { 0 };
  if( etir_hip_plan_describe( l_bin.plan(), l_desc, sizeof( l_desc ) ) == 0 ) {
    std::cout << "  plan: " << l_desc << std::endl;
  }

  // float64 host check
  std::vector< std::vector< int64_t > > const l_in_dims = { l_dims[0], l_dims[1] };
  std::vector< Step > const l_steps = { { 0, 1, l_dims[2] } };
  Keep const l_keep = choose_keep( l_in_dims, l_steps, l_dims[2], l_sizes );
  std::vector< HostTensor > l_host = { restrict_tensor( l_dims[0], l_left.val, l_sizes, l_keep ),
                                       restrict_tensor( l_dims[1], l_right.val, l_sizes, l_keep ) };
  HostTensor const l_ref = run_steps( l_host, l_steps, l_sizes, l_keep );
  l_d_out.download( l_out );
  Comparison const l_cmp = compare( l_ref.v, restricted_output( l_out, l_dims[2], l_sizes, l_keep ) );
  bool const l_ok = report( l_cmp, tolerance( l_in ), describe_keep( l_keep, l_sizes, l_names ) );

  std::cout << "CSV_DATA: einsum_ir,\"" << l_arg << "\",\"" << i_argv[2] << "\"," << l_dtype_arg << ","
            << l_flops << "," << l_time_compile << "," << l_time << "," << l_gflops << std::endl;
  etir_hip_stream_destroy( l_stream );
  std::cout << "finished running bench_binary!" << std::endl;
  return l_ok ? EXIT_SUCCESS : EXIT_FAILURE;
}

} // namespace

int main( int i_argc, char * i_argv[] ) {
  std::cout << "running bench_binary!" << std::endl;
  if( i_argc < 3 ) return usage();
  try {
    return run( i_argc, i_argv );
  }
  catch( std::exception const & l_e ) {
    std::cerr << "error: " << l_e.what() << std::endl;
    return EXIT_FAILURE;
  }
}
