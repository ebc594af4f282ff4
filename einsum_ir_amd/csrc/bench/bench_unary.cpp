// bench_unary: one permutation through UnaryHip.
//
//   bench_unary einsum_string dimension_sizes [dtype]
//
// Arguments and report follow reference src/bench_unary.cpp:55-336: a
// single-character expression "abcd->dbac" (the standard format is accepted
// too), sizes in ascending order of the dimension ids, dtype FP32 or FP64
// (BF16 is additive).  Data: N(0,1).  The tensors live on the GPU; the time
// is per call of eval_async over a run of calls (one warm-up).  The output
// is compared with the host's permutation of the same input, bit for bit;
// the exit status is 1 when any entry differs.
#include <cstdlib>

#include "bench_util.h"
#include "backend/UnaryHip.h"
#include "frontend/EinsumExpressionAscii.h"

using namespace etir_bench;
using einsum_ir::frontend::EinsumExpressionAscii;

namespace {

int usage() {
  std::cerr << "usage: bench_unary einsum_string dimension_sizes [dtype]\n"
               "  dimension sizes in ascending order of the dimension ids\n"
               "  dtype FP32 (default), FP64 or BF16\n"
               "example: ./bench_unary \"abcd->dbac\" \"32,32,32,32\" FP64" << std::endl;
  return EXIT_FAILURE;
}

int run( int i_argc, char * i_argv[] ) {
  std::string l_arg( i_argv[1] );
  l_arg.erase( std::remove( l_arg.begin(), l_arg.end(), ' ' ), l_arg.end() );
  std::string l_std;
  if( !l_arg.empty() && l_arg[0] == '[' ) l_std = l_arg;
  else EinsumExpressionAscii::schar_to_standard( l_arg, l_std );
  std::vector< std::string > l_tensors;
  EinsumExpressionAscii::parse_tensors( l_std, l_tensors );
  if( l_tensors.size() != 2 ) {
    std::cerr << "error: expected one input and one output tensor" << std::endl;
    return EXIT_FAILURE;
  }
  std::cout << "parsed tensors:" << std::endl;
  for( auto const & l_t : l_tensors ) std::cout << "  " << l_t << std::endl;

  std::map< std::string, int64_t > l_ids;
  EinsumExpressionAscii::parse_dim_ids( l_std, l_ids );
  std::vector< int64_t > l_size_vec;
  EinsumExpressionAscii::parse_dim_sizes( i_argv[2], l_size_vec );
  if( l_size_vec.size() != l_ids.size() ) {
    std::cerr << "error: " << l_ids.size() << " dimension sizes expected, got " << l_size_vec.size() << std::endl;
    return EXIT_FAILURE;
  }
  SizeMap l_sizes;
  std::cout << "parsed dimension sizes:" << std::endl;
  for( auto const & l_e : l_ids ) {
    l_sizes[l_e.second] = l_size_vec[l_e.second];
    std::cout << "  " << l_e.first << ": " << l_size_vec[l_e.second] << std::endl;
  }

  std::string const l_dtype_arg = ( i_argc > 3 ) ? i_argv[3] : "FP32";
  Elem l_elem;
  einsum_ir::data_t l_dt;
  if( l_dtype_arg == "FP32" )      { l_elem = Elem::F32;  l_dt = einsum_ir::FP32; }
  else if( l_dtype_arg == "FP64" ) { l_elem = Elem::F64;  l_dt = einsum_ir::FP64; }
  else if( l_dtype_arg == "BF16" ) { l_elem = Elem::BF16; l_dt = einsum_ir::BF16; }
  else {
    std::cerr << "error: unsupported dtype" << std::endl;
    return EXIT_FAILURE;
  }
  std::cout << "dtype: " << l_dtype_arg << std::endl;

  std::vector< int64_t > l_dims[2];
  for( int l_te = 0; l_te < 2; l_te++ ) {
    std::vector< std::string > l_nm;
    EinsumExpressionAscii::split_string( l_tensors[l_te], ",", l_nm );
    for( auto const & l_n : l_nm ) l_dims[l_te].push_back( l_ids.at( l_n ) );
  }
  if( l_dims[0].size() != l_dims[1].size() ) {
    std::cerr << "error: number of tensor dimensions does not match" << std::endl;
    return EXIT_FAILURE;
  }
  int64_t const l_num_dims = (int64_t) l_dims[0].size();
  std::cout << "assembled einsum_ir data structures" << std::endl;
  for( int l_te = 0; l_te < 2; l_te++ ) {
    std::cout << ( l_te == 0 ? "  string_dim_ids (input):  " : "  string_dim_ids (output): " );
    for( int64_t l_id : l_dims[l_te] ) std::cout << l_id << " ";
    std::cout << std::endl;
  }

  int64_t l_n = 1;
  for( int64_t l_id : l_dims[0] ) l_n *= l_sizes.at( l_id );
  int64_t const l_bytes = 2 * l_n * elem_bytes( l_elem );
  std::cout << "total amount of transferred data (read + write):" << std::endl;
  std::cout << "  B:   " << l_bytes << std::endl;
  std::cout << "  MiB: " << double( l_bytes ) / ( 1024.0 * 1024.0 ) << std::endl;
  std::cout << "  GiB: " << double( l_bytes ) / ( 1024.0 * 1024.0 * 1024.0 ) << std::endl;

  Rng l_rng( 7 );
  HostData l_x = make_data( l_elem, l_n, Fill::NORMAL, l_rng );
  HostData l_y( l_elem, l_n );
  DeviceBuffer l_d_x( l_x.bytes() ), l_d_y( l_y.bytes() );
  l_d_x.upload( l_x );
  check_hip( etir_hip_memset( l_d_y.ptr(), 0, l_y.bytes() ), "etir_hip_memset" );

  void * l_stream = nullptr;
  check_hip( etir_hip_stream_create( &l_stream ), "etir_hip_stream_create" );
  einsum_ir::backend::UnaryHip l_unary;
  auto l_t0 = std::chrono::steady_clock::now();
  l_unary.init( l_num_dims, &l_sizes, l_dims[0].data(), l_dims[1].data(), l_dt, l_dt, l_dt,
                einsum_ir::COPY, 1 );
  l_unary.set_stream( l_stream );
  einsum_ir::err_t const l_err = l_unary.compile();
  double const l_time_compile = seconds_since( l_t0 );
  if( l_err != einsum_ir::SUCCESS ) {
    std::cerr << "error: compile failed (" << (int) l_err << "): " << etir_hip_last_error() << std::endl;
    return EXIT_FAILURE;
  }
  double const l_time = time_per_call(
      [&]() {
        if( l_unary.eval_async( l_d_x.ptr(), l_d_y.ptr() ) != einsum_ir::SUCCESS ) {
          throw std::runtime_error( std::string( "eval_async failed: " ) + etir_hip_last_error() );
        }
      },
      [&]() { check_hip( etir_hip_synchronize( l_stream ), "etir_hip_synchronize" ); } );
  double const l_gib = double( l_bytes ) / ( 1024.0 * 1024.0 * 1024.0 );
  std::cout << "einsum_ir:" << std::endl;
  std::cout << "  time (compile): " << l_time_compile << std::endl;
  std::cout << "  time (eval):    " << l_time << std::endl;
  std::cout << "  gibs (eval):    " << l_gib / l_time << std::endl;
  std::cout << "  gibs (total):   " << l_gib / ( l_time + l_time_compile ) << std::endl;
  char l_desc[512] = { 0 };
  if( etir_hip_plan_describe( l_unary.plan(), l_desc, sizeof( l_desc ) ) == 0 ) {
    std::cout << "  plan: " << l_desc << std::endl;
  }

  // host permutation of the input's bytes, compared bit for bit
  l_d_y.download( l_y );
  int64_t const l_esz = elem_bytes( l_elem );
  std::map< int64_t, int64_t > l_stride_in;
  for( int64_t l_d = l_num_dims - 1, l_s = 1; l_d >= 0; l_d-- ) {
    l_stride_in[l_dims[0][l_d]] = l_s;
    l_s *= l_sizes.at( l_dims[0][l_d] );
  }
  std::vector< int64_t > l_idx( l_num_dims, 0 );
  int64_t l_bad = 0;
  for( int64_t l_o = 0; l_o < l_n; l_o++ ) {
    int64_t l_src = 0;
    for( int64_t l_d = 0; l_d < l_num_dims; l_d++ ) l_src += l_idx[l_d] * l_stride_in[l_dims[1][l_d]];
    if( std::memcmp( l_y.raw.data() + l_o * l_esz, l_x.raw.data() + l_src * l_esz, l_esz ) != 0 ) l_bad++;
    for( int64_t l_d = l_num_dims - 1; l_d >= 0; l_d-- ) {
      if( ++l_idx[l_d] < l_sizes.at( l_dims[1][l_d] ) ) break;
      l_idx[l_d] = 0;
    }
  }
  std::cout << "\n*** comparing solution ***:" << std::endl;
  if( l_bad == 0 ) std::cout << "  results are equal (bit-exact, " << l_n << " entries)" << std::endl;
  else std::cerr << "error: " << l_bad << " of " << l_n << " entries differ from the host permutation" << std::endl;

  std::cout << "CSV_DATA: einsum_ir,\"" << i_argv[1] << "\",\"" << i_argv[2] << "\"," << l_dtype_arg << ","
            << l_bytes << "," << l_time_compile << "," << l_time << "," << l_gib / l_time << std::endl;
  etir_hip_stream_destroy( l_stream );
  return l_bad == 0 ? EXIT_SUCCESS : EXIT_FAILURE;
}

} // namespace

int main( int i_argc, char * i_argv[] ) {
  if( i_argc < 3 ) return usage();
  try {
    return run( i_argc, i_argv );
  }
  catch( std::exception const & l_e ) {
    std::cerr << "error: " << l_e.what() << std::endl;
    return EXIT_FAILURE;
  }
}
