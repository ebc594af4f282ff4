// bench_expression: an einsum expression evaluated along a contraction path
// by EinsumExpression.
//
//   bench_expression einsum_string dimension_sizes contraction_path
//                    [dtype [store_lock [print_tree]]]
//
// Arguments and report follow reference src/bench_expression.cpp:8-545: the
// expression in single-character or standard format (numeric names sort by
// value), sizes in ascending order of the dimension names, the path in
// opt_einsum's standard form "(1,2),(2,3),(0,1)", dtype FP32, FP64, CPX_FP32
// or CPX_FP64 (complex numbers interleaved: a trailing dim of size 2),
// store_lock 1 to store and lock every input before the evaluation, and
// print_tree 1-4 to print the compiled tree (1: exchange format with dim
// ids, 2: with dim names, 3: drawn with ids, 4: drawn with names).  Data:
// N(0,1).  The tensors live on the GPU; the time is per eval() over a run of
// calls (one warm-up).  The result is checked against a float64 host
// evaluation along the same path (relative Frobenius error: fp32 1e-5, fp64
// 1e-12); the exit status is 1 when it is not met.
#include <cctype>
#include <cstdlib>

#include "bench_util.h"
#include "frontend/EinsumExpression.h"
#include "frontend/EinsumExpressionAscii.h"

using namespace etir_bench;
using einsum_ir::frontend::EinsumExpressionAscii;

namespace {

int usage() {
  std::cerr << "usage: bench_expression einsum_string dimension_sizes contraction_path [dtype [store_lock [print_tree]]]\n"
               "  einsum_string     e.g. \"iae,bf,dcba,cg,dh->hgfei\" or \"[i,a,e],[b,f],[d,c,b,a],[c,g],[d,h]->[h,g,f,e,i]\"\n"
               "  dimension_sizes   sizes in ascending order of the dimension names (numeric names by value)\n"
               "  contraction_path  opt_einsum standard form, e.g. \"(1,2),(2,3),(0,1),(0,1)\"\n"
               "  dtype             FP32 (default), FP64, CPX_FP32 or CPX_FP64\n"
               "  store_lock        1: store and lock all inputs before the evaluation (default 0)\n"
               "  print_tree        1/2: exchange format with ids/names, 3/4: drawing with ids/names (default 0)"
            << std::endl;
  return EXIT_FAILURE;
}

//! replaces every dim id in a tree string by its name (ids without a name stay)
std::string name_ids( std::string const & i_tree, std::map< int64_t, std::string > const & i_names ) {
  std::string l_out;
  for( std::size_t l_i = 0; l_i < i_tree.size(); ) {
    if( std::isdigit( (unsigned char) i_tree[l_i] ) ) {
      std::size_t l_j = l_i;
      while( l_j < i_tree.size() && std::isdigit( (unsigned char) i_tree[l_j] ) ) l_j++;
      int64_t const l_id = std::stoll( i_tree.substr( l_i, l_j - l_i ) );
      auto const l_n = i_names.find( l_id );
      l_out += ( l_n != i_names.end() ) ? l_n->second : i_tree.substr( l_i, l_j - l_i );
      l_i = l_j;
    }
    else {
      l_out += i_tree[l_i++];
    }
  }
  return l_out;
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
  int64_t const l_num_tensors = (int64_t) l_tensors.size();
  std::cout << "parsed tensors:" << std::endl;
  for( auto const & l_t : l_tensors ) std::cout << "  " << l_t << std::endl;
  if( l_num_tensors < 3 ) {
    std::cerr << "error: the expression needs at least two input tensors" << std::endl;
    return EXIT_FAILURE;
  }

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

  std::vector< int64_t > l_path;
  EinsumExpressionAscii::parse_path( i_argv[3], l_path );
  std::cout << "parsed contraction path:";
  for( std::size_t l_i = 0; l_i < l_path.size(); l_i += 2 ) std::cout << " (" << l_path[l_i] << "," << l_path[l_i + 1] << ")";
  std::cout << std::endl;
  if( (int64_t) l_path.size() != 2 * ( l_num_tensors - 2 ) ) {
    std::cerr << "error: the path has " << l_path.size() / 2 << " contractions, the expression needs "
              << l_num_tensors - 2 << std::endl;
    return EXIT_FAILURE;
  }

  std::string const l_dtype_arg = ( i_argc > 4 ) ? i_argv[4] : "FP32";
  Elem l_elem;
  einsum_ir::data_t l_dt;
  einsum_ir::complex_t l_ct = einsum_ir::REAL_ONLY;
  if( l_dtype_arg == "FP32" )          { l_elem = Elem::F32;  l_dt = einsum_ir::FP32; }
  else if( l_dtype_arg == "FP64" )     { l_elem = Elem::F64;  l_dt = einsum_ir::FP64; }
  else if( l_dtype_arg == "CPX_FP32" ) { l_elem = Elem::C64;  l_dt = einsum_ir::FP32; l_ct = einsum_ir::BATCH_INNER; }
  else if( l_dtype_arg == "CPX_FP64" ) { l_elem = Elem::C128; l_dt = einsum_ir::FP64; l_ct = einsum_ir::BATCH_INNER; }
  else {
    std::cerr << "failed to determine dtype" << std::endl;
    return EXIT_FAILURE;
  }
  std::cout << "dtype: " << l_dtype_arg << std::endl;
  bool const l_store_lock = ( i_argc > 5 ) && std::stoi( i_argv[5] ) == 1;
  std::cout << "store and lock: " << l_store_lock << std::endl;
  int const l_print_tree = ( i_argc > 6 ) ? std::stoi( i_argv[6] ) : 0;
  if( l_print_tree < 0 || l_print_tree > 4 ) {
    std::cerr << "error: invalid print_tree argument" << std::endl;
    return EXIT_FAILURE;
  }
  std::cout << "print_tree: " << l_print_tree << std::endl;

  // dim ids per tensor (real dims); complex data adds a trailing dim of size 2
  std::vector< std::vector< int64_t > > l_dims( l_num_tensors );
  for( int64_t l_te = 0; l_te < l_num_tensors; l_te++ ) {
    std::vector< std::string > l_nm;
    EinsumExpressionAscii::split_string( l_tensors[l_te], ",", l_nm );
    for( auto const & l_n : l_nm ) l_dims[l_te].push_back( l_ids.at( l_n ) );
  }
  int64_t const l_cpx_id = (int64_t) l_size_vec.size();
  std::vector< int64_t > l_all_sizes = l_size_vec;
  std::vector< int64_t > l_string_num_dims, l_string_dim_ids;
  if( l_ct != einsum_ir::REAL_ONLY ) l_all_sizes.push_back( 2 );
  for( auto const & l_d : l_dims ) {
    l_string_dim_ids.insert( l_string_dim_ids.end(), l_d.begin(), l_d.end() );
    if( l_ct != einsum_ir::REAL_ONLY ) l_string_dim_ids.push_back( l_cpx_id );
    l_string_num_dims.push_back( (int64_t) l_d.size() + ( l_ct != einsum_ir::REAL_ONLY ? 1 : 0 ) );
  }
  std::cout << "assembled einsum_ir data structures" << std::endl;
  std::cout << "  string_num_dims: ";
  for( int64_t l_v : l_string_num_dims ) std::cout << l_v << " ";
  std::cout << std::endl << "  string_dim_ids: ";
  for( int64_t l_v : l_string_dim_ids ) std::cout << l_v << " ";
  std::cout << std::endl;

  Rng l_rng( 11 );
  std::vector< HostData > l_data;
  std::vector< DeviceBuffer > l_dev;
  std::vector< void * > l_ptrs;
  for( auto const & l_d : l_dims ) {
    int64_t l_n = 1;
    for( int64_t l_id : l_d ) l_n *= l_sizes.at( l_id );
    l_data.push_back( make_data( l_elem, l_n, Fill::NORMAL, l_rng ) );
    l_dev.emplace_back( l_data.back().bytes() );
    l_dev.back().upload( l_data.back() );
    l_ptrs.push_back( l_dev.back().ptr() );
  }

  std::cout << "\n*** benchmarking einsum_ir ***" << std::endl;
  void * l_stream = nullptr;
  check_hip( etir_hip_stream_create( &l_stream ), "etir_hip_stream_create" );
  einsum_ir::frontend::EinsumExpression l_exp;
  l_exp.init( (int64_t) l_all_sizes.size(), l_all_sizes.data(), l_num_tensors - 2,
              l_string_num_dims.data(), l_string_dim_ids.data(), l_path.data(),
              l_ct, l_dt, l_ptrs.data() );
  l_exp.set_stream( l_stream );
  auto l_t0 = std::chrono::steady_clock::now();
  einsum_ir::err_t l_err = l_exp.compile();
  double const l_time_compile = seconds_since( l_t0 );
  if( l_err != einsum_ir::SUCCESS ) {
    std::cerr << "error: failed to compile einsum_ir expression (" << (int) l_err << "): "
              << etir_hip_last_error() << std::endl;
    return EXIT_FAILURE;
  }
  if( l_print_tree > 0 ) {
    std::string l_tree = ( l_print_tree <= 2 ) ? l_exp.to_string_exchange_format() : l_exp.to_string_render();
    if( l_print_tree == 2 || l_print_tree == 4 ) l_tree = name_ids( l_tree, l_names );
    std::cout << l_tree << std::endl;
  }
  if( l_store_lock ) {
    for( int64_t l_te = 0; l_te < l_num_tensors - 1; l_te++ ) {
      if( l_exp.store_and_lock_data( l_te ) != einsum_ir::SUCCESS ) {
        std::cerr << "error: failed to store and lock tensor with id: " << l_te << std::endl;
        return EXIT_FAILURE;
      }
    }
  }
  double const l_time_eval = time_per_call( [&]() { l_exp.eval(); }, []() {} );
  int64_t const l_flops = l_exp.num_ops();
  double const l_gflops_eval = 1.0e-9 * double( l_flops ) / l_time_eval;
  double const l_gflops_total = 1.0e-9 * double( l_flops ) / ( l_time_eval + l_time_compile );
  std::cout << "  #flops:         " << l_flops << std::endl;
  std::cout << "  time (compile): " << l_time_compile << std::endl;
  std::cout << "  time (eval):    " << l_time_eval << std::endl;
  std::cout << "  gflops (eval):  " << l_gflops_eval << std::endl;
  std::cout << "  gflops (total): " << l_gflops_total << std::endl;
  std::cout << "CSV_DATA: einsum_ir,\"" << l_arg << "\",\"" << i_argv[2] << "\",\"" << i_argv[3] << "\","
            << l_flops << "," << l_time_compile << "," << l_time_eval << "," << l_gflops_eval << ","
            << l_gflops_total << std::endl;

  // float64 host evaluation along the same path
  int64_t const l_num_in = l_num_tensors - 1;
  std::vector< std::vector< int64_t > > const l_in_dims( l_dims.begin(), l_dims.begin() + l_num_in );
  std::vector< int64_t > const & l_out_dims = l_dims.back();
  std::vector< Step > const l_steps = path_steps( l_in_dims, l_out_dims, l_path );
  Keep const l_keep = choose_keep( l_in_dims, l_steps, l_out_dims, l_sizes );
  std::vector< HostTensor > l_host;
  for( int64_t l_te = 0; l_te < l_num_in; l_te++ ) {
    l_host.push_back( restrict_tensor( l_dims[l_te], l_data[l_te].val, l_sizes, l_keep ) );
  }
  HostTensor const l_ref = run_steps( l_host, l_steps, l_sizes, l_keep );
  l_dev.back().download( l_data.back() );
  Comparison const l_cmp = compare( l_ref.v, restricted_output( l_data.back(), l_out_dims, l_sizes, l_keep ) );
  bool const l_ok = report( l_cmp, tolerance( l_elem ), describe_keep( l_keep, l_sizes, l_names ) );
  etir_hip_stream_destroy( l_stream );
  return l_ok ? EXIT_SUCCESS : EXIT_FAILURE;
}

} // namespace

int main( int i_argc, char * i_argv[] ) {
  if( i_argc < 4 ) return usage();
  try {
    return run( i_argc, i_argv );
  }
  catch( std::exception const & l_e ) {
    std::cerr << "error: " << l_e.what() << std::endl;
    return EXIT_FAILURE;
  }
}
