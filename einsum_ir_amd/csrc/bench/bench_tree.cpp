// bench_tree: an einsum tree in the exchange format evaluated by EinsumTree.
//
//   bench_tree einsum_tree dimension_sizes [dtype]
//
// Arguments and report follow reference src/bench_tree.cpp:8-173: a tree such
// as "[[3,0]->[0,3]],[[3,2,4],[1,4,2]->[1,2,3]]->[0,1,2]", sizes in ascending
// order of the dimension ids, dtype FP32 or FP64.  Leaves and the root get
// tensors of N(0,1) data on the GPU; the time is per eval() over a run of
// calls (one warm-up).  The root is checked against a float64 host
// evaluation node by node (relative Frobenius error: fp32 1e-5, fp64 1e-12);
// the exit status is 1 when it is not met.
#include <cstdlib>

#include "bench_util.h"
#include "frontend/EinsumTree.h"
#include "frontend/EinsumTreeAscii.h"

using namespace etir_bench;
using einsum_ir::frontend::EinsumTreeAscii;

namespace {

int usage() {
  std::cerr << "usage: bench_tree einsum_tree dimension_sizes [dtype]\n"
               "  einsum_tree      e.g. \"[[3,0]->[0,3]],[[3,2,4],[1,4,2]->[1,2,3]]->[0,1,2]\"\n"
               "  dimension_sizes  sizes in ascending order of the dimension ids, e.g. \"2,3,4,5,6\"\n"
               "  dtype            FP32 (default) or FP64" << std::endl;
  return EXIT_FAILURE;
}

int run( int i_argc, char * i_argv[] ) {
  std::string const l_tree( i_argv[1] );
  int64_t const l_num_nodes = EinsumTreeAscii::count_nodes( l_tree );
  std::vector< std::vector< int64_t > > l_dim_ids( l_num_nodes ), l_children( l_num_nodes );
  int64_t l_parsed = 0;
  einsum_ir::err_t l_err = EinsumTreeAscii::parse_tree( l_tree, l_dim_ids, l_children, l_parsed );
  if( l_err != einsum_ir::SUCCESS || l_parsed != l_num_nodes ) {
    std::cerr << "error: failed to parse einsum tree" << std::endl;
    return EXIT_FAILURE;
  }
  SizeMap l_sizes;
  EinsumTreeAscii::parse_dim_size( i_argv[2], l_dim_ids, l_sizes );

  std::string const l_dtype_arg = ( i_argc > 3 ) ? i_argv[3] : "FP32";
  Elem l_elem;
  einsum_ir::data_t l_dt;
  if( l_dtype_arg == "FP32" )      { l_elem = Elem::F32; l_dt = einsum_ir::FP32; }
  else if( l_dtype_arg == "FP64" ) { l_elem = Elem::F64; l_dt = einsum_ir::FP64; }
  else {
    std::cerr << "failed to determine dtype" << std::endl;
    return EXIT_FAILURE;
  }

  // external tensors: leaves and the root
  Rng l_rng( 13 );
  std::vector< HostData > l_data( l_num_nodes );
  std::vector< DeviceBuffer > l_dev;
  std::vector< void * > l_ptrs( l_num_nodes, nullptr );
  std::vector< int64_t > l_dev_of( l_num_nodes, -1 );
  for( int64_t l_no = 0; l_no < l_num_nodes; l_no++ ) {
    if( !l_children[l_no].empty() && l_no != l_num_nodes - 1 ) continue;
    int64_t l_n = 1;
    for( int64_t l_id : l_dim_ids[l_no] ) {
      if( l_sizes.count( l_id ) == 0 ) {
        std::cerr << "error: no size for dimension " << l_id << std::endl;
        return EXIT_FAILURE;
      }
      l_n *= l_sizes.at( l_id );
    }
    l_data[l_no] = make_data( l_elem, l_n, Fill::NORMAL, l_rng );
    l_dev.emplace_back( l_data[l_no].bytes() );
    l_dev.back().upload( l_data[l_no] );
    l_dev_of[l_no] = (int64_t) l_dev.size() - 1;
  }
  for( int64_t l_no = 0; l_no < l_num_nodes; l_no++ ) {
    if( l_dev_of[l_no] >= 0 ) l_ptrs[l_no] = l_dev[l_dev_of[l_no]].ptr();
  }

  std::cout << "\n*** benchmarking einsum_ir ***" << std::endl;
  void * l_stream = nullptr;
  check_hip( etir_hip_stream_create( &l_stream ), "etir_hip_stream_create" );
  einsum_ir::frontend::EinsumTree l_et;
  l_et.init( &l_dim_ids, &l_children, &l_sizes, l_dt, l_ptrs.data() );
  l_et.set_stream( l_stream );
  auto l_t0 = std::chrono::steady_clock::now();
  l_err = l_et.compile();
  double const l_time_compile = seconds_since( l_t0 );
  if( l_err != einsum_ir::SUCCESS ) {
    std::cerr << "error: failed to compile einsum_ir tree (" << (int) l_err << "): "
              << etir_hip_last_error() << std::endl;
    return EXIT_FAILURE;
  }
  double const l_time_eval = time_per_call( [&]() { l_et.eval(); }, []() {} );
  int64_t const l_flops = l_et.num_ops();
  double const l_gflops_eval = 1.0e-9 * double( l_flops ) / l_time_eval;
  double const l_gflops_total = 1.0e-9 * double( l_flops ) / ( l_time_eval + l_time_compile );
  std::cout << "  #flops:         " << l_flops << std::endl;
  std::cout << "  time (compile): " << l_time_compile << std::endl;
  std::cout << "  time (eval):    " << l_time_eval << std::endl;
  std::cout << "  gflops (eval):  " << l_gflops_eval << std::endl;
  std::cout << "  gflops (total): " << l_gflops_total << std::endl;
  std::cout << "CSV_DATA: einsum_ir,\"" << l_tree << "\",\"" << i_argv[2] << "\"," << l_flops << ","
            << l_time_compile << "," << l_time_eval << "," << l_gflops_eval << "," << l_gflops_total << std::endl;

  // float64 host evaluation node by node (children come before parents)
  std::vector< std::vector< int64_t > > l_leaf_dims;
  std::vector< int64_t > l_slot( l_num_nodes, -1 );
  for( int64_t l_no = 0; l_no < l_num_nodes; l_no++ ) {
    if( l_children[l_no].empty() ) {
      l_slot[l_no] = (int64_t) l_leaf_dims.size();
      l_leaf_dims.push_back( l_dim_ids[l_no] );
    }
  }
  std::vector< Step > l_steps;
  for( int64_t l_no = 0; l_no < l_num_nodes; l_no++ ) {
    std::vector< int64_t > const & l_ch = l_children[l_no];
    if( l_ch.empty() ) continue;
    l_steps.push_back( { l_slot[l_ch[0]], l_ch.size() > 1 ? l_slot[l_ch[1]] : -1, l_dim_ids[l_no] } );
    l_slot[l_no] = (int64_t) ( l_leaf_dims.size() + l_steps.size() - 1 );
  }
  std::vector< int64_t > const & l_root_dims = l_dim_ids.back();
  Keep const l_keep = choose_keep( l_leaf_dims, l_steps, l_root_dims, l_sizes );
  std::vector< HostTensor > l_host;
  for( int64_t l_no = 0; l_no < l_num_nodes; l_no++ ) {
    if( l_children[l_no].empty() ) {
      l_host.push_back( restrict_tensor( l_dim_ids[l_no], l_data[l_no].val, l_sizes, l_keep ) );
    }
  }
  HostTensor const l_ref = l_steps.empty() ? l_host.back() : run_steps( l_host, l_steps, l_sizes, l_keep );
  HostData & l_root = l_data[l_num_nodes - 1];
  l_dev[l_dev_of[l_num_nodes - 1]].download( l_root );
  std::map< int64_t, std::string > l_names;
  Comparison const l_cmp = compare( l_ref.v, restricted_output( l_root, l_root_dims, l_sizes, l_keep ) );
  bool const l_ok = report( l_cmp, tolerance( l_elem ), describe_keep( l_keep, l_sizes, l_names ) );
  etir_hip_stream_destroy( l_stream );
  return l_ok ? EXIT_SUCCESS : EXIT_FAILURE;
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
