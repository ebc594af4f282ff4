// CPU tests of the harnesses' float64 host evaluation (einsum_ir_amd/csrc/
// bench/bench_util.h): pairwise contraction against closed forms, output
// order, complex values, sums over dims of one operand, restriction to an
// index grid, path steps, the error measure and bf16 rounding.  No GPU call.
#include <cstdio>
#include <functional>
#include <vector>
#include "../../einsum_ir_amd/csrc/bench/bench_util.h"

using namespace etir_bench;

static int g_failures = 0, g_checks = 0;
#define CHECK( cond )                                                        \
  do {                                                                       \
    g_checks++;                                                              \
    if( !( cond ) ) {                                                        \
      g_failures++;                                                          \
      std::printf( "  FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond );      \
    }                                                                        \
  } while( 0 )

static HostTensor tensor( std::vector< int64_t > i_dims, SizeMap const & i_sizes,
                          std::function< cplx( std::vector< int64_t > const & ) > i_f ) {
  HostTensor l_t;
  l_t.dims = i_dims;
  int64_t l_n = 1;
  for( int64_t l_d : i_dims ) l_n *= i_sizes.at( l_d );
  std::vector< int64_t > l_idx( i_dims.size(), 0 );
  for( int64_t l_e = 0; l_e < l_n; l_e++ ) {
    l_t.v.push_back( i_f( l_idx ) );
    for( std::size_t l_d = i_dims.size(); l_d-- > 0; ) {
      if( ++l_idx[l_d] < i_sizes.at( i_dims[l_d] ) ) break;
      l_idx[l_d] = 0;
    }
  }
  return l_t;
}

static bool near( cplx a, cplx b ) { return std::abs( a - b ) <= 1e-9 * ( 1 + std::abs( b ) ); }

int main() {
  enum { M = 0, N = 1, K = 2, L = 3 };
  SizeMap const l_sizes = { { M, 5 }, { N, 3 }, { K, 7 }, { L, 4 } };
  Keep const l_all;
  // A[m][k] = m + 1, B[k][n] = k + n: out[m][n] = (m+1) (K(K-1)/2 + K n)
  HostTensor const l_a = tensor( { M, K }, l_sizes, []( auto const & i ) { return cplx( i[0] + 1, 0 ); } );
  HostTensor const l_b = tensor( { K, N }, l_sizes, []( auto const & i ) { return cplx( i[0] + i[1], 0 ); } );
  HostTensor const l_c = host_contract( l_a, l_b, { M, N }, l_sizes, l_all );
  CHECK( l_c.v.size() == 15 );
  for( int m = 0; m < 5; m++ ) {
    for( int n = 0; n < 3; n++ ) CHECK( near( l_c.v[m * 3 + n], double( ( m + 1 ) * ( 21 + 7 * n ) ) ) );
  }
  // the same contraction written with the output transposed
  HostTensor const l_ct = host_contract( l_a, l_b, { N, M }, l_sizes, l_all );
  for( int m = 0; m < 5; m++ ) {
    for( int n = 0; n < 3; n++ ) CHECK( near( l_ct.v[n * 5 + m], l_c.v[m * 3 + n] ) );
  }
  // a dim of only one operand that the output lacks is summed: sum_l D[m][l]
  HostTensor const l_d = tensor( { M, L }, l_sizes, []( auto const & i ) { return cplx( 10 * i[0] + i[1], 0 ); } );
  HostTensor const l_sum = host_contract( l_d, scalar_one(), { M }, l_sizes, l_all );
  for( int m = 0; m < 5; m++ ) CHECK( near( l_sum.v[m], 40.0 * m + 6 ) );
  // unary step: a permutation
  HostTensor const l_p = host_contract( l_d, scalar_one(), { L, M }, l_sizes, l_all );
  for( int m = 0; m < 5; m++ ) {
    for( int l = 0; l < 4; l++ ) CHECK( near( l_p.v[l * 5 + m], l_d.v[m * 4 + l] ) );
  }
  // complex: (i) * (2 - i) summed over k = K (1 + 2i)
  HostTensor const l_zi = tensor( { M, K }, l_sizes, []( auto const & ) { return cplx( 0, 1 ); } );
  HostTensor const l_zb = tensor( { K, N }, l_sizes, []( auto const & ) { return cplx( 2, -1 ); } );
  HostTensor const l_z = host_contract( l_zi, l_zb, { M, N }, l_sizes, l_all );
  for( cplx l_v : l_z.v ) CHECK( near( l_v, cplx( 7, 14 ) ) );

  // restriction: kept rows of the full result equal the restricted evaluation
  Keep const l_keep = { { M, { 0, 2, 4 } }, { N, { 2 } } };
  HostTensor const l_ar = restrict_tensor( { M, K }, l_a.v, l_sizes, l_keep );
  HostTensor const l_br = restrict_tensor( { K, N }, l_b.v, l_sizes, l_keep );
  CHECK( l_ar.v.size() == 21 && l_br.v.size() == 7 );
  HostTensor const l_cr = host_contract( l_ar, l_br, { M, N }, l_sizes, l_keep );
  std::vector< cplx > const l_full_r = restrict_tensor( { M, N }, l_c.v, l_sizes, l_keep ).v;
  CHECK( l_cr.v.size() == 3 && l_full_r.size() == 3 );
  for( int l_i = 0; l_i < 3; l_i++ ) CHECK( near( l_cr.v[l_i], l_full_r[l_i] ) );
  CHECK( near( l_cr.v[1], 3.0 * ( 21 + 14 ) ) );

  // path steps of ab,bc,cd->ad along (0,1),(0,1) and (1,2),(0,1)
  enum { A = 10, B = 11, C = 12, D = 13 };
  std::vector< std::vector< int64_t > > const l_in = { { A, B }, { B, C }, { C, D } };
  std::vector< Step > const l_s1 = path_steps( l_in, { A, D }, { 0, 1, 0, 1 } );
  CHECK( l_s1.size() == 2 && l_s1[0].a == 0 && l_s1[0].b == 1 && l_s1[0].out == std::vector< int64_t >( { A, C } ) );
  CHECK( l_s1[1].a == 2 && l_s1[1].b == 3 && l_s1[1].out == std::vector< int64_t >( { A, D } ) );
  std::vector< Step > const l_s2 = path_steps( l_in, { A, D }, { 1, 2, 0, 1 } );
  CHECK( l_s2[0].a == 1 && l_s2[0].b == 2 && l_s2[0].out == std::vector< int64_t >( { B, D } ) );
  CHECK( l_s2[1].a == 0 && l_s2[1].b == 3 );
  bool l_threw = false;
  try { path_steps( l_in, { A, D }, { 0, 0, 0, 1 } ); } catch( std::exception const & ) { l_threw = true; }
  CHECK( l_threw );
  l_threw = false;
  try { path_steps( l_in, { A, D }, { 0, 1 } ); } catch( std::exception const & ) { l_threw = true; }
  CHECK( l_threw );

  // the chain evaluated along either path agrees; a small budget restricts
  // the output dims and keeps their first and last index
  SizeMap const l_cs = { { A, 6 }, { B, 5 }, { C, 4 }, { D, 9 } };
  Rng l_rng( 3 );
  std::vector< HostTensor > l_ts;
  for( auto const & l_dims : l_in ) {
    l_ts.push_back( tensor( l_dims, l_cs, [&]( auto const & ) { return cplx( l_rng.normal(), 0 ); } ) );
  }
  HostTensor const l_r1 = run_steps( l_ts, l_s1, l_cs, l_all );
  HostTensor const l_r2 = run_steps( l_ts, l_s2, l_cs, l_all );
  for( std::size_t l_i = 0; l_i < l_r1.v.size(); l_i++ ) CHECK( near( l_r1.v[l_i], l_r2.v[l_i] ) );
  Keep const l_small = choose_keep( l_in, l_s1, { A, D }, l_cs, 100.0 );
  CHECK( l_small.count( D ) == 1 && l_small.at( D ).front() == 0 && l_small.at( D ).back() == 8 );
  CHECK( steps_cost( l_in, l_s1, l_cs, l_small ) < steps_cost( l_in, l_s1, l_cs, l_all ) );
  std::vector< HostTensor > l_tr;
  for( std::size_t l_t = 0; l_t < l_in.size(); l_t++ ) l_tr.push_back( restrict_tensor( l_in[l_t], l_ts[l_t].v, l_cs, l_small ) );
  HostTensor const l_r3 = run_steps( l_tr, l_s1, l_cs, l_small );
  std::vector< cplx > const l_r1r = restrict_tensor( { A, D }, l_r1.v, l_cs, l_small ).v;
  CHECK( l_r3.v.size() == l_r1r.size() );
  for( std::size_t l_i = 0; l_i < l_r3.v.size(); l_i++ ) CHECK( near( l_r3.v[l_i], l_r1r[l_i] ) );

  // relative Frobenius error: |(3,4) - (3,4.5)| / |(3,4)| = 0.5 / 5
  Comparison const l_cmp = compare( { 3.0, 4.0 }, { 3.0, 4.5 } );
  CHECK( std::abs( l_cmp.rel - 0.1 ) < 1e-15 && l_cmp.max_diff == 0.5 && l_cmp.entries == 2 );
  CHECK( std::isinf( compare( { 1.0 }, { cplx( NAN, 0 ) } ).rel ) );

  // bf16: exact values pass, ties round to even, NaN stays NaN
  CHECK( to_bf16( 1.0f ) == 0x3F80 && from_bf16( 0x3F80 ) == 1.0f );
  CHECK( to_bf16( 1.0f + 0x1.0p-8f ) == 0x3F80 );               // tie, even below
  CHECK( to_bf16( 1.0f + 3 * 0x1.0p-8f ) == 0x3F82 );           // tie, even above
  CHECK( to_bf16( 1.0f + 0x1.0p-8f + 0x1.0p-20f ) == 0x3F81 );  // above the tie
  CHECK( std::isnan( from_bf16( to_bf16( NAN ) ) ) );

  std::printf( "%d checks, %d failures\n", g_checks, g_failures );
  return g_failures == 0 ? 0 : 1;
}
