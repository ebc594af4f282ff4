// Known-answer tests of the host logic of libeinsum_ir.so (no GPU calls).
//
// The expected values restate the integer known answers of the reference's
// own unit tests:
//   dim typing            reference src/backend/BinaryContraction.test.cpp:4-126
//   unary strides         reference src/backend/Unary.test.cpp:4-36
//   histogram, substrings, unique path ids
//                         reference src/frontend/EinsumExpression.test.cpp:4-61
//   swap_inputs / blocking / reorder
//                         reference src/backend/BinaryPrimitives.test.cpp:4-62, 64-626, 627-1198
//   ASCII parsers         reference src/frontend/EinsumExpressionAscii.test.cpp:4-94
// plus tests of this library's own planning code (memory arena, tree parser).
#include <array>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>
#include "backend/BinaryContraction.h"
#include "backend/BinaryPrimitives.h"
#include "backend/MemoryManager.h"
#include "backend/Unary.h"
#include "frontend/EinsumExpression.h"
#include "frontend/EinsumExpressionAscii.h"
#include "frontend/EinsumTreeAscii.h"

using namespace einsum_ir;

static int g_failures = 0;
static int g_checks = 0;
#define CHECK( cond )                                                                 \
  do {                                                                                \
    g_checks++;                                                                       \
    if( !( cond ) ) {                                                                 \
      g_failures++;                                                                   \
      std::printf( "  FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond );               \
    }                                                                                 \
  } while( 0 )

struct Case { char const * name; std::function< void() > fn; };
static std::vector< Case > & cases() { static std::vector< Case > l_c; return l_c; }
struct Reg { Reg( char const * n, std::function< void() > f ) { cases().push_back( { n, f } ); } };
#define TEST( name ) static void name(); static Reg reg_##name( #name, name ); static void name()

// ids of a string of single-character dims
static std::vector< int64_t > ids( char const * s ) {
  std::vector< int64_t > l_v;
  for( ; *s; s++ ) l_v.push_back( *s );
  return l_v;
}

TEST( dim_types_of_out_left_right ) {
  // out iexfghy, left ieaxcgy, right afxchy (letters mapped to 0..8)
  int64_t l_out[7]   = { 0, 1, 2, 3, 4, 5, 6 };
  int64_t l_left[7]  = { 0, 1, 7, 2, 8, 4, 6 };
  int64_t l_right[6] = { 7, 3, 2, 8, 5, 6 };
  dim_t l_t_out[7], l_t_left[7], l_t_right[6];
  backend::BinaryContraction::dim_types( 7, 6, 7, l_left, l_right, l_out, UNDEFINED_DIM, M, N, C, l_t_out );
  dim_t const l_e_out[7] = { M, M, C, N, M, N, C };
  for( int l_i = 0; l_i < 7; l_i++ ) CHECK( l_t_out[l_i] == l_e_out[l_i] );
  backend::BinaryContraction::dim_types( 6, 7, 7, l_right, l_out, l_left, I, K, M, C, l_t_left );
  dim_t const l_e_left[7] = { M, M, K, C, K, M, C };
  for( int l_i = 0; l_i < 7; l_i++ ) CHECK( l_t_left[l_i] == l_e_left[l_i] );
  backend::BinaryContraction::dim_types( 7, 7, 6, l_left, l_out, l_right, J, K, N, C, l_t_right );
  dim_t const l_e_right[6] = { K, N, C, K, N, C };
  for( int l_i = 0; l_i < 6; l_i++ ) CHECK( l_t_right[l_i] == l_e_right[l_i] );
}

TEST( filter_dim_ids_by_type ) {
  int64_t l_ids[7] = { 10, 11, 12, 13, 14, 15, 16 };
  dim_t l_types[7] = { M, M, C, N, M, N, C };
  int64_t l_m[3], l_n[2], l_c[2];
  CHECK( backend::BinaryContraction::filter_dim_ids( 7, M, l_types, l_ids, l_m ) == 3 );
  CHECK( l_m[0] == 10 && l_m[1] == 11 && l_m[2] == 14 );
  CHECK( backend::BinaryContraction::filter_dim_ids( 7, N, l_types, l_ids, l_n ) == 2 );
  CHECK( l_n[0] == 13 && l_n[1] == 15 );
  CHECK( backend::BinaryContraction::filter_dim_ids( 7, C, l_types, l_ids, l_c ) == 2 );
  CHECK( l_c[0] == 12 && l_c[1] == 16 );
}

TEST( dim_types_ids_and_strides ) {
  // abkl,cdkl->abcd
  std::vector< int64_t > l_l = ids( "abkl" ), l_r = ids( "cdkl" ), l_o = ids( "abcd" );
  std::vector< dim_t > l_t;
  std::vector< int64_t > l_c, l_m, l_n, l_k, l_i, l_j;
  backend::BinaryContraction::dim_types_ids( 4, 4, 4, l_l.data(), l_r.data(), l_o.data(), &l_t,
                                             &l_c, &l_m, &l_n, &l_k, &l_i, &l_j );
  CHECK( l_c.empty() && l_i.empty() && l_j.empty() );
  CHECK( l_m == ids( "ab" ) && l_n == ids( "cd" ) && l_k == ids( "kl" ) );
  std::map< int64_t, int64_t > l_sizes = { { 'a', 32 }, { 'b', 16 }, { 'c', 32 }, { 'd', 16 }, { 'k', 32 }, { 'l', 16 } };
  std::map< int64_t, int64_t > l_s;
  backend::BinaryContraction::strides( 4, l_l.data(), &l_sizes, &l_s );
  CHECK( l_s['a'] == 8192 && l_s['b'] == 512 && l_s['k'] == 16 && l_s['l'] == 1 );
  // size-1 dims get stride 0
  std::map< int64_t, int64_t > l_sizes1 = { { 'a', 3 }, { 'b', 1 }, { 'c', 5 } };
  std::vector< int64_t > l_abc = ids( "abc" );
  backend::BinaryContraction::strides( 3, l_abc.data(), &l_sizes1, &l_s );
  CHECK( l_s['a'] == 5 && l_s['b'] == 0 && l_s['c'] == 1 );
}

TEST( unary_stride_derivation ) {
  std::map< int64_t, int64_t > l_sizes = { { 0, 2 }, { 1, 3 }, { 2, 4 } };
  int64_t l_in[3] = { 0, 1, 2 }, l_out[3] = { 0, 2, 1 };
  int64_t l_s_in[3], l_s_out[3];
  backend::Unary::strides( 3, &l_sizes, l_in, l_s_in );
  backend::Unary::strides( 3, &l_sizes, l_out, l_s_out );
  backend::Unary::order_strides_output_based( 3, l_in, l_out, l_s_in );
  CHECK( l_s_in[0] == 12 && l_s_in[1] == 1 && l_s_in[2] == 4 );
  CHECK( l_s_out[0] == 12 && l_s_out[1] == 3 && l_s_out[2] == 1 );
}

TEST( expression_histogram ) {
  int64_t l_str[8] = { 0, 2, 3, 1, 0, 4, 0, 2 };
  int64_t l_h[5] = { -1, -1, -1, -1, -1 };
  frontend::EinsumExpression::histogram( 5, 8, l_str, l_h );
  CHECK( l_h[0] == 3 && l_h[1] == 1 && l_h[2] == 2 && l_h[3] == 1 && l_h[4] == 1 );
}

TEST( expression_substring_out ) {
  int64_t l_left[4] = { 1, 4, 2, 0 }, l_right[3] = { 0, 5, 2 };
  int64_t l_h[6] = { 3, 5, 2, 7, 9, 2 };
  std::vector< int64_t > l_sub;
  frontend::EinsumExpression::substring_out( 4, 3, l_left, l_right, l_h, l_sub );
  CHECK( l_sub == std::vector< int64_t >( { 0, 1, 4, 5 } ) );
}

TEST( expression_unique_tensor_ids ) {
  int64_t l_path[6] = { 1, 2, 2, 0, 0, 1 };
  int64_t l_u[6] = { 0 };
  frontend::EinsumExpression::unique_tensor_ids( 3, l_path, l_u );
  int64_t const l_e[6] = { 1, 2, 4, 0, 3, 5 };
  for( int l_i = 0; l_i < 6; l_i++ ) CHECK( l_u[l_i] == l_e[l_i] );
}

TEST( swap_inputs_cases ) {
  auto swap = []( char const * l, char const * r, char const * o ) {
    std::vector< int64_t > a = ids( l ), b = ids( r ), c = ids( o );
    return backend::BinaryPrimitives::swap_inputs( a.size(), b.size(), c.size(), a.data(), b.data(), c.data() );
  };
  CHECK( swap( "ab", "ca", "cb" ) == false );
  CHECK( swap( "ca", "ab", "cb" ) == true );
  CHECK( swap( "abd", "cad", "cbd" ) == false );
  CHECK( swap( "cad", "abd", "cbd" ) == true );
  // MLP layer of BASELINE config 4: bi,ih->bh has N (h) fastest -> swap
  CHECK( swap( "bi", "ih", "bh" ) == true );
}

// runs reorder on single-character ids and returns "left|right|out"
static std::string reorder( tenord_t i_ord, std::map< int64_t, int64_t > const & i_sizes,
                            char const * i_l, char const * i_r, char const * i_o,
                            int64_t cb0, int64_t cb1, int64_t mb0, int64_t mb1,
                            int64_t nb0, int64_t nb1, int64_t kb0, int64_t kb1 ) {
  backend::BinaryPrimitives l_bp;
  l_bp.init( cb0, cb1, mb0, mb1, nb0, nb1, kb0, kb1 );
  std::vector< int64_t > l = ids( i_l ), r = ids( i_r ), o = ids( i_o );
  err_t l_err = l_bp.reorder( i_ord, l.size(), r.size(), o.size(), &i_sizes, l.data(), r.data(), o.data() );
  if( l_err != err_t::SUCCESS ) return "error";
  std::string s;
  for( int64_t x : l ) s += char( x );
  s += "|";
  for( int64_t x : r ) s += char( x );
  s += "|";
  for( int64_t x : o ) s += char( x );
  return s;
}

TEST( reorder_known_answers ) {
  tenord_t const T1 = tenord_t::LEFT_BC_BM_BK_BI_KB_MB_RIGHT_BC_BN_BK_BJ_NB_KB_OUT_NATIVE;
  tenord_t const T2 = tenord_t::LEFT_BC_BM_BK_BI_KB_MB_CB_RIGHT_BC_BN_BK_BJ_NB_KB_CB_OUT_NATIVE;
  tenord_t const T3 = tenord_t::LEFT_BC_BM_BK_BI_CB_KB_MB_RIGHT_BC_BN_BK_BJ_CB_NB_KB_OUT_NATIVE;
  std::map< int64_t, int64_t > s2 = { { 'a', 2 }, { 'b', 2 }, { 'c', 2 } };
  CHECK( reorder( T1, s2, "ab", "ca", "cb", 2, 8, 2, 8, 2, 8, 2, 8 ) == "ab|ca|cb" );
  std::map< int64_t, int64_t > sk = { { 'a', 2 }, { 'b', 3 }, { 'c', 2 }, { 'd', 2 } };
  CHECK( reorder( T1, sk, "bac", "dba", "dc", 2, 8, 2, 8, 2, 8, 2, 8 ) == "abc|dab|dc" );
  CHECK( reorder( T1, s2, "ba", "ca", "cb", 2, 8, 2, 8, 2, 8, 2, 8 ) == "ab|ca|cb" );
  CHECK( reorder( T1, s2, "ab", "ac", "cb", 2, 8, 2, 8, 2, 8, 2, 8 ) == "ab|ca|cb" );
  std::map< int64_t, int64_t > s6 = { { 'a', 2 }, { 'b', 2 }, { 'c', 2 }, { 'd', 2 }, { 'e', 2 }, { 'f', 2 }, { 'x', 2 } };
  CHECK( reorder( T1, s6, "abcde", "fde", "bfca", 2, 8, 2, 8, 2, 8, 2, 8 ) == "bdeca|fde|bfca" );
  CHECK( reorder( T1, s6, "xabcd", "bcaxef", "fxed", 2, 8, 2, 8, 2, 8, 2, 8 ) == "xabcd|xfeabc|fxed" );
  // TCCG setting #1 shapes
  std::map< int64_t, int64_t > st = { { 'a', 48 }, { 'b', 36 }, { 'c', 24 }, { 'd', 36 }, { 'e', 48 }, { 'f', 36 }, { 'x', 16 } };
  CHECK( reorder( T1, st, "efbad", "cf", "abcde", 4, 8, 32, 128, 16, 64, 64, 512 ) == "abdfe|cf|abcde" );
  CHECK( reorder( T2, st, "efbadx", "cfx", "abcdex", 4, 8, 32, 128, 16, 64, 64, 512 ) == "abdfex|cfx|abcdex" );
  CHECK( reorder( T1, st, "efbadx", "cfx", "abcdxe", 4, 8, 32, 128, 16, 64, 64, 512 ) == "xabdfe|xcf|abcdxe" );
  CHECK( reorder( T1, st, "efbadx", "cfx", "abcxde", 4, 8, 32, 128, 16, 64, 64, 512 ) == "xabdfe|xcf|abcxde" );
  // TCCG setting #8, inputs already swapped
  std::map< int64_t, int64_t > s8 = { { 'a', 24 }, { 'b', 20 }, { 'c', 20 }, { 'd', 24 }, { 'e', 20 }, { 'f', 20 }, { 'g', 24 } };
  CHECK( reorder( T1, s8, "gfbc", "dega", "abcdef", 4, 8, 32, 128, 16, 64, 64, 512 ) == "bcgf|adeg|abcdef" );
  // packed GEMM ordering (C blocks outside the K block)
  std::map< int64_t, int64_t > sp = { { 'a', 4 }, { 'b', 4 }, { 'c', 4 }, { 'x', 16 } };
  CHECK( reorder( T3, sp, "abx", "cax", "cbx", 4, 8, 32, 128, 16, 64, 64, 512 ) == "xab|xca|cbx" );
}

// blocked dims as "cb|mb|nb|kb" (single-character ids)
static std::string blocking( primblo_t i_pb, std::map< int64_t, int64_t > const & i_sizes,
                             char const * i_left, char const * i_right, char const * i_out,
                             std::array< int64_t, 8 > i_targets,
                             std::map< int64_t, int64_t > const * i_sl = nullptr,
                             std::map< int64_t, int64_t > const * i_sr = nullptr,
                             std::map< int64_t, int64_t > const * i_so = nullptr ) {
  backend::BinaryPrimitives l_bp;
  l_bp.init( i_targets[0], i_targets[1], i_targets[2], i_targets[3],
             i_targets[4], i_targets[5], i_targets[6], i_targets[7] );
  std::vector< int64_t > l_l = ids( i_left ), l_r = ids( i_right ), l_o = ids( i_out );
  std::vector< int64_t > l_cb, l_mb, l_nb, l_kb;
  err_t l_err = l_bp.blocking( i_pb, (int64_t) l_l.size(), (int64_t) l_r.size(), (int64_t) l_o.size(),
                               l_l.data(), l_r.data(), l_o.data(), &i_sizes, i_sl, i_sr, i_so,
                               &l_cb, &l_mb, &l_nb, &l_kb );
  if( l_err != err_t::SUCCESS ) return "error";
  std::string l_s;
  bool l_first = true;
  for( auto const * l_v : { &l_cb, &l_mb, &l_nb, &l_kb } ) {
    if( !l_first ) l_s += "|";
    l_first = false;
    for( int64_t l_id : *l_v ) l_s += char( l_id );
  }
  return l_s;
}

// reference src/backend/BinaryPrimitives.test.cpp:64-626
TEST( blocking_known_answers ) {
  primblo_t const B1 = primblo_t::LEFT_KB_X_MB_CB_RIGHT_NB_X_KB_CB_OUT_NB_X_MB_CB;
  primblo_t const B2 = primblo_t::LEFT_X_CB_KB_MB_RIGHT_X_CB_NB_KB_OUT_NB_X_MB_CB;
  std::array< int64_t, 8 > const small = { 2, 8, 2, 8, 2, 8, 2, 8 };
  std::array< int64_t, 8 > const tccg = { 4, 8, 32, 128, 16, 64, 64, 512 };
  std::array< int64_t, 8 > const tccg_large_m = { 4, 8, 32, 4096, 16, 64, 64, 512 };
  // matrix-matrix multiplication
  std::map< int64_t, int64_t > s3 = { { 'a', 2 }, { 'b', 2 }, { 'c', 2 } };
  CHECK( blocking( B1, s3, "ab", "ca", "cb", small ) == "|b|c|a" );
  // non-contiguous strides: only d (M) and e, f (N) are blocked
  std::map< int64_t, int64_t > s6 = { { 'a', 2 }, { 'b', 2 }, { 'c', 2 }, { 'd', 2 }, { 'e', 2 }, { 'f', 2 } };
  std::map< int64_t, int64_t > sl = { { 'd', 1 }, { 'c', 2 }, { 'b', 4 }, { 'a', 8 } };
  std::map< int64_t, int64_t > sr = { { 'b', 3 }, { 'a', 6 }, { 'f', 12 }, { 'e', 24 } };
  std::map< int64_t, int64_t > so = { { 'd', 1 }, { 'c', 3 }, { 'f', 6 }, { 'e', 12 } };
  CHECK( blocking( B1, s6, "abcd", "efab", "efcd", small, &sl, &sr, &so ) == "|d|ef|" );
  // high-dimensional contraction (integer ids 0..14): one dim per blocked type
  {
    std::map< int64_t, int64_t > sz = { { 0, 32 }, { 1, 96 }, { 2, 3 }, { 3, 3 }, { 4, 3 }, { 5, 3 }, { 6, 2 },
                                        { 7, 2 }, { 8, 64 }, { 9, 2 }, { 10, 2 }, { 11, 64 }, { 12, 2 },
                                        { 13, 2 }, { 14, 64 } };
    int64_t const l_l[8] = { 12, 13, 2, 3, 9, 10, 11, 14 };
    int64_t const l_r[5] = { 0, 9, 10, 1, 11 };
    int64_t const l_o[5] = { 0, 1, 12, 13, 14 };
    backend::BinaryPrimitives l_bp;
    l_bp.init( 4, 16, 32, 128, 12, 64, 32, 512 );
    std::vector< int64_t > l_cb, l_mb, l_nb, l_kb;
    CHECK( l_bp.blocking( B1, 8, 5, 5, l_l, l_r, l_o, &sz, nullptr, nullptr, nullptr,
                          &l_cb, &l_mb, &l_nb, &l_kb ) == err_t::SUCCESS );
    CHECK( l_cb.size() == 0 && l_mb.size() == 1 && l_nb.size() == 1 && l_kb.size() == 1 );
  }
  // TCCG setting #1, plain and reordered, with and without a batch dim
  std::map< int64_t, int64_t > st = { { 'a', 48 }, { 'b', 36 }, { 'c', 24 }, { 'd', 36 }, { 'e', 48 }, { 'f', 36 },
                                      { 'x', 16 } };
  CHECK( blocking( B1, st, "efbad", "cf", "abcde", tccg ) == "||c|f" );
  CHECK( blocking( B1, st, "fbade", "cf", "abcde", tccg ) == "|e|c|f" );
  CHECK( blocking( B1, st, "efbadx", "cfx", "abcdex", tccg ) == "x||c|f" );
  CHECK( blocking( B1, st, "fbadex", "cfx", "abcdex", tccg ) == "x|e|c|f" );
  CHECK( blocking( B1, st, "fbadex", "cfx", "abcdex", tccg_large_m ) == "x|de|c|f" );
  CHECK( blocking( B1, st, "fbade", "cf", "abcde", tccg_large_m ) == "|de|c|f" );
  // batched GEMM: left kb cb mb, right nb cb kb, out nb mb cb
  std::map< int64_t, int64_t > sb = { { 'a', 2 }, { 'b', 3 }, { 'c', 2 }, { 'd', 2 } };
  CHECK( blocking( B2, sb, "abc", "adb", "dca", small ) == "a|c|d|b" );
  // unknown blocking
  CHECK( blocking( primblo_t::UNDEFINED_PRIMBLO, s3, "ab", "ca", "cb", small ) == "error" );
}

TEST( ascii_parsers ) {
  std::string l_std;
  frontend::EinsumExpressionAscii::schar_to_standard( "iae,bf,dcba,cg,dh->hgfei", l_std );
  CHECK( l_std == "[i,a,e],[b,f],[d,c,b,a],[c,g],[d,h]->[h,g,f,e,i]" );
  std::string l_sc;
  frontend::EinsumExpressionAscii::standard_to_schar( "[xix,a,e],[b,f],[d,c,b,a],[c,g],[d,h]->[h,g,f,e,xix]", l_sc );
  CHECK( l_sc == "IAE,BF,DCBA,CG,DH->HGFEI" );
  frontend::EinsumExpressionAscii::standard_to_schar( "[13,5,9],[6,10],[8,7,6,5],[7,11],[8,12]->[12,11,10,9,13]", l_sc );
  CHECK( l_sc == "IAE,BF,DCBA,CG,DH->HGFEI" );
  std::vector< std::string > l_t;
  frontend::EinsumExpressionAscii::parse_tensors( "[i,a,e],[b,f],[d,c,b,a],[c,g],[d,h]->[h,g,f,e,i]", l_t );
  CHECK( l_t.size() == 6 && l_t[0] == "i,a,e" && l_t[2] == "d,c,b,a" && l_t[5] == "h,g,f,e,i" );
  frontend::EinsumExpressionAscii::parse_tensors( "[13,5,9],[6,10],[8,7,6,5],[7,11],[8,12]->[12,11,10,9,13]", l_t );
  CHECK( l_t.size() == 6 && l_t[0] == "13,5,9" && l_t[4] == "8,12" && l_t[5] == "12,11,10,9,13" );
  std::map< std::string, int64_t > l_ids;
  frontend::EinsumExpressionAscii::parse_dim_ids( "[i,aaa,e],[b,f],[d,c,b,aaa],[c,g],[d,h]->[h,g,f,e,i]", l_ids );
  CHECK( l_ids.size() == 9 && l_ids["aaa"] == 0 && l_ids["b"] == 1 && l_ids["e"] == 4 && l_ids["i"] == 8 );
  frontend::EinsumExpressionAscii::parse_dim_ids( "[13,5,9],[6,10],[8,7,6,5],[7,11],[8,12]->[12,11,10,9,13]", l_ids );
  CHECK( l_ids.size() == 9 && l_ids["5"] == 0 && l_ids["9"] == 4 && l_ids["10"] == 5 && l_ids["13"] == 8 );
  std::vector< int64_t > l_v;
  frontend::EinsumExpressionAscii::parse_dim_sizes( "32, 16,32,16,32,16", l_v );
  CHECK( l_v == std::vector< int64_t >( { 32, 16, 32, 16, 32, 16 } ) );
  frontend::EinsumExpressionAscii::parse_path( "(0,1),(0,3),(0,2),(0,1)", l_v );
  CHECK( l_v == std::vector< int64_t >( { 0, 1, 0, 3, 0, 2, 0, 1 } ) );
  data_t l_dt;
  frontend::EinsumExpressionAscii::parse_dtype( "BF16", l_dt );
  CHECK( l_dt == BF16 );
  frontend::EinsumExpressionAscii::parse_dtype( "FP64", l_dt );
  CHECK( l_dt == FP64 );
  frontend::EinsumExpressionAscii::parse_dtype( "INT8", l_dt );
  CHECK( l_dt == UNDEFINED_DTYPE );
}

TEST( tree_parser ) {
  std::string l_tree = "[[3,0]->[0,3]],[[3,2,4],[1,4,2]->[1,2,3]]->[0,1,2]";
  int64_t l_n = frontend::EinsumTreeAscii::count_nodes( l_tree );
  CHECK( l_n == 6 );
  std::vector< std::vector< int64_t > > l_ids( l_n ), l_ch( l_n );
  int64_t l_parsed = 0;
  CHECK( frontend::EinsumTreeAscii::parse_tree( l_tree, l_ids, l_ch, l_parsed ) == err_t::SUCCESS );
  CHECK( l_parsed == 6 );
  // post-order: leaf [3,0], unary [0,3], leaf [3,2,4], leaf [1,4,2], binary [1,2,3], root [0,1,2]
  CHECK( l_ids[0] == std::vector< int64_t >( { 3, 0 } ) && l_ch[0].empty() );
  CHECK( l_ids[1] == std::vector< int64_t >( { 0, 3 } ) && l_ch[1] == std::vector< int64_t >( { 0 } ) );
  CHECK( l_ids[4] == std::vector< int64_t >( { 1, 2, 3 } ) && l_ch[4] == std::vector< int64_t >( { 2, 3 } ) );
  CHECK( l_ids[5] == std::vector< int64_t >( { 0, 1, 2 } ) && l_ch[5] == std::vector< int64_t >( { 1, 4 } ) );
  std::map< int64_t, int64_t > l_sizes;
  frontend::EinsumTreeAscii::parse_dim_size( "2,3,4,5,6", l_ids, l_sizes );
  CHECK( l_sizes.size() == 5 && l_sizes[0] == 2 && l_sizes[4] == 6 );
}

TEST( memory_arena_two_sided_stack ) {
  backend::MemoryManager l_mm;
  // layer 1 (odd): right side; layer 2 (even): left side
  l_mm.m_layer_id = 2;
  int64_t l_a = l_mm.reserve_memory( 1000 );   // left [0, 1024) (256-byte granules)
  int64_t l_b = l_mm.reserve_memory( 300 );    // left [1024, 1536)
  l_mm.m_layer_id = 1;
  int64_t l_c = l_mm.reserve_memory( 512 );    // right [-512, 0)
  CHECK( l_a > 0 && l_b > 0 && l_c < 0 );
  CHECK( l_mm.get_required_memory() == 1536 + 512 );
  l_mm.remove_reservation( l_b );
  l_mm.m_layer_id = 2;
  int64_t l_d = l_mm.reserve_memory( 256 );    // reuses [1024, 1280)
  CHECK( l_d > 0 && l_mm.get_required_memory() == 1536 + 512 );
  l_mm.remove_reservation( l_a );
  l_mm.remove_reservation( l_c );
  l_mm.remove_reservation( l_d );
}

// host stand-ins for the arena allocator, counting live allocations
static int g_live_allocs = 0;
static int host_alloc( void ** o_ptr, int64_t i_bytes ) {
  *o_ptr = std::malloc( std::size_t( i_bytes ) );
  if( *o_ptr != nullptr ) g_live_allocs++;
  return *o_ptr == nullptr;
}
static int host_free( void * i_ptr ) {
  std::free( i_ptr );
  g_live_allocs--;
  return 0;
}

TEST( memory_arena_grows_with_a_later_plan ) {
  {
    backend::MemoryManager l_mm;
    l_mm.set_allocator( host_alloc, host_free );
    // first plan: peak 1024 + 512
    l_mm.m_layer_id = 0;
    int64_t l_a = l_mm.reserve_memory( 1024 );
    l_mm.m_layer_id = 1;
    int64_t l_b = l_mm.reserve_memory( 512 );
    CHECK( l_mm.alloc_all_memory() == err_t::SUCCESS );
    CHECK( l_mm.get_allocated_memory() == 1536 && l_mm.get_required_memory() == 1536 );
    char * l_base = static_cast< char * >( l_mm.get_mem_ptr( l_a ) );
    CHECK( static_cast< char * >( l_mm.get_mem_ptr( l_b ) ) == l_base + 1024 );
    l_mm.remove_reservation( l_a );
    l_mm.remove_reservation( l_b );
    // second plan on the same manager with a larger peak: every pointer it
    // hands out must stay inside the (grown) allocation
    l_mm.m_layer_id = 0;
    int64_t l_c = l_mm.reserve_memory( 4096 );
    l_mm.m_layer_id = 1;
    int64_t l_d = l_mm.reserve_memory( 2048 );
    CHECK( l_mm.get_required_memory() == 6144 );
    CHECK( l_mm.alloc_all_memory() == err_t::SUCCESS );
    CHECK( l_mm.get_allocated_memory() >= l_mm.get_required_memory() );
    CHECK( g_live_allocs == 1 );
    char * l_lo = static_cast< char * >( l_mm.get_mem_ptr( l_c ) );
    char * l_hi = static_cast< char * >( l_mm.get_mem_ptr( l_d ) );
    CHECK( l_hi - l_lo == 4096 );
    CHECK( l_hi + 2048 - l_lo <= l_mm.get_allocated_memory() );
    // a smaller plan afterwards keeps the allocation
    l_mm.remove_reservation( l_c );
    l_mm.remove_reservation( l_d );
    l_mm.m_layer_id = 0;
    l_mm.reserve_memory( 256 );
    CHECK( l_mm.alloc_all_memory() == err_t::SUCCESS && g_live_allocs == 1 );
  }
  CHECK( g_live_allocs == 0 );
}

int main() {
  for( Case const & l_c : cases() ) {
    int const l_before = g_failures;
    l_c.fn();
    std::printf( "%s %s\n", g_failures == l_before ? "PASS" : "FAIL", l_c.name );
  }
  std::printf( "%d checks, %d failures\n", g_checks, g_failures );
  return g_failures == 0 ? EXIT_SUCCESS : EXIT_FAILURE;
}
