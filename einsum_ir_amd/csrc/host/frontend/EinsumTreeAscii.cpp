#include "EinsumTreeAscii.h"
#include "EinsumExpressionAscii.h"
#include <algorithm>
#include <set>

void einsum_ir::frontend::EinsumTreeAscii::split_string( std::string                const & i_input,
                                                         std::string                const & i_separation,
                                                         std::vector< std::string >       & o_output ) {
  EinsumExpressionAscii::split_string( i_input, i_separation, o_output );
}

int64_t einsum_ir::frontend::EinsumTreeAscii::count_nodes( std::string const & i_string_tree ) {
  // one node per "],[" (a second operand) and per "]->[" (an operation), plus the root's leaf
  int64_t l_count = 1;
  for( std::size_t l_off = 0; l_off + 3 < i_string_tree.size(); l_off++ ) {
    if( i_string_tree.compare( l_off, 3, "],[" ) == 0 ) l_count++;
    if( i_string_tree.compare( l_off, 4, "]->[" ) == 0 ) l_count++;
  }
  return l_count;
}

einsum_ir::err_t einsum_ir::frontend::EinsumTreeAscii::parse_tree( std::string                            const & i_string_tree,
                                                                   std::vector< std::vector < int64_t > >       & o_dim_ids,
                                                                   std::vector< std::vector < int64_t > >       & o_children,
                                                                   int64_t                                      & o_node_id ) {
  if( o_node_id < 0 || (std::size_t) o_node_id >= o_dim_ids.size() || o_dim_ids.size() != o_children.size() ) {
    return err_t::COMPILATION_FAILED;
  }
  if( i_string_tree.empty() || i_string_tree[0] != '[' ) {
    parse_vector( i_string_tree, o_dim_ids[o_node_id] );
    o_node_id++;
    return err_t::SUCCESS;
  }
  std::string l_left, l_right, l_out;
  err_t l_err = split_outer_operation( i_string_tree, l_left, l_right, l_out );
  if( l_err != err_t::SUCCESS ) return l_err;

  l_err = parse_tree( l_left, o_dim_ids, o_children, o_node_id );
  if( l_err != err_t::SUCCESS ) return l_err;
  int64_t const l_id_left = o_node_id - 1;
  int64_t l_id_right = -1;
  if( !l_right.empty() ) {
    l_err = parse_tree( l_right, o_dim_ids, o_children, o_node_id );
    if( l_err != err_t::SUCCESS ) return l_err;
    l_id_right = o_node_id - 1;
  }
  if( (std::size_t) o_node_id >= o_dim_ids.size() ) return err_t::COMPILATION_FAILED;
  o_children[o_node_id].push_back( l_id_left );
  if( l_id_right >= 0 ) o_children[o_node_id].push_back( l_id_right );
  parse_vector( l_out, o_dim_ids[o_node_id] );
  o_node_id++;
  return err_t::SUCCESS;
}

void einsum_ir::frontend::EinsumTreeAscii::parse_vector( std::string            const & i_string_vector,
                                                         std::vector< int64_t >       & o_int_vector ) {
  o_int_vector.clear();
  std::string l_s = i_string_vector;
  l_s.erase( std::remove( l_s.begin(), l_s.end(), ' ' ), l_s.end() );
  std::vector< std::string > l_parts;
  split_string( l_s, ",", l_parts );
  for( std::string const & l_p : l_parts ) o_int_vector.push_back( std::stoll( l_p ) );
}

void einsum_ir::frontend::EinsumTreeAscii::parse_dim_size( std::string                            const & i_string_sizes,
                                                           std::vector< std::vector < int64_t > > const & i_dim_ids,
                                                           std::map< int64_t, int64_t >                 & o_map_dim_sizes ) {
  std::vector< int64_t > l_sizes;
  parse_vector( i_string_sizes, l_sizes );
  std::set< int64_t > l_ids;
  for( auto const & l_t : i_dim_ids ) l_ids.insert( l_t.begin(), l_t.end() );
  o_map_dim_sizes.clear();
  std::size_t l_i = 0;
  for( int64_t l_id : l_ids ) {
    if( l_i >= l_sizes.size() ) break;
    o_map_dim_sizes.insert( { l_id, l_sizes[l_i++] } );
  }
}

einsum_ir::err_t einsum_ir::frontend::EinsumTreeAscii::split_outer_operation( std::string const & i_string_tree,
                                                                              std::string       & o_left_tree,
                                                                              std::string       & o_right_tree,
                                                                              std::string       & o_out_tree ) {
  // top-level "," separates the operands, top-level "->" starts the output
  int64_t l_comma = 0, l_arrow = 0, l_depth = 0;
  int64_t const l_n = (int64_t) i_string_tree.size();
  for( int64_t l_off = 0; l_off < l_n; l_off++ ) {
    char const l_c = i_string_tree[l_off];
    if( l_c == '[' ) l_depth++;
    if( l_c == ']' ) l_depth--;
    if( l_c == ',' && l_depth == 0 ) l_comma = l_off;
    if( l_c == '-' && l_depth == 0 ) {
      l_arrow = l_off;
      break;
    }
  }
  if( l_arrow == 0 || l_arrow + 3 > l_n ) return err_t::COMPILATION_FAILED;
  // operands are "[...]" around l_comma / l_arrow, the output "[...]" after "->"
  if( l_comma != 0 ) {
    o_left_tree  = i_string_tree.substr( 1, l_comma - 2 );
    o_right_tree = i_string_tree.substr( l_comma + 2, l_arrow - l_comma - 3 );
  }
  else {
    o_left_tree = i_string_tree.substr( 1, l_arrow - 2 );
  }
  o_out_tree = i_string_tree.substr( l_arrow + 3, l_n - l_arrow - 4 );
  return err_t::SUCCESS;
}
