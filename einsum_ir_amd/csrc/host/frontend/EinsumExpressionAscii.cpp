#include "EinsumExpressionAscii.h"
#include <algorithm>
#include <set>

namespace {
  std::string strip_spaces( std::string i_s ) {
    i_s.erase( std::remove( i_s.begin(), i_s.end(), ' ' ), i_s.end() );
    return i_s;
  }

  // numeric names compare as numbers, everything else lexicographically
  bool name_less( std::string const & i_a, std::string const & i_b ) {
    try {
      return std::stoi( i_a ) < std::stoi( i_b );
    }
    catch( ... ) {
      return i_a < i_b;
    }
  }

  std::string utf8( uint32_t i_cp ) {
    std::string l_s;
    if( i_cp < 0x80 ) {
      l_s += char( i_cp );
    }
    else if( i_cp < 0x800 ) {
      l_s += char( 0xC0 | ( i_cp >> 6 ) );
      l_s += char( 0x80 | ( i_cp & 0x3F ) );
    }
    else if( i_cp < 0x10000 ) {
      l_s += char( 0xE0 | ( i_cp >> 12 ) );
      l_s += char( 0x80 | ( ( i_cp >> 6 ) & 0x3F ) );
      l_s += char( 0x80 | ( i_cp & 0x3F ) );
    }
    else {
      l_s += char( 0xF0 | ( i_cp >> 18 ) );
      l_s += char( 0x80 | ( ( i_cp >> 12 ) & 0x3F ) );
      l_s += char( 0x80 | ( ( i_cp >> 6 ) & 0x3F ) );
      l_s += char( 0x80 | ( i_cp & 0x3F ) );
    }
    return l_s;
  }
}

void einsum_ir::frontend::EinsumExpressionAscii::split_string( std::string                const & i_input,
                                                               std::string                const & i_separation,
                                                               std::vector< std::string >       & o_output ) {
  std::string l_rest = i_input;
  while( !l_rest.empty() ) {
    std::size_t l_pos = l_rest.find( i_separation );
    if( l_pos == std::string::npos ) break;
    o_output.push_back( l_rest.substr( 0, l_pos ) );
    l_rest.erase( 0, l_pos + i_separation.size() );
  }
  if( !l_rest.empty() ) {
    o_output.push_back( l_rest );
  }
}

void einsum_ir::frontend::EinsumExpressionAscii::schar_to_standard( std::string const & i_expr_string,
                                                                    std::string       & o_expr_string ) {
  o_expr_string.clear();
  std::string l_expr = strip_spaces( i_expr_string );
  std::vector< std::string > l_sides;
  split_string( l_expr, "->", l_sides );
  if( l_sides.empty() ) return;
  std::vector< std::string > l_inputs;
  split_string( l_sides[0], ",", l_inputs );
  auto bracket = []( std::string const & i_t ) {
    std::string l_s = "[";
    for( std::size_t l_i = 0; l_i < i_t.size(); l_i++ ) {
      if( l_i ) l_s += ",";
      l_s += i_t[l_i];
    }
    return l_s + "]";
  };
  for( std::size_t l_te = 0; l_te < l_inputs.size(); l_te++ ) {
    if( l_te ) o_expr_string += ",";
    o_expr_string += bracket( l_inputs[l_te] );
  }
  o_expr_string += "->" + bracket( l_sides.size() > 1 ? l_sides[1] : std::string() );
}

void einsum_ir::frontend::EinsumExpressionAscii::standard_to_schar( std::string const & i_expr_string,
                                                                    std::string       & o_expr_string ) {
  o_expr_string.clear();
  std::vector< std::string > l_tensors;
  parse_tensors( i_expr_string, l_tensors );
  if( l_tensors.empty() ) return;

  std::map< std::string, int64_t > l_ids;
  // ids over the input tensors (as the reference: output names are expected to occur in an input)
  std::vector< std::string > l_inputs( l_tensors.begin(), l_tensors.end() - 1 );
  std::set< std::string > l_names;
  for( std::string const & l_t : l_inputs ) {
    std::vector< std::string > l_dims;
    split_string( l_t, ",", l_dims );
    l_names.insert( l_dims.begin(), l_dims.end() );
  }
  std::vector< std::string > l_sorted( l_names.begin(), l_names.end() );
  std::sort( l_sorted.begin(), l_sorted.end(), name_less );
  for( std::size_t l_i = 0; l_i < l_sorted.size(); l_i++ ) l_ids[ l_sorted[l_i] ] = (int64_t) l_i;

  bool const l_ascii = l_sorted.size() <= 52;
  auto to_char = [&]( std::string const & i_name ) {
    int64_t l_id = l_ids[i_name];
    if( l_ascii ) return std::string( 1, char( l_id < 26 ? 'A' + l_id : 'a' + l_id - 26 ) );
    return utf8( uint32_t( l_id + 161 ) );
  };
  for( std::size_t l_te = 0; l_te < l_tensors.size(); l_te++ ) {
    if( l_te == l_tensors.size() - 1 ) o_expr_string += "->";
    else if( l_te ) o_expr_string += ",";
    std::vector< std::string > l_dims;
    split_string( l_tensors[l_te], ",", l_dims );
    for( std::string const & l_d : l_dims ) o_expr_string += to_char( l_d );
  }
}

void einsum_ir::frontend::EinsumExpressionAscii::parse_tensors( std::string                const & i_expr_string,
                                                                std::vector< std::string >       & o_tensors ) {
  o_tensors.clear();
  std::string l_expr = strip_spaces( i_expr_string );
  if( l_expr.size() < 2 ) return;
  l_expr = l_expr.substr( 1, l_expr.size() - 2 );   // outer brackets
  std::vector< std::string > l_sides;
  split_string( l_expr, "]->[", l_sides );
  if( l_sides.size() == 1 ) l_sides.push_back( "" );
  split_string( l_sides[0], "],[", o_tensors );
  o_tensors.push_back( l_sides[1] );
}

void einsum_ir::frontend::EinsumExpressionAscii::parse_dim_sizes( std::string            const & i_dim_sizes_string,
                                                                  std::vector< int64_t >       & o_dim_sizes ) {
  o_dim_sizes.clear();
  std::vector< std::string > l_parts;
  split_string( strip_spaces( i_dim_sizes_string ), ",", l_parts );
  for( std::string const & l_p : l_parts ) o_dim_sizes.push_back( std::stoll( l_p ) );
}

void einsum_ir::frontend::EinsumExpressionAscii::parse_path( std::string            const & i_expr_string,
                                                             std::vector< int64_t >       & o_path ) {
  o_path.clear();
  std::string l_s = strip_spaces( i_expr_string );
  l_s.erase( std::remove( l_s.begin(), l_s.end(), '(' ), l_s.end() );
  l_s.erase( std::remove( l_s.begin(), l_s.end(), ')' ), l_s.end() );
  std::vector< std::string > l_parts;
  split_string( l_s, ",", l_parts );
  for( std::string const & l_p : l_parts ) o_path.push_back( std::stoll( l_p ) );
}

void einsum_ir::frontend::EinsumExpressionAscii::parse_dim_ids( std::string                      const & i_expr_string,
                                                                std::map< std::string, int64_t >       & o_map_dim_name_to_id ) {
  o_map_dim_name_to_id.clear();
  std::vector< std::string > l_tensors;
  parse_tensors( i_expr_string, l_tensors );
  std::set< std::string > l_names;
  for( std::string const & l_t : l_tensors ) {
    std::vector< std::string > l_dims;
    split_string( l_t, ",", l_dims );
    l_names.insert( l_dims.begin(), l_dims.end() );
  }
  std::vector< std::string > l_sorted( l_names.begin(), l_names.end() );
  std::sort( l_sorted.begin(), l_sorted.end(), name_less );
  for( std::size_t l_i = 0; l_i < l_sorted.size(); l_i++ ) {
    o_map_dim_name_to_id.insert( { l_sorted[l_i], (int64_t) l_i } );
  }
}

void einsum_ir::frontend::EinsumExpressionAscii::parse_dtype( std::string const & i_dtype_string,
                                                              data_t            & o_dtype ) {
  if(      i_dtype_string == "FP32" || i_dtype_string == "CPX_FP32" ) o_dtype = FP32;
  else if( i_dtype_string == "FP64" || i_dtype_string == "CPX_FP64" ) o_dtype = FP64;
  else if( i_dtype_string == "BF16" )                                 o_dtype = BF16;
  else                                                                o_dtype = UNDEFINED_DTYPE;
}

void einsum_ir::frontend::EinsumExpressionAscii::parse_ctype( std::string const & i_dtype_string,
                                                              complex_t         & o_ctype ) {
  if(      i_dtype_string == "FP32" || i_dtype_string == "FP64" || i_dtype_string == "BF16" ) o_ctype = REAL_ONLY;
  else if( i_dtype_string == "CPX_FP32" || i_dtype_string == "CPX_FP64" )                    o_ctype = BATCH_INNER;
  else                                                                                       o_ctype = UNDEFINED_CTYPE;
}

void einsum_ir::frontend::EinsumExpressionAscii::parse_loop_order( std::string                      const & i_loop_string,
                                                                   std::map< std::string, int64_t > const & i_map_dim_name_to_id,
                                                                   std::vector< int64_t >                 & o_loop_order ) {
  o_loop_order.clear();
  std::vector< std::string > l_parts;
  split_string( strip_spaces( i_loop_string ), ",", l_parts );
  for( std::string const & l_p : l_parts ) o_loop_order.push_back( i_map_dim_name_to_id.at( l_p ) );
}
