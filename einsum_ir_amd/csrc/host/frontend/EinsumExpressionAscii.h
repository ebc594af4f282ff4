// String formats of the bench harnesses (reference
// src/frontend/EinsumExpressionAscii.{h,cpp}): "ab,bc->ac" and
// "[a,b],[b,c]->[a,c]" expressions, dimension sizes "2,3,4", contraction
// paths "(0,1),(0,2)", dtype names, loop orders.  Dimension ids are the
// positions of the sorted dimension names (numeric names sort numerically).
#ifndef EINSUM_IR_FRONTEND_EINSUM_EXPRESSION_ASCII
#define EINSUM_IR_FRONTEND_EINSUM_EXPRESSION_ASCII

#include <cstdint>
#include <map>
#include <string>
#include <vector>
#include "../constants.h"

namespace einsum_ir {
  namespace frontend {
    class EinsumExpressionAscii;
  }
}

class einsum_ir::frontend::EinsumExpressionAscii {
  public:
    static void split_string( std::string                const & i_input,
                              std::string                const & i_separation,
                              std::vector< std::string >       & o_output );

    /** "ab,bc->ac" -> "[a,b],[b,c]->[a,c]" **/
    static void schar_to_standard( std::string const & i_expr_string,
                                   std::string       & o_expr_string );

    /** "[x,y],[y,z]->[x,z]" -> single characters A..Z a..z (UTF-8 beyond 52 dims) **/
    static void standard_to_schar( std::string const & i_expr_string,
                                   std::string       & o_expr_string );

    /** tensors of a standard expression; the output is the last entry **/
    static void parse_tensors( std::string                const & i_expr_string,
                               std::vector< std::string >       & o_tensors );

    static void parse_dim_sizes( std::string            const & i_dim_sizes_string,
                                 std::vector< int64_t >       & o_dim_sizes );

    static void parse_path( std::string            const & i_expr_string,
                            std::vector< int64_t >       & o_path );

    static void parse_dim_ids( std::string                      const & i_expr_string,
                               std::map< std::string, int64_t >       & o_map_dim_name_to_id );

    /** FP32, FP64, CPX_FP32, CPX_FP64 and the additive BF16 **/
    static void parse_dtype( std::string const & i_dtype_string,
                             data_t            & o_dtype );

    static void parse_ctype( std::string const & i_dtype_string,
                             complex_t         & o_ctype );

    static void parse_loop_order( std::string                      const & i_loop_string,
                                  std::map< std::string, int64_t > const & i_map_dim_name_to_id,
                                  std::vector< int64_t >                 & o_loop_order );
};

#endif
