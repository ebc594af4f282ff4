// Parser of the tree format "[[3,0]->[0,3]],[[3,2,4],[1,4,2]->[1,2,3]]->[0,1,2]"
// (reference src/frontend/EinsumTreeAscii.{h,cpp}:23-199).
#ifndef EINSUM_IR_FRONTEND_EINSUM_TREE_ASCII
#define EINSUM_IR_FRONTEND_EINSUM_TREE_ASCII

#include <cstdint>
#include <map>
#include <string>
#include <vector>
#include "../constants.h"

namespace einsum_ir {
  namespace frontend {
    class EinsumTreeAscii;
  }
}

class einsum_ir::frontend::EinsumTreeAscii {
  public:
    static void split_string( std::string                const & i_input,
                              std::string                const & i_separation,
                              std::vector< std::string >       & o_output );

    /** Post-order parse: children before parents, root last. **/
    static err_t parse_tree( std::string                            const & i_string_tree,
                             std::vector< std::vector < int64_t > >       & o_dim_ids,
                             std::vector< std::vector < int64_t > >       & o_children,
                             int64_t                                      & o_node_id );

    static void parse_vector( std::string            const & i_string_vector,
                              std::vector< int64_t >       & o_int_vector );

    static int64_t count_nodes( std::string const & i_string_tree );

    /** Sizes are given for the sorted distinct dim ids of the tree. **/
    static void parse_dim_size( std::string                            const & i_string_sizes,
                                std::vector< std::vector < int64_t > > const & i_dim_ids,
                                std::map< int64_t, int64_t >                 & o_map_dim_sizes );

    static err_t split_outer_operation( std::string const & i_string_tree,
                                       std::string       & o_left_tree,
                                       std::string       & o_right_tree,
                                       std::string       & o_out_tree );
};

#endif
