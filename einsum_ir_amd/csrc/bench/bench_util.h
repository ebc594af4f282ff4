// Shared parts of the command-line harnesses bench_binary, bench_unary,
// bench_expression and bench_tree: seeded input data, device buffers,
// timing, and the float64 host evaluation that checks every run.
//
// The harnesses drive the operator classes of libeinsum_ir.so on device
// buffers.  The check evaluates the same contractions on the host in float64
// (complex<double> for complex data) from the values the GPU was given.  When
// that would take more than kHostBudget multiply-adds, output dims are
// restricted to evenly spaced index values (first and last included) until it
// fits; every output entry of the restricted grid is compared.
#ifndef EINSUM_IR_BENCH_UTIL_H
#define EINSUM_IR_BENCH_UTIL_H

#include <algorithm>
#include <chrono>
#include <cmath>
#include <complex>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "einsum_ir_hip.h"

namespace etir_bench {

// ---------------------------------------------------------------------------
// input data
// ---------------------------------------------------------------------------

//! splitmix64 stream (Steele, Lea, Flood 2014): uniform [0,1) and N(0,1)
class Rng {
  uint64_t m_state;
 public:
  explicit Rng( uint64_t i_seed ) : m_state( i_seed ) {}
  uint64_t next() {
    uint64_t l_z = ( m_state += 0x9E3779B97F4A7C15ull );
    l_z = ( l_z ^ ( l_z >> 30 ) ) * 0xBF58476D1CE4E5B9ull;
    l_z = ( l_z ^ ( l_z >> 27 ) ) * 0x94D049BB133111EBull;
    return l_z ^ ( l_z >> 31 );
  }
  double uniform() { return double( next() >> 11 ) * 0x1.0p-53; }
  //! Box-Muller on two uniforms
  double normal() {
    double l_u1 = uniform(), l_u2 = uniform();
    if( l_u1 < 1e-300 ) l_u1 = 1e-300;
    return std::sqrt( -2.0 * std::log( l_u1 ) ) * std::cos( 6.283185307179586 * l_u2 );
  }
};

//! storage type of a tensor on the device
enum class Elem { F32, F64, BF16, C64, C128 };

inline int64_t elem_bytes( Elem i_e ) {
  switch( i_e ) {
    case Elem::F32:  return 4;
    case Elem::F64:  return 8;
    case Elem::BF16: return 2;
    case Elem::C64:  return 8;
    case Elem::C128: return 16;
  }
  return 0;
}

inline bool is_complex( Elem i_e ) { return i_e == Elem::C64 || i_e == Elem::C128; }

//! float -> bfloat16, round to nearest even (NaN stays NaN)
inline uint16_t to_bf16( float i_f ) {
  uint32_t l_u;
  std::memcpy( &l_u, &i_f, 4 );
  if( ( l_u & 0x7fffffffu ) > 0x7f800000u ) return uint16_t( ( l_u >> 16 ) | 0x40u );
  l_u += 0x7fffu + ( ( l_u >> 16 ) & 1u );
  return uint16_t( l_u >> 16 );
}

inline float from_bf16( uint16_t i_h ) {
  uint32_t l_u = uint32_t( i_h ) << 16;
  float l_f;
  std::memcpy( &l_f, &l_u, 4 );
  return l_f;
}

enum class Fill { UNIFORM, ONES, NORMAL };

//! A tensor's bytes as the device gets them and the same values in float64
//! (the imaginary part is 0 for real types).
struct HostData {
  Elem elem = Elem::F32;
  int64_t n = 0;
  std::vector< unsigned char > raw;
  std::vector< std::complex< double > > val;

  HostData() = default;
  HostData( Elem i_elem, int64_t i_n ) : elem( i_elem ), n( i_n ),
      raw( std::size_t( i_n * elem_bytes( i_elem ) ) ), val( std::size_t( i_n ) ) {}

  int64_t bytes() const { return n * elem_bytes( elem ); }

  void set( int64_t i_idx, double i_re, double i_im ) {
    unsigned char * l_p = raw.data() + i_idx * elem_bytes( elem );
    switch( elem ) {
      case Elem::F32:  { float  l_v = float( i_re ); std::memcpy( l_p, &l_v, 4 ); val[i_idx] = l_v; break; }
      case Elem::F64:  { std::memcpy( l_p, &i_re, 8 ); val[i_idx] = i_re; break; }
      case Elem::BF16: { uint16_t l_h = to_bf16( float( i_re ) ); std::memcpy( l_p, &l_h, 2 );
                         val[i_idx] = from_bf16( l_h ); break; }
      case Elem::C64:  { float l_v[2] = { float( i_re ), float( i_im ) }; std::memcpy( l_p, l_v, 8 );
                         val[i_idx] = { l_v[0], l_v[1] }; break; }
      case Elem::C128: { double l_v[2] = { i_re, i_im }; std::memcpy( l_p, l_v, 16 );
                         val[i_idx] = { i_re, i_im }; break; }
    }
  }

  //! decodes raw (e.g. after a download) into val
  void decode() {
    for( int64_t l_i = 0; l_i < n; l_i++ ) {
      unsigned char const * l_p = raw.data() + l_i * elem_bytes( elem );
      switch( elem ) {
        case Elem::F32:  { float l_v; std::memcpy( &l_v, l_p, 4 ); val[l_i] = l_v; break; }
        case Elem::F64:  { double l_v; std::memcpy( &l_v, l_p, 8 ); val[l_i] = l_v; break; }
        case Elem::BF16: { uint16_t l_h; std::memcpy( &l_h, l_p, 2 ); val[l_i] = from_bf16( l_h ); break; }
        case Elem::C64:  { float l_v[2]; std::memcpy( l_v, l_p, 8 ); val[l_i] = { l_v[0], l_v[1] }; break; }
        case Elem::C128: { double l_v[2]; std::memcpy( l_v, l_p, 16 ); val[l_i] = { l_v[0], l_v[1] }; break; }
      }
    }
  }
};

inline HostData make_data( Elem i_elem, int64_t i_n, Fill i_fill, Rng & io_rng ) {
  HostData l_d( i_elem, i_n );
  for( int64_t l_i = 0; l_i < i_n; l_i++ ) {
    double l_re = 1.0, l_im = 0.0;
    if( i_fill == Fill::UNIFORM ) {
      l_re = io_rng.uniform();
      if( is_complex( i_elem ) ) l_im = io_rng.uniform();
    }
    else if( i_fill == Fill::NORMAL ) {
      l_re = io_rng.normal();
      if( is_complex( i_elem ) ) l_im = io_rng.normal();
    }
    l_d.set( l_i, l_re, l_im );
  }
  return l_d;
}

// ---------------------------------------------------------------------------
// device buffers and timing
// ---------------------------------------------------------------------------

inline void check_hip( int i_code, char const * i_what ) {
  if( i_code != 0 ) {
    throw std::runtime_error( std::string( i_what ) + " failed: " + etir_hip_last_error() );
  }
}

class DeviceBuffer {
  void * m_ptr = nullptr;
  int64_t m_bytes = 0;
 public:
  explicit DeviceBuffer( int64_t i_bytes ) : m_bytes( i_bytes ) {
    check_hip( etir_hip_malloc( &m_ptr, std::max< int64_t >( i_bytes, 1 ) ), "etir_hip_malloc" );
  }
  DeviceBuffer( DeviceBuffer const & ) = delete;
  DeviceBuffer & operator=( DeviceBuffer const & ) = delete;
  DeviceBuffer( DeviceBuffer && io_o ) noexcept : m_ptr( io_o.m_ptr ), m_bytes( io_o.m_bytes ) { io_o.m_ptr = nullptr; }
  ~DeviceBuffer() { if( m_ptr != nullptr ) etir_hip_free( m_ptr ); }
  void * ptr() const { return m_ptr; }
  void upload( HostData const & i_d ) {
    check_hip( etir_hip_memcpy_h2d( m_ptr, i_d.raw.data(), i_d.bytes() ), "etir_hip_memcpy_h2d" );
  }
  void download( HostData & io_d ) const {
    check_hip( etir_hip_memcpy_d2h( io_d.raw.data(), m_ptr, io_d.bytes() ), "etir_hip_memcpy_d2h" );
    io_d.decode();
  }
};

inline double seconds_since( std::chrono::steady_clock::time_point i_t0 ) {
  return std::chrono::duration< double >( std::chrono::steady_clock::now() - i_t0 ).count();
}

//! Seconds per call: one warm-up call, then rounds of 1, 2, 4, ... calls
//! (each round closed by i_wait) until the rounds add up to i_min_seconds.
template< class Call, class Wait >
double time_per_call( Call i_call, Wait i_wait, double i_min_seconds = 0.2 ) {
  i_call();
  i_wait();
  int64_t l_calls = 0, l_round = 1;
  double l_total = 0;
  while( l_total < i_min_seconds ) {
    auto l_t0 = std::chrono::steady_clock::now();
    for( int64_t l_i = 0; l_i < l_round; l_i++ ) i_call();
    i_wait();
    l_total += seconds_since( l_t0 );
    l_calls += l_round;
    l_round *= 2;
  }
  return l_total / double( l_calls );
}

// ---------------------------------------------------------------------------
// float64 host evaluation
// ---------------------------------------------------------------------------
typedef std::complex< double > cplx;
typedef std::map< int64_t, int64_t > SizeMap;
//! kept index values of restricted dims
typedef std::map< int64_t, std::vector< int64_t > > Keep;

//! row-major tensor over dim ids (first dim slowest)
struct HostTensor {
  std::vector< int64_t > dims;
  std::vector< cplx > v;
};

inline int64_t extent( SizeMap const & i_sizes, Keep const & i_keep, int64_t i_dim ) {
  auto l_k = i_keep.find( i_dim );
  return l_k != i_keep.end() ? int64_t( l_k->second.size() ) : i_sizes.at( i_dim );
}

//! the entries of a full tensor (dims, full sizes) that lie on the kept grid
inline HostTensor restrict_tensor( std::vector< int64_t > const & i_dims,
                                   std::vector< cplx > const & i_full,
                                   SizeMap const & i_sizes,
                                   Keep const & i_keep ) {
  HostTensor l_t;
  l_t.dims = i_dims;
  std::size_t const l_n = i_dims.size();
  std::vector< int64_t > l_full_stride( l_n ), l_ext( l_n );
  int64_t l_total = 1;
  for( std::size_t l_d = l_n; l_d-- > 0; ) {
    l_full_stride[l_d] = ( l_d + 1 < l_n ) ? l_full_stride[l_d + 1] * i_sizes.at( i_dims[l_d + 1] ) : 1;
    l_ext[l_d] = extent( i_sizes, i_keep, i_dims[l_d] );
    l_total *= l_ext[l_d];
  }
  l_t.v.resize( std::size_t( l_total ) );
  std::vector< int64_t > l_idx( l_n, 0 );
  for( int64_t l_e = 0; l_e < l_total; l_e++ ) {
    int64_t l_off = 0;
    for( std::size_t l_d = 0; l_d < l_n; l_d++ ) {
      auto l_k = i_keep.find( i_dims[l_d] );
      int64_t const l_i = ( l_k != i_keep.end() ) ? l_k->second[l_idx[l_d]] : l_idx[l_d];
      l_off += l_i * l_full_stride[l_d];
    }
    l_t.v[l_e] = i_full[l_off];
    for( std::size_t l_d = l_n; l_d-- > 0; ) {
      if( ++l_idx[l_d] < l_ext[l_d] ) break;
      l_idx[l_d] = 0;
    }
  }
  return l_t;
}

//! multiply-adds of one pairwise contraction (product over the dims involved)
inline double pair_cost( std::vector< int64_t > const & i_a,
                         std::vector< int64_t > const & i_b,
                         std::vector< int64_t > const & i_out,
                         SizeMap const & i_sizes, Keep const & i_keep ) {
  std::set< int64_t > l_all( i_a.begin(), i_a.end() );
  l_all.insert( i_b.begin(), i_b.end() );
  l_all.insert( i_out.begin(), i_out.end() );
  double l_c = 1;
  for( int64_t l_d : l_all ) l_c *= double( extent( i_sizes, i_keep, l_d ) );
  return l_c;
}

//! out[i_out] = sum over the other dims of a and b of a * b (b may be the
//! scalar 1: dims {} and one value), in float64 / complex<double>
inline HostTensor host_contract( HostTensor const & i_a,
                                 HostTensor const & i_b,
                                 std::vector< int64_t > const & i_out,
                                 SizeMap const & i_sizes, Keep const & i_keep ) {
  auto strides_of = [&]( std::vector< int64_t > const & i_dims ) {
    std::map< int64_t, int64_t > l_s;
    int64_t l_st = 1;
    for( std::size_t l_d = i_dims.size(); l_d-- > 0; ) {
      l_s[i_dims[l_d]] += l_st;   // a repeated dim adds its strides (diagonal)
      l_st *= extent( i_sizes, i_keep, i_dims[l_d] );
    }
    return l_s;
  };
  std::map< int64_t, int64_t > const l_sa = strides_of( i_a.dims ), l_sb = strides_of( i_b.dims );
  auto get = []( std::map< int64_t, int64_t > const & i_m, int64_t i_d ) {
    auto l_it = i_m.find( i_d );
    return l_it == i_m.end() ? int64_t( 0 ) : l_it->second;
  };
  // summed dims: in a or b, not in the output
  std::vector< int64_t > l_sum;
  for( auto const * l_dims : { &i_a.dims, &i_b.dims } ) {
    for( int64_t l_d : *l_dims ) {
      if(    std::find( i_out.begin(), i_out.end(), l_d ) == i_out.end()
          && std::find( l_sum.begin(), l_sum.end(), l_d ) == l_sum.end() ) l_sum.push_back( l_d );
    }
  }
  std::size_t const l_no = i_out.size(), l_ns = l_sum.size();
  std::vector< int64_t > l_oe( l_no ), l_oa( l_no ), l_ob( l_no ), l_se( l_ns ), l_sa_( l_ns ), l_sb_( l_ns );
  int64_t l_n_out = 1, l_n_sum = 1;
  for( std::size_t l_d = 0; l_d < l_no; l_d++ ) {
    l_oe[l_d] = extent( i_sizes, i_keep, i_out[l_d] );
    l_oa[l_d] = get( l_sa, i_out[l_d] );
    l_ob[l_d] = get( l_sb, i_out[l_d] );
    l_n_out *= l_oe[l_d];
  }
  for( std::size_t l_d = 0; l_d < l_ns; l_d++ ) {
    l_se[l_d] = extent( i_sizes, i_keep, l_sum[l_d] );
    l_sa_[l_d] = get( l_sa, l_sum[l_d] );
    l_sb_[l_d] = get( l_sb, l_sum[l_d] );
    l_n_sum *= l_se[l_d];
  }
  // the innermost summed dim runs as a plain loop
  int64_t const l_in_e  = l_ns ? l_se[l_ns - 1] : 1;
  int64_t const l_in_sa = l_ns ? l_sa_[l_ns - 1] : 0;
  int64_t const l_in_sb = l_ns ? l_sb_[l_ns - 1] : 0;
  int64_t const l_n_outer_sum = l_n_sum / std::max< int64_t >( l_in_e, 1 );

  HostTensor l_r;
  l_r.dims = i_out;
  l_r.v.assign( std::size_t( l_n_out ), cplx( 0, 0 ) );
  std::vector< int64_t > l_oi( l_no, 0 ), l_si( l_ns, 0 );
  for( int64_t l_o = 0; l_o < l_n_out; l_o++ ) {
    int64_t l_base_a = 0, l_base_b = 0;
    for( std::size_t l_d = 0; l_d < l_no; l_d++ ) {
      l_base_a += l_oi[l_d] * l_oa[l_d];
      l_base_b += l_oi[l_d] * l_ob[l_d];
    }
    cplx l_acc( 0, 0 );
    std::fill( l_si.begin(), l_si.end(), 0 );
    for( int64_t l_s = 0; l_s < l_n_outer_sum; l_s++ ) {
      int64_t l_pa = l_base_a, l_pb = l_base_b;
      for( std::size_t l_d = 0; l_d + 1 < l_ns; l_d++ ) {
        l_pa += l_si[l_d] * l_sa_[l_d];
        l_pb += l_si[l_d] * l_sb_[l_d];
      }
      for( int64_t l_i = 0; l_i < l_in_e; l_i++ ) {
        l_acc += i_a.v[l_pa + l_i * l_in_sa] * i_b.v[l_pb + l_i * l_in_sb];
      }
      // odometer over the summed dims but the innermost
      for( std::size_t l_d = ( l_ns > 0 ? l_ns - 1 : 0 ); l_d-- > 0; ) {
        if( ++l_si[l_d] < l_se[l_d] ) break;
        l_si[l_d] = 0;
      }
    }
    l_r.v[l_o] = l_acc;
    for( std::size_t l_d = l_no; l_d-- > 0; ) {
      if( ++l_oi[l_d] < l_oe[l_d] ) break;
      l_oi[l_d] = 0;
    }
  }
  return l_r;
}

inline HostTensor scalar_one() {
  HostTensor l_t;
  l_t.v.assign( 1, cplx( 1, 0 ) );
  return l_t;
}

//! One pairwise step of a host evaluation: operands by index into the list of
//! tensors, result dims.
struct Step {
  int64_t a, b;                  // b < 0: unary step (permute / sum of a)
  std::vector< int64_t > out;
};

//! Multiply-adds of all steps under a restriction.
inline double steps_cost( std::vector< std::vector< int64_t > > const & i_dims,
                          std::vector< Step > const & i_steps,
                          SizeMap const & i_sizes, Keep const & i_keep ) {
  std::vector< std::vector< int64_t > > l_dims = i_dims;
  double l_c = 0;
  for( Step const & l_s : i_steps ) {
    static std::vector< int64_t > const l_none;
    l_c += pair_cost( l_dims[l_s.a], l_s.b >= 0 ? l_dims[l_s.b] : l_none, l_s.out, i_sizes, i_keep );
    l_dims.push_back( l_s.out );
  }
  return l_c;
}

//! Steps of a contraction path in opt_einsum's standard form (flat pairs of
//! positions in the list of live tensors; both operands leave the list and
//! the result is appended).  A result keeps, in order of first appearance in
//! its operands, the dims that a live tensor or the output still has; the
//! last result has the output's dims in the output's order.
inline std::vector< Step > path_steps( std::vector< std::vector< int64_t > > const & i_in_dims,
                                       std::vector< int64_t > const & i_out_dims,
                                       std::vector< int64_t > const & i_path ) {
  std::vector< std::vector< int64_t > > l_all = i_in_dims;
  std::vector< int64_t > l_live;
  for( std::size_t l_te = 0; l_te < i_in_dims.size(); l_te++ ) l_live.push_back( (int64_t) l_te );
  if( i_path.size() % 2 != 0 || i_path.size() / 2 + 1 != i_in_dims.size() ) {
    throw std::runtime_error( "the path has " + std::to_string( i_path.size() / 2 ) + " contractions for "
                              + std::to_string( i_in_dims.size() ) + " input tensors" );
  }
  std::vector< Step > l_steps;
  for( std::size_t l_p = 0; l_p < i_path.size(); l_p += 2 ) {
    int64_t const l_i = i_path[l_p], l_j = i_path[l_p + 1];
    if( l_i == l_j || l_i < 0 || l_j < 0 || l_i >= (int64_t) l_live.size() || l_j >= (int64_t) l_live.size() ) {
      throw std::runtime_error( "invalid contraction path entry (" + std::to_string( l_i ) + ","
                                + std::to_string( l_j ) + ")" );
    }
    int64_t const l_a = l_live[l_i], l_b = l_live[l_j];
    l_live.erase( l_live.begin() + std::max( l_i, l_j ) );
    l_live.erase( l_live.begin() + std::min( l_i, l_j ) );
    std::vector< int64_t > l_res;
    if( l_live.empty() ) {
      l_res = i_out_dims;
    }
    else {
      std::set< int64_t > l_needed( i_out_dims.begin(), i_out_dims.end() );
      for( int64_t l_t : l_live ) l_needed.insert( l_all[l_t].begin(), l_all[l_t].end() );
      for( int64_t l_src : { l_a, l_b } ) {
        for( int64_t l_d : l_all[l_src] ) {
          if( l_needed.count( l_d ) && std::find( l_res.begin(), l_res.end(), l_d ) == l_res.end() ) l_res.push_back( l_d );
        }
      }
    }
    l_steps.push_back( { l_a, l_b, l_res } );
    l_live.push_back( (int64_t) l_all.size() );
    l_all.push_back( l_res );
  }
  return l_steps;
}

constexpr double kHostBudget = 4.0e8;

//! Restricts output dims (largest first, repeatedly) until the steps cost at
//! most i_budget multiply-adds or no output dim can shrink further.
inline Keep choose_keep( std::vector< std::vector< int64_t > > const & i_dims,
                         std::vector< Step > const & i_steps,
                         std::vector< int64_t > const & i_out_dims,
                         SizeMap const & i_sizes,
                         double i_budget = kHostBudget ) {
  Keep l_keep;
  for( int l_iter = 0; l_iter < 64; l_iter++ ) {
    double const l_cost = steps_cost( i_dims, i_steps, i_sizes, l_keep );
    if( l_cost <= i_budget ) break;
    int64_t l_pick = -1;
    for( int64_t l_d : i_out_dims ) {
      if( extent( i_sizes, l_keep, l_d ) > 1
          && ( l_pick < 0 || extent( i_sizes, l_keep, l_d ) > extent( i_sizes, l_keep, l_pick ) ) ) l_pick = l_d;
    }
    if( l_pick < 0 ) break;
    int64_t const l_size = i_sizes.at( l_pick );
    int64_t const l_cur = extent( i_sizes, l_keep, l_pick );
    int64_t const l_new = std::max< int64_t >( 1, int64_t( std::ceil( l_cur * i_budget / l_cost ) ) );
    int64_t const l_k = std::min( l_new, l_cur - 1 );
    std::vector< int64_t > l_vals;
    if( l_k == 1 ) l_vals.push_back( l_size - 1 );
    for( int64_t l_j = 0; l_k > 1 && l_j < l_k; l_j++ ) l_vals.push_back( l_j * ( l_size - 1 ) / ( l_k - 1 ) );
    l_keep[l_pick] = l_vals;
  }
  return l_keep;
}

//! Evaluates the steps on restricted inputs; returns the last step's tensor.
inline HostTensor run_steps( std::vector< HostTensor > io_tensors,
                             std::vector< Step > const & i_steps,
                             SizeMap const & i_sizes, Keep const & i_keep ) {
  HostTensor const l_one = scalar_one();
  for( Step const & l_s : i_steps ) {
    HostTensor const & l_b = l_s.b >= 0 ? io_tensors[l_s.b] : l_one;
    io_tensors.push_back( host_contract( io_tensors[l_s.a], l_b, l_s.out, i_sizes, i_keep ) );
  }
  return io_tensors.back();
}

//! Relative Frobenius error of the device result against the host result
//! (both over the same entries), with the figures the harnesses print.
struct Comparison {
  int64_t entries = 0;
  double max_ref = 0, max_got = 0, max_diff = 0;
  double frob_ref = 0, frob_got = 0, frob_diff = 0, rel = 0;
};

inline Comparison compare( std::vector< cplx > const & i_ref, std::vector< cplx > const & i_got ) {
  Comparison l_c;
  l_c.entries = int64_t( i_ref.size() );
  for( std::size_t l_i = 0; l_i < i_ref.size(); l_i++ ) {
    double const l_r = std::abs( i_ref[l_i] ), l_g = std::abs( i_got[l_i] ), l_d = std::abs( i_ref[l_i] - i_got[l_i] );
    l_c.max_ref = std::max( l_c.max_ref, l_r );
    l_c.max_got = std::max( l_c.max_got, l_g );
    // NaN differences count as infinitely large
    l_c.max_diff = ( l_d == l_d ) ? std::max( l_c.max_diff, l_d ) : INFINITY;
    l_c.frob_ref += l_r * l_r;
    l_c.frob_got += l_g * l_g;
    l_c.frob_diff += ( l_d == l_d ) ? l_d * l_d : INFINITY;
  }
  l_c.frob_ref = std::sqrt( l_c.frob_ref );
  l_c.frob_got = std::sqrt( l_c.frob_got );
  l_c.frob_diff = std::sqrt( l_c.frob_diff );
  l_c.rel = l_c.frob_ref > 0 ? l_c.frob_diff / l_c.frob_ref : l_c.frob_diff;
  return l_c;
}

//! the device output's entries on the kept grid
inline std::vector< cplx > restricted_output( HostData const & i_out,
                                              std::vector< int64_t > const & i_dims,
                                              SizeMap const & i_sizes, Keep const & i_keep ) {
  return restrict_tensor( i_dims, i_out.val, i_sizes, i_keep ).v;
}

//! "dims 3 (64 of 512), 0 (all)": what the check covered
inline std::string describe_keep( Keep const & i_keep, SizeMap const & i_sizes,
                                  std::map< int64_t, std::string > const & i_names ) {
  if( i_keep.empty() ) return "all output entries";
  std::ostringstream l_s;
  l_s << "output dims restricted to";
  for( auto const & l_k : i_keep ) {
    auto l_n = i_names.find( l_k.first );
    l_s << " " << ( l_n != i_names.end() ? l_n->second : std::to_string( l_k.first ) )
        << " (" << l_k.second.size() << " of " << i_sizes.at( l_k.first ) << " values)";
  }
  return l_s.str();
}

//! Prints the comparison block; true when the relative error is within tol.
inline bool report( Comparison const & i_c, double i_tol, std::string const & i_coverage ) {
  std::cout << "\n*** comparing solution ***:" << std::endl;
  std::cout << "  reference: float64 on the host, " << i_coverage << " (" << i_c.entries << " entries)" << std::endl;
  std::cout << "  maximum absolute entry in host solution:      " << i_c.max_ref << std::endl;
  std::cout << "  maximum absolute entry in einsum_ir solution: " << i_c.max_got << std::endl;
  std::cout << "  maximum element-wise difference:              " << i_c.max_diff << std::endl;
  std::cout << "  frobenius norm of host solution:              " << i_c.frob_ref << std::endl;
  std::cout << "  frobenius norm of einsum_ir solution:         " << i_c.frob_got << std::endl;
  std::cout << "  frobenius norm of difference:                 " << i_c.frob_diff << std::endl;
  std::cout << "  relative error:                               " << i_c.rel << std::endl;
  bool const l_ok = i_c.rel <= i_tol;
  if( l_ok ) std::cout << "  results are close (tolerance " << i_tol << ")" << std::endl;
  else std::cerr << "error: relative error " << i_c.rel << " above tolerance " << i_tol << std::endl;
  return l_ok;
}

//! relative Frobenius tolerance by compute type: fp32 1e-5, fp64 1e-12,
//! bf16 inputs with fp32 accumulation 2e-3
inline double tolerance( Elem i_in ) {
  switch( i_in ) {
    case Elem::F64: case Elem::C128: return 1e-12;
    case Elem::BF16: return 2e-3;
    default: return 1e-5;
  }
}

} // namespace etir_bench

#endif
