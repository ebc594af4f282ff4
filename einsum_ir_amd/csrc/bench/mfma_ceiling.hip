// Sustained matrix-core rate and shader clock of this GPU.
//
// Two workgroups of four waves per CU run nothing but independent MFMAs
// (four accumulators per wave) for about 30-200 ms; every wave reads the
// shader clock (s_memtime) and the 100 MHz constant clock (s_memrealtime) at
// its start and end.  Printed per case, one JSON line each: TFLOP/s from HIP
// events, the fraction of the published dense peak, and the median clock of
// the waves.  Operands are either constant (little switching activity) or 16
// random values per lane and operand, cycled through the MFMAs (switching
// like real data): the second case shows the power-limited clock the
// contraction kernels can expect.
//
//   usage: mfma_ceiling        (no arguments; about one second of GPU time)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef float  f32x16 __attribute__( ( ext_vector_type( 16 ) ) );
typedef __bf16 bf16x8 __attribute__( ( ext_vector_type( 8 ) ) );

constexpr int kThreads = 256;

#define CHECK( x )                                                                  \
  do {                                                                              \
    hipError_t l_e = ( x );                                                         \
    if( l_e != hipSuccess ) {                                                       \
      std::fprintf( stderr, "%s: %s\n", #x, hipGetErrorString( l_e ) );             \
      std::exit( 1 );                                                               \
    }                                                                               \
  } while( 0 )

// KIND 0: v_mfma_f32_32x32x2_f32, KIND 1: v_mfma_f32_32x32x16_bf16
template< int KIND, bool RANDOM >
__global__ __launch_bounds__( kThreads ) void spin( float * out, unsigned long long * clocks, int iters ) {
  uint32_t l_x = 2463534242u ^ ( ( blockIdx.x * kThreads + threadIdx.x ) * 2654435761u );
  auto l_rnd = [&]() {
    l_x ^= l_x << 13;
    l_x ^= l_x >> 17;
    l_x ^= l_x << 5;
    return float( l_x & 0xffffffu ) / 8388608.0f - 1.0f;
  };
  float  l_a[16], l_b[16];
  bf16x8 l_ha[4], l_hb[4];
  for( int l_e = 0; l_e < 16; l_e++ ) {
    l_a[l_e] = RANDOM ? l_rnd() : 1e-7f * threadIdx.x;
    l_b[l_e] = RANDOM ? l_rnd() : 1e-7f;
  }
  for( int l_q = 0; l_q < 4; l_q++ )
    for( int l_e = 0; l_e < 8; l_e++ ) {
      l_ha[l_q][l_e] = __bf16( RANDOM ? l_rnd() : 1e-3f );
      l_hb[l_q][l_e] = __bf16( RANDOM ? l_rnd() : 1e-3f );
    }
  f32x16 l_acc[4];
  for( int l_j = 0; l_j < 4; l_j++ ) l_acc[l_j] = f32x16( 0.0f );
  __syncthreads();

  unsigned long long const l_c0 = clock64();
  unsigned long long const l_w0 = wall_clock64();
  for( int l_it = 0; l_it < iters; l_it++ ) {
#pragma unroll
    for( int l_r = 0; l_r < 4; l_r++ )
#pragma unroll
      for( int l_j = 0; l_j < 4; l_j++ ) {
        if constexpr( KIND == 0 )
          l_acc[l_j] = __builtin_amdgcn_mfma_f32_32x32x2f32( l_a[l_r * 4 + l_j], l_b[( l_r * 4 + l_j + 5 ) & 15],
                                                             l_acc[l_j], 0, 0, 0 );
        else
          l_acc[l_j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16( l_ha[l_r], l_hb[( l_r + l_j ) & 3],
                                                                l_acc[l_j], 0, 0, 0 );
      }
  }
  unsigned long long const l_c1 = clock64();
  unsigned long long const l_w1 = wall_clock64();

  float l_s = 0.0f;
  for( int l_j = 0; l_j < 4; l_j++ )
    for( int l_e = 0; l_e < 16; l_e++ ) l_s += l_acc[l_j][l_e];
  out[blockIdx.x * kThreads + threadIdx.x] = l_s;
  if( ( threadIdx.x & 63 ) == 0 ) {
    size_t const l_w = size_t( blockIdx.x ) * ( kThreads / 64 ) + threadIdx.x / 64;
    clocks[4 * l_w + 0] = l_c0;
    clocks[4 * l_w + 1] = l_c1;
    clocks[4 * l_w + 2] = l_w0;
    clocks[4 * l_w + 3] = l_w1;
  }
}

template< int KIND, bool RANDOM >
void run( int cus, int wall_khz ) {
  int const    l_blocks = 2 * cus;
  int const    l_waves  = l_blocks * ( kThreads / 64 );
  // about 35 ms per launch at the published peak
  int const    l_iters  = KIND == 0 ? 40000 : 80000;
  double const l_flop_per_mfma = KIND == 0 ? 32.0 * 32 * 2 * 2 : 32.0 * 32 * 16 * 2;
  double const l_peak = KIND == 0 ? 157.3 : 2516.6;   // TFLOP/s, dense, published

  float * l_out = nullptr;
  unsigned long long * l_clk = nullptr;
  CHECK( hipMalloc( &l_out, size_t( l_blocks ) * kThreads * sizeof( float ) ) );
  CHECK( hipMalloc( &l_clk, size_t( l_waves ) * 4 * sizeof( unsigned long long ) ) );
  hipEvent_t l_e0, l_e1;
  CHECK( hipEventCreate( &l_e0 ) );
  CHECK( hipEventCreate( &l_e1 ) );

  spin< KIND, RANDOM ><<< l_blocks, kThreads >>>( l_out, l_clk, l_iters / 8 );
  CHECK( hipGetLastError() );
  CHECK( hipDeviceSynchronize() );
  float l_best = 1e30f;
  std::vector< unsigned long long > l_h( size_t( l_waves ) * 4 );
  for( int l_rep = 0; l_rep < 3; l_rep++ ) {
    CHECK( hipEventRecord( l_e0 ) );
    spin< KIND, RANDOM ><<< l_blocks, kThreads >>>( l_out, l_clk, l_iters );
    CHECK( hipGetLastError() );
    CHECK( hipEventRecord( l_e1 ) );
    CHECK( hipEventSynchronize( l_e1 ) );
    float l_ms = 0.0f;
    CHECK( hipEventElapsedTime( &l_ms, l_e0, l_e1 ) );
    if( l_ms < l_best ) {
      l_best = l_ms;
      CHECK( hipMemcpy( l_h.data(), l_clk, l_h.size() * sizeof( unsigned long long ), hipMemcpyDeviceToHost ) );
    }
  }
  double const l_tflops = double( l_waves ) * l_iters * 16 * l_flop_per_mfma / ( l_best * 1e-3 ) * 1e-12;
  std::vector< double > l_ghz;
  for( int l_w = 0; l_w < l_waves; l_w++ ) {
    double const l_dc = double( l_h[4 * l_w + 1] - l_h[4 * l_w + 0] );
    double const l_dw = double( l_h[4 * l_w + 3] - l_h[4 * l_w + 2] );
    if( l_dw > 0 ) l_ghz.push_back( l_dc / ( l_dw / ( wall_khz * 1e3 ) ) * 1e-9 );
  }
  std::sort( l_ghz.begin(), l_ghz.end() );
  double const l_med = l_ghz.empty() ? 0.0 : l_ghz[l_ghz.size() / 2];
  std::printf( "{\"mfma\": \"%s\", \"operands\": \"%s\", \"workgroups\": %d, \"ms\": %.3f, \"tflops\": %.1f, "
               "\"frac_peak\": %.4f, \"peak_tflops\": %.1f, \"clock_ghz_median\": %.3f, \"clock_ghz_min\": %.3f}\n",
               KIND == 0 ? "f32_32x32x2" : "bf16_32x32x16", RANDOM ? "random" : "constant", l_blocks, l_best,
               l_tflops, l_tflops / l_peak, l_peak, l_med, l_ghz.empty() ? 0.0 : l_ghz.front() );
  std::fflush( stdout );
  CHECK( hipEventDestroy( l_e0 ) );
  CHECK( hipEventDestroy( l_e1 ) );
  CHECK( hipFree( l_out ) );
  CHECK( hipFree( l_clk ) );
}

}  // namespace

int main() {
  int l_wall_khz = 0, l_cus = 0;
  CHECK( hipDeviceGetAttribute( &l_wall_khz, hipDeviceAttributeWallClockRate, 0 ) );
  CHECK( hipDeviceGetAttribute( &l_cus, hipDeviceAttributeMultiprocessorCount, 0 ) );
  if( l_wall_khz <= 0 || l_cus <= 0 ) {
    std::fprintf( stderr, "mfma_ceiling: device attributes unavailable\n" );
    return 1;
  }
  run< 0, false >( l_cus, l_wall_khz );
  run< 0, true >( l_cus, l_wall_khz );
  run< 1, false >( l_cus, l_wall_khz );
  run< 1, true >( l_cus, l_wall_khz );
  return 0;
}
