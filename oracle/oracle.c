/*
 * oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the numerics of einsum_ir's binary-contraction and
 * permutation path, used as the checker by tests/, by __graft_entry__.smoke()
 * and as the timed CPU baseline in bench.py.  Nothing in the product
 * (einsum_ir_amd/, include/) links, loads or calls this file.
 *
 * Functions and the reference behaviour they restate:
 *
 *  oracle_contract         Exact (fp64-accumulating) contraction over the loop IR.
 *                          Loop IR = reference basic::iter_property
 *                          (src/basic/constants.h:85-95) as produced by
 *                          BinaryContractionTpp::compile (src/backend/BinaryContractionTpp.cpp:46-66,
 *                          which lowers only C/M/N/K loops: I/J loops are not iterated).
 *                          Touch semantics per output element follow
 *                          ContractionBackend::contract_iter / contract_iter_kernel
 *                          (src/basic/binary/ContractionBackend.cpp:296-348, 495-515) and the TPP
 *                          element-wise kernels (src/basic/binary/ContractionBackendTpp.cpp:15-49,
 *                          127-163): first touch ZERO -> 0, COPY -> aux, ADD -> out + aux,
 *                          (none) -> out; main MADD accumulates; last touch RELU -> max(.,0),
 *                          ADD -> + aux.
 *                          Pinned by tests/test_oracle.py: numpy.einsum in float64 on random
 *                          layouts (incl. strided/broadcast aux and skipped I/J loops),
 *                          right = ones -> row sums, identity operands, closed forms of every
 *                          touch kernel, brute-force 1x1x1 cases.
 *
 *  oracle_contract_blocked The CPU baseline: the reference's CPU algorithm restated -- loops
 *                          of a type fused into one index (ContractionOptimizer::sort_and_fuse_iters,
 *                          src/basic/binary/ContractionOptimizer.cpp:76-111), outer C/M/N blocks run
 *                          as OpenMP tasks (execute_threaded, src/basic/threading.h:60-104), each
 *                          task packs its operand blocks (ContractionBackend::create_packing,
 *                          ContractionBackend.cpp:680-737) and runs an fp32 blocked GEMM
 *                          microkernel with the first/last touch applied around the K loop.
 *                          Pinned by tests/test_oracle.py against oracle_contract.
 *
 *  oracle_permute          Permutation with COPY / ZERO / ADD: Unary::compile_base derives the
 *                          input strides in output-dimension order (src/backend/Unary.cpp:82-113);
 *                          UnaryBackendTpp applies IDENTITY/TRANSPOSE copy, XOR zero, or ADD
 *                          (src/basic/unary/UnaryBackendTpp.cpp:14-29, 77-96).
 *                          Pinned by tests/test_oracle.py: numpy.transpose bit-exact, zero fill,
 *                          addition.
 *
 *  oracle_permute_blocked  The permutation CPU baseline: the reference's sequential unary loop nest
 *                          around a 2-D transpose primitive (UnaryBackend.cpp:106-226,
 *                          UnaryBackendTpp.cpp:45-93) with a 64 x 64 blocked transpose.  Pinned by
 *                          tests/test_oracle.py against oracle_permute (bit-exact).
 *
 *  oracle_f32_to_bf16 /    bf16 round-to-nearest-even / widening, from the IEEE-754 binary32 and
 *  oracle_bf16_to_f32      bfloat16 definitions (the reference has no bf16).  Pinned by
 *                          tests/test_oracle.py against hand-computed tie cases and torch.bfloat16.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_FP32 0
#define OR_FP64 1
#define OR_BF16 2

#define OR_ZERO 0
#define OR_RELU 1
#define OR_ADD 2
#define OR_COPY 3
#define OR_MADD 4
#define OR_UNDEF 99

#define OR_DIM_C 0
#define OR_DIM_M 1
#define OR_DIM_N 2
#define OR_DIM_K 3

#define OR_MAX_LOOPS 64

/* ------------------------------------------------------------------ bf16 */
static uint16_t f32_to_bf16_one( float f ) {
  uint32_t u;
  memcpy( &u, &f, 4 );
  if( ( u & 0x7f800000u ) == 0x7f800000u && ( u & 0x007fffffu ) ) {
    return (uint16_t) ( ( u >> 16 ) | 0x40u );   /* quiet NaN */
  }
  uint32_t lsb = ( u >> 16 ) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t) ( u >> 16 );
}

static float bf16_to_f32_one( uint16_t b ) {
  uint32_t u = ( (uint32_t) b ) << 16;
  float f;
  memcpy( &f, &u, 4 );
  return f;
}

void oracle_f32_to_bf16( float const * in, uint16_t * out, int64_t n ) {
  for( int64_t i = 0; i < n; i++ ) out[i] = f32_to_bf16_one( in[i] );
}

void oracle_bf16_to_f32( uint16_t const * in, float * out, int64_t n ) {
  for( int64_t i = 0; i < n; i++ ) out[i] = bf16_to_f32_one( in[i] );
}

static double load_as_f64( void const * p, int64_t off, int32_t dt ) {
  if( dt == OR_FP32 ) return (double) ( (float const *) p )[off];
  if( dt == OR_FP64 ) return ( (double const *) p )[off];
  return (double) bf16_to_f32_one( ( (uint16_t const *) p )[off] );
}

static void store_from_f64( void * p, int64_t off, int32_t dt, double v ) {
  if( dt == OR_FP32 )      ( (float *) p )[off] = (float) v;
  else if( dt == OR_FP64 ) ( (double *) p )[off] = v;
  else                     ( (uint16_t *) p )[off] = f32_to_bf16_one( (float) v );
}

/* --------------------------------------------------------- contraction */
int oracle_contract( int64_t         num_loops,
                     int32_t const * types,
                     int64_t const * sizes,
                     int64_t const * s_left,
                     int64_t const * s_right,
                     int64_t const * s_aux,
                     int64_t const * s_out,
                     int32_t         dt_left,
                     int32_t         dt_right,
                     int32_t         dt_out,
                     int32_t         first_touch,
                     int32_t         last_touch,
                     void const    * left,
                     void const    * right,
                     void const    * aux,
                     void          * out ) {
  int64_t o_size[OR_MAX_LOOPS], o_sl[OR_MAX_LOOPS], o_sr[OR_MAX_LOOPS], o_sa[OR_MAX_LOOPS], o_so[OR_MAX_LOOPS];
  int64_t k_size[OR_MAX_LOOPS], k_sl[OR_MAX_LOOPS], k_sr[OR_MAX_LOOPS];
  int no = 0, nk = 0;
  if( num_loops > OR_MAX_LOOPS ) return 1;
  for( int64_t l = 0; l < num_loops; l++ ) {
    if( sizes[l] == 0 ) return 0;
    if( types[l] == OR_DIM_K ) {
      k_size[nk] = sizes[l]; k_sl[nk] = s_left[l]; k_sr[nk] = s_right[l]; nk++;
    }
    else if( types[l] == OR_DIM_C || types[l] == OR_DIM_M || types[l] == OR_DIM_N ) {
      o_size[no] = sizes[l]; o_sl[no] = s_left[l]; o_sr[no] = s_right[l];
      o_sa[no] = s_aux ? s_aux[l] : s_out[l]; o_so[no] = s_out[l]; no++;
    }
    /* I/J loops are not part of the reference's lowered loop nest */
  }
  int64_t oi[OR_MAX_LOOPS], ki[OR_MAX_LOOPS];
  for( int d = 0; d < no; d++ ) oi[d] = 0;
  for( ;; ) {
    int64_t ol = 0, orr = 0, oa = 0, oo = 0;
    for( int d = 0; d < no; d++ ) {
      ol += oi[d] * o_sl[d]; orr += oi[d] * o_sr[d]; oa += oi[d] * o_sa[d]; oo += oi[d] * o_so[d];
    }
    /* reduction over K in fp64 */
    double sum = 0.0;
    for( int d = 0; d < nk; d++ ) ki[d] = 0;
    for( ;; ) {
      int64_t kl = ol, kr = orr;
      for( int d = 0; d < nk; d++ ) { kl += ki[d] * k_sl[d]; kr += ki[d] * k_sr[d]; }
      sum += load_as_f64( left, kl, dt_left ) * load_as_f64( right, kr, dt_right );
      int d = nk - 1;
      while( d >= 0 ) {
        if( ++ki[d] < k_size[d] ) break;
        ki[d] = 0;
        d--;
      }
      if( d < 0 ) break;
    }
    double v;
    double av = 0.0;
    int need_aux = ( first_touch == OR_COPY || first_touch == OR_ADD || last_touch == OR_ADD );
    if( need_aux ) av = load_as_f64( aux, oa, dt_out );
    if(      first_touch == OR_ZERO ) v = sum;
    else if( first_touch == OR_COPY ) v = av + sum;
    else if( first_touch == OR_ADD )  v = load_as_f64( out, oo, dt_out ) + av + sum;
    else                              v = load_as_f64( out, oo, dt_out ) + sum;
    if(      last_touch == OR_RELU ) v = v > 0.0 ? v : 0.0;
    else if( last_touch == OR_ADD )  v = v + av;
    store_from_f64( out, oo, dt_out, v );

    int d = no - 1;
    while( d >= 0 ) {
      if( ++oi[d] < o_size[d] ) break;
      oi[d] = 0;
      d--;
    }
    if( d < 0 ) break;
  }
  return 0;
}

/* ------------------------------------------------- blocked CPU baseline */
typedef struct {
  int64_t size;
  int64_t s[4];  /* left, right, aux, out */
} or_loop;

/* enumerates the mixed-radix offsets of loops (outer -> inner) in slot */
static int64_t * or_table( or_loop const * lo, int n, int slot, int64_t * o_count ) {
  int64_t total = 1;
  for( int d = 0; d < n; d++ ) total *= lo[d].size;
  int64_t * t = (int64_t *) malloc( sizeof( int64_t ) * ( total > 0 ? total : 1 ) );
  t[0] = 0;
  int64_t filled = 1;
  for( int d = n - 1; d >= 0; d-- ) {
    for( int64_t it = 1; it < lo[d].size; it++ )
      for( int64_t e = 0; e < filled; e++ )
        t[it * filled + e] = t[e] + it * lo[d].s[slot];
    filled *= lo[d].size;
  }
  *o_count = total;
  return t;
}

#define OR_MB 64
#define OR_NB 64
#define OR_KB 256

int oracle_contract_blocked( int64_t         num_loops,
                             int32_t const * types,
                             int64_t const * sizes,
                             int64_t const * s_left,
                             int64_t const * s_right,
                             int64_t const * s_aux,
                             int64_t const * s_out,
                             int32_t         first_touch,
                             int32_t         last_touch,
                             float const   * left,
                             float const   * right,
                             float const   * aux,
                             float         * out,
                             int32_t         num_threads ) {
  or_loop lc[OR_MAX_LOOPS], lm[OR_MAX_LOOPS], ln[OR_MAX_LOOPS], lk[OR_MAX_LOOPS];
  int nc = 0, nm = 0, nn = 0, nk = 0;
  if( num_loops > OR_MAX_LOOPS ) return 1;
  for( int64_t l = 0; l < num_loops; l++ ) {
    or_loop x;
    x.size = sizes[l];
    x.s[0] = s_left[l]; x.s[1] = s_right[l]; x.s[2] = s_aux ? s_aux[l] : s_out[l]; x.s[3] = s_out[l];
    if( x.size == 0 ) return 0;
    if( types[l] == OR_DIM_C ) lc[nc++] = x;
    else if( types[l] == OR_DIM_M ) lm[nm++] = x;
    else if( types[l] == OR_DIM_N ) ln[nn++] = x;
    else if( types[l] == OR_DIM_K ) lk[nk++] = x;
  }
  int64_t C, M, N, K, tmp;
  int64_t * tc_l = or_table( lc, nc, 0, &C );
  int64_t * tc_r = or_table( lc, nc, 1, &tmp );
  int64_t * tc_a = or_table( lc, nc, 2, &tmp );
  int64_t * tc_o = or_table( lc, nc, 3, &tmp );
  int64_t * tm_l = or_table( lm, nm, 0, &M );
  int64_t * tm_a = or_table( lm, nm, 2, &tmp );
  int64_t * tm_o = or_table( lm, nm, 3, &tmp );
  int64_t * tn_r = or_table( ln, nn, 1, &N );
  int64_t * tn_a = or_table( ln, nn, 2, &tmp );
  int64_t * tn_o = or_table( ln, nn, 3, &tmp );
  int64_t * tk_l = or_table( lk, nk, 0, &K );
  int64_t * tk_r = or_table( lk, nk, 1, &tmp );

  int64_t const bm = ( M + OR_MB - 1 ) / OR_MB;
  int64_t const bn = ( N + OR_NB - 1 ) / OR_NB;
  int64_t const tasks = C * bm * bn;
  int const need_aux = ( first_touch == OR_COPY || first_touch == OR_ADD || last_touch == OR_ADD );
  (void) num_threads;

#ifdef _OPENMP
  if( num_threads > 0 ) omp_set_num_threads( num_threads );
#pragma omp parallel
#endif
  {
    /* per-thread packing buffers: A block [kb][mb], B block [kb][nb] */
    float * pa = (float *) aligned_alloc( 64, sizeof( float ) * OR_KB * OR_MB );
    float * pb = (float *) aligned_alloc( 64, sizeof( float ) * OR_KB * OR_NB );
    float acc[OR_MB][OR_NB];
#ifdef _OPENMP
#pragma omp for schedule( dynamic, 1 )
#endif
    for( int64_t t = 0; t < tasks; t++ ) {
      int64_t c  = t / ( bm * bn );
      int64_t r  = t % ( bm * bn );
      int64_t m0 = ( r / bn ) * OR_MB;
      int64_t n0 = ( r % bn ) * OR_NB;
      int64_t mc = M - m0 < OR_MB ? M - m0 : OR_MB;
      int64_t ncn = N - n0 < OR_NB ? N - n0 : OR_NB;
      for( int i = 0; i < OR_MB; i++ ) for( int j = 0; j < OR_NB; j++ ) acc[i][j] = 0.0f;
      float const * lb = left + tc_l[c];
      float const * rb = right + tc_r[c];
      for( int64_t k0 = 0; k0 < K; k0 += OR_KB ) {
        int64_t kc = K - k0 < OR_KB ? K - k0 : OR_KB;
        for( int64_t k = 0; k < kc; k++ ) {
          for( int64_t i = 0; i < mc; i++ ) pa[k * OR_MB + i] = lb[tm_l[m0 + i] + tk_l[k0 + k]];
          for( int64_t i = mc; i < OR_MB; i++ ) pa[k * OR_MB + i] = 0.0f;
          for( int64_t j = 0; j < ncn; j++ ) pb[k * OR_NB + j] = rb[tn_r[n0 + j] + tk_r[k0 + k]];
          for( int64_t j = ncn; j < OR_NB; j++ ) pb[k * OR_NB + j] = 0.0f;
        }
        /* microkernel: rank-1 updates, inner loop over n vectorises */
        for( int64_t k = 0; k < kc; k++ ) {
          float const * ak = pa + k * OR_MB;
          float const * bk = pb + k * OR_NB;
          for( int i = 0; i < OR_MB; i++ ) {
            float const av = ak[i];
            for( int j = 0; j < OR_NB; j++ ) acc[i][j] += av * bk[j];
          }
        }
      }
      float * ob = out + tc_o[c];
      float const * xb = aux ? aux + tc_a[c] : 0;
      for( int64_t i = 0; i < mc; i++ ) {
        for( int64_t j = 0; j < ncn; j++ ) {
          int64_t oo = tm_o[m0 + i] + tn_o[n0 + j];
          float xv = 0.0f;
          if( need_aux ) xv = xb[tm_a[m0 + i] + tn_a[n0 + j]];
          float v = acc[i][j];
          if(      first_touch == OR_COPY ) v = xv + v;
          else if( first_touch == OR_ADD )  v = ob[oo] + xv + v;
          else if( first_touch != OR_ZERO ) v = ob[oo] + v;
          if(      last_touch == OR_RELU ) v = v > 0.0f ? v : 0.0f;
          else if( last_touch == OR_ADD )  v = v + xv;
          ob[oo] = v;
        }
      }
    }
    free( pa );
    free( pb );
  }
  free( tc_l ); free( tc_r ); free( tc_a ); free( tc_o );
  free( tm_l ); free( tm_a ); free( tm_o );
  free( tn_r ); free( tn_a ); free( tn_o );
  free( tk_l ); free( tk_r );
  return 0;
}

/* --------------------------------------------------------- permutation */
int oracle_permute( int64_t         num_dims,
                    int64_t const * sizes,
                    int64_t const * s_in,
                    int64_t const * s_out,
                    int32_t         dtype,
                    int32_t         ktype,
                    void const    * in,
                    void          * out,
                    int32_t         num_threads ) {
  int64_t eb = dtype == OR_FP64 ? 8 : ( dtype == OR_FP32 ? 4 : 2 );
  int64_t total = 1;
  if( num_dims > OR_MAX_LOOPS ) return 1;
  for( int64_t d = 0; d < num_dims; d++ ) total *= sizes[d];
  if( total == 0 ) return 0;
  /* parallelise over the outermost dimension */
  int64_t outer = num_dims > 0 ? sizes[0] : 1;
  (void) num_threads;
#ifdef _OPENMP
  if( num_threads > 0 ) omp_set_num_threads( num_threads );
#pragma omp parallel for schedule( static )
#endif
  for( int64_t o = 0; o < outer; o++ ) {
    int64_t idx[OR_MAX_LOOPS];
    for( int64_t d = 0; d < num_dims; d++ ) idx[d] = 0;
    if( num_dims > 0 ) idx[0] = o;
    for( ;; ) {
      int64_t oi = 0, oo = 0;
      for( int64_t d = 0; d < num_dims; d++ ) {
        oi += idx[d] * ( ktype == OR_ZERO ? 0 : s_in[d] );
        oo += idx[d] * s_out[d];
      }
      char * po = (char *) out + oo * eb;
      if( ktype == OR_ZERO ) {
        memset( po, 0, (size_t) eb );
      }
      else if( ktype == OR_COPY ) {
        memcpy( po, (char const *) in + oi * eb, (size_t) eb );
      }
      else {
        if( dtype == OR_FP32 ) ( (float *) out )[oo] += ( (float const *) in )[oi];
        else if( dtype == OR_FP64 ) ( (double *) out )[oo] += ( (double const *) in )[oi];
        else {
          float s = bf16_to_f32_one( ( (uint16_t *) out )[oo] ) + bf16_to_f32_one( ( (uint16_t const *) in )[oi] );
          ( (uint16_t *) out )[oo] = f32_to_bf16_one( s );
        }
      }
      int64_t d = num_dims - 1;
      while( d >= 1 ) {
        if( ++idx[d] < sizes[d] ) break;
        idx[d] = 0;
        d--;
      }
      if( d < 1 ) break;
    }
  }
  return 0;
}

/* The CPU baseline of a permutation: the reference's unary loop nest restated
 * (UnaryBackend::eval / eval_iter, src/basic/unary/UnaryBackend.cpp:106-226:
 * sequential loops, no OpenMP, around a 2-D transpose primitive of the
 * input's and the output's unit-stride dims, UnaryBackendTpp.cpp:45-93) with a
 * 64 x 64 blocked transpose as the primitive.  fp32 COPY; single thread, as
 * the reference runs it.  Pinned by tests/test_oracle.py against
 * oracle_permute (bit-exact).  Returns 2 for layouts it does not cover (no
 * distinct unit-stride dims in input and output). */
int oracle_permute_blocked( int64_t         num_dims,
                            int64_t const * sizes,
                            int64_t const * s_in,
                            int64_t const * s_out,
                            float const   * in,
                            float         * out ) {
  int64_t di = -1, dout = -1;
  if( num_dims > OR_MAX_LOOPS ) return 1;
  for( int64_t d = 0; d < num_dims; d++ ) {
    if( sizes[d] == 0 ) return 0;
    if( s_in[d] == 1 && di < 0 ) di = d;
    if( s_out[d] == 1 && dout < 0 ) dout = d;
  }
  if( di < 0 || dout < 0 || di == dout ) return 2;
  int64_t const ni = sizes[di], no = sizes[dout];
  int64_t const si_o = s_in[dout], so_i = s_out[di];
  /* batch dims: every other dim, outer -> inner */
  int64_t bsz[OR_MAX_LOOPS], bsi[OR_MAX_LOOPS], bso[OR_MAX_LOOPS], idx[OR_MAX_LOOPS];
  int nb = 0;
  for( int64_t d = 0; d < num_dims; d++ ) {
    if( d == di || d == dout ) continue;
    bsz[nb] = sizes[d]; bsi[nb] = s_in[d]; bso[nb] = s_out[d]; idx[nb] = 0; nb++;
  }
  for( ;; ) {
    int64_t bi = 0, bo = 0;
    for( int b = 0; b < nb; b++ ) { bi += idx[b] * bsi[b]; bo += idx[b] * bso[b]; }
    for( int64_t o0 = 0; o0 < no; o0 += 64 ) {
      int64_t const o1 = o0 + 64 < no ? o0 + 64 : no;
      for( int64_t i0 = 0; i0 < ni; i0 += 64 ) {
        int64_t const i1 = i0 + 64 < ni ? i0 + 64 : ni;
        for( int64_t x = i0; x < i1; x++ ) {
          float const * src = in + bi + x;
          float * dst = out + bo + x * so_i;
          for( int64_t y = o0; y < o1; y++ ) dst[y] = src[y * si_o];
        }
      }
    }
    int b = nb - 1;
    while( b >= 0 ) {
      if( ++idx[b] < bsz[b] ) break;
      idx[b] = 0;
      b--;
    }
    if( b < 0 ) break;
  }
  return 0;
}
