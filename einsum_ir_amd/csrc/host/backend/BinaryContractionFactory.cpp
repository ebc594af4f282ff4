#include "BinaryContractionFactory.h"
#include "BinaryContractionHip.h"

bool einsum_ir::backend::BinaryContractionFactory::supports( backend_t i_backend ) {
  return i_backend == backend_t::HIP;
}

einsum_ir::backend::BinaryContraction * einsum_ir::backend::BinaryContractionFactory::create( backend_t i_backend ) {
  if( i_backend == backend_t::HIP ) {
    return new BinaryContractionHip();
  }
  return nullptr;
}
