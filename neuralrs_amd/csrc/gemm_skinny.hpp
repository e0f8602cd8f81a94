// Skinny GEMMs (gemm_skinny.hip): at most 32 output rows, B [K][N] streamed
// from HBM straight into registers.
#pragma once

#include "gemm_call.hpp"

namespace nrs {

// Whether c is a dense NN or TN product with 1..32 rows, at least 1024
// columns (whole float4s, B 16-byte aligned) and K >= 256.
bool skinny_eligible(const GemmCall& c);
int skinny_run(const GemmCall& c);

}  // namespace nrs
