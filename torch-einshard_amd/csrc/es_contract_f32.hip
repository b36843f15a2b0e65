// es_contract kernel instances for one element type (f32); compiled as a
// separate translation unit so the kernel variants build in parallel.
#include "es_contract_kernel.h"

namespace es {
int launch_contract_f32(const ContractArgs& p, int config, int la, int lb, hipStream_t s) {
  return contract::launch_typed<float>(p, config, la, lb, s);
}
}  // namespace es
