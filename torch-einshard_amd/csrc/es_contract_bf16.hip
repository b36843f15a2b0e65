// es_contract kernel instances for one element type (bf16); compiled as a
// separate translation unit so the kernel variants build in parallel.
#include "es_contract_kernel.h"

namespace es {
int launch_contract_bf16(const ContractArgs& p, int config, int la, int lb, hipStream_t s) {
  return contract::launch_typed<bf16_t>(p, config, la, lb, s);
}
}  // namespace es
