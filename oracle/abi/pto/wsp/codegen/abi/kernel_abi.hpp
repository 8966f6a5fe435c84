// TEST INFRASTRUCTURE (the CPU oracle's side of cpp_tu_path kernels).
// The task descriptor a cpp_tu_path translation unit includes, as the
// reference's include/pto/wsp/codegen/abi/kernel_abi.hpp:21-71 declares it:
// the layouts of include/ptowsp_abi.h, and PTO_WSP_KERNEL_ATTR empty on the
// host.
#pragma once
#include <cstddef>
#include <cstdint>
#include "ptowsp_abi.h"
#define PTO_WSP_KERNEL_ATTR
