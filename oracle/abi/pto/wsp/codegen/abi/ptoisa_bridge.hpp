// TEST INFRASTRUCTURE (the CPU oracle's side of cpp_tu_path kernels).
// What a cpp_tu_path translation unit may use of the reference's
// include/pto/wsp/codegen/abi/ptoisa_bridge.hpp without PTO-ISA: the
// PTO_WSP_ADVANCE macro (:33-38) and the pto::cpu_sim cycle counter
// (:58-64), a thread-local that starts at zero.
#pragma once
#include <cstdint>
#include "pto/wsp/codegen/abi/kernel_abi.hpp"
#define PTO_WSP_ADVANCE(cspt_ptr, cycles_expr) \
    do { \
        if ((cspt_ptr) && (cspt_ptr)->advance_cycles && (cycles_expr) != 0) \
            (cspt_ptr)->advance_cycles((cspt_ptr)->ctx, static_cast<uint64_t>(cycles_expr)); \
    } while (0)
namespace pto { namespace cpu_sim {
inline thread_local std::uint64_t cycle_counter = 0;
inline void reset_cycles() { cycle_counter = 0; }
inline void add_cycles(std::uint64_t cycles) { cycle_counter += cycles; }
inline std::uint64_t read_cycles() { return cycle_counter; }
} }
