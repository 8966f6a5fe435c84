// Test driver for the product's scalar-expression evaluator
// (pto-wsp_amd/csrc/host/scalar.cpp): one expression per input line in the
// module's token form; prints "<type> <value bits>" or "E <message>".
// Symbols and slots hold fixed functions of their id / index, the same ones
// tests/test_scalar_expr.py gives the oracle and the compiled C++ reference.
#include <cstdint>
#include <iostream>
#include <sstream>
#include <stdexcept>
#include <string>

#include "../pto-wsp_amd/csrc/host/scalar.hpp"

int main() {
    ptowsp::SEnv env;
    env.symbol = [](uint64_t id) { return id * 0x9E3779B97F4A7C15ull + 0x1234567ull; };
    env.slot = [](uint32_t i) -> uint64_t { return i < 256 ? i * 0x0123456789ABCDEFull + 7 : 0; };
    std::string line;
    while (std::getline(std::cin, line)) {
        std::istringstream is(line);
        try {
            auto e = ptowsp::parse_scalar([&] {
                std::string t;
                if (!(is >> t)) throw std::runtime_error("end of expression");
                return t;
            });
            const ptowsp::SValue v = ptowsp::eval_scalar(*e, env);
            const char t = v.t == ptowsp::SType::Bool ? 'b' : v.t == ptowsp::SType::I64 ? 'i' : 'u';
            std::cout << t << ' ' << v.v << '\n';
        } catch (const std::exception& ex) {
            std::cout << "E " << ex.what() << '\n';
        }
    }
    return 0;
}
