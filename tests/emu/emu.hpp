// Harness-facing part of the CPU emulation runtime (emu_runtime.cpp).  Test infrastructure.
#pragma once
#include <stddef.h>

namespace emu {
// host memory that ends at a PROT_NONE page (an out-of-bounds access faults)
void* dalloc(size_t bytes, const char* name);
void dfree(void* p);
// SIGSEGV / SIGBUS: print the nearest allocation and the running lane, exit(3)
void install_fault_handler();
// launches of this kernel keep every block live at once (its blocks wait on each other)
void set_persistent(const void* kernel);
extern long long oob_loads, oob_stores;  // out-of-range buffer accesses so far
}  // namespace emu
