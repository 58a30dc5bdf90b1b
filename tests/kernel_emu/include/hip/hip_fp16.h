// The CPU emulation stands in for <hip/hip_fp16.h> (tests/kernel_emu/kvb_emu.hpp).
#pragma once
#include "kvb_emu.hpp"
