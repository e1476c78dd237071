// Test-only stand-in for <hip/hip_runtime.h>: see tests/emu/emu_hip.h.
#pragma once
#include "../../emu_hip.h"
