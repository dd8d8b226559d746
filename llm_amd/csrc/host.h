// Internal header of the host layer (host.cpp); its C-ABI is in llmhip.h.
#pragma once

#include "common.h"
