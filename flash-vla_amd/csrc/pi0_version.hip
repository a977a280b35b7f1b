#include "pi0_hip.h"
extern "C" int pi0hip_version(void) { return 2; }
