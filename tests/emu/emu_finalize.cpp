// Builds tachyon_amd/csrc/tsm_finalize.hip for the CPU emulation (test only).
#include "../../tachyon_amd/csrc/tsm_finalize.hip"
