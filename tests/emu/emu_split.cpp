// Builds tachyon_amd/csrc/tsm_split.hip for the CPU emulation (test only).
#include "../../tachyon_amd/csrc/tsm_split.hip"
