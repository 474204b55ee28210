// Builds tachyon_amd/csrc/tsm_sample.hip for the CPU emulation (test only).
#include "../../tachyon_amd/csrc/tsm_sample.hip"
