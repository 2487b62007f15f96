// Host handle of one field group (sbx_fdm_* and the vec's field scenarios):
// the scenario's device tables, the group's buffers, the initial field.
#pragma once
#include <hip/hip_runtime_api.h>

#include <vector>

#include "fdm.h"
#include "sbenv.h"

struct SbxFdm {
    sbf::Tables tab{};
    sbf::Group grp{};
    SbxFdmInfo info{};
    unsigned char* d_tables = nullptr;
    double* d_temp_init = nullptr;
    double* d_mass_init = nullptr;
    std::vector<void*> owned;     // device buffers of the group
};

extern "C" int sbf_launch_step(const sbf::Tables* t, const sbf::Group* g, const sbf::StepIn* in, hipStream_t s);
extern "C" int sbf_launch_init(const sbf::Tables* t, const sbf::Group* g, const double* temp_init,
                               const double* mass_init, hipStream_t s);
