// Status checking for the C ABI (reference include/csrspmm/error_check.h:11-40
// wraps CUDA, cuBLAS and cuSPARSE status codes).  Here every device call goes
// through include/csrspmm_c.h, whose entry points return one int status.
#pragma once
#include <cstdio>
#include <cstdlib>

#include "../csrspmm_c.h"

namespace csrspmm {

inline void statusCheck(int status, const char* file, int line) {
    if (status != CSRSPMM_STATUS_SUCCESS) {
        std::fprintf(stderr, "csrspmm error %d (%s) at %s:%d\n", status,
                     csrspmm_status_string(status), file, line);
        std::exit(EXIT_FAILURE);
    }
}

}  // namespace csrspmm

#define csrspmmCheck(status) (::csrspmm::statusCheck((status), __FILE__, __LINE__))
