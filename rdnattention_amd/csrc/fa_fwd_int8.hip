// INT8 forward (placeholder until the int8 MFMA kernel lands).
#include "fa_host.hpp"
#include "fa_internal.hpp"

namespace rdna_amd {

int fwd_int8(const AttnArgs&, hipStream_t, std::string& err) {
    err = "int8 kernel not built";
    return -1;
}

int int8_scores(const AttnArgs&, int32_t*, hipStream_t, std::string& err) {
    err = "int8 kernel not built";
    return -1;
}


} // namespace rdna_amd
