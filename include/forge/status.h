// Status of the last forge:: call on this thread. The reference's launchers return
// void and never report errors; these wrappers keep void and record the C-ABI status.
#pragma once

namespace forge {

/// FORGE_OK (0), FORGE_EINVAL (-1), FORGE_ENODEV (-2) or a hipError_t value.
int last_error();

} // namespace forge
