// The device-side pieces the runtime's set-up references, stubbed for the
// host-only sanitizer build of the reader (the parse and read paths never
// reach them).
#include "apus_rt.h"
namespace apus {
int noalloc_setup(int) { return 0; }
const ActTables *act_tables() { return nullptr; }
}  // namespace apus
