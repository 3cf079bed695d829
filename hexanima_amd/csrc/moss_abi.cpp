// libhexanima_moss.so: the reference's MOSS block entry under its own symbol (see include/hexanima_moss.h). The
// block itself runs in libhexanima_hip.so (mega_moss_block); this library only binds the name mossrun calls.
#include "../../include/hexanima_moss.h"

extern "C" int mega_block(remote_handle64 h, const int *meta, int nmeta, int wfd, int bfd, const uint8_t *mod, int modlen,
                          int *times, int ntimes, int *rc) {
  return mega_moss_block(h, meta, nmeta, wfd, bfd, mod, modlen, times, ntimes, rc);
}
