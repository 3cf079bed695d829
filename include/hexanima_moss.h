/* hexanima_moss.h -- the MOSS build of the reference's block interface, libhexanima_moss.so.
 *
 * The reference builds its MOSS-Image mega-kernel as a separate DSP module whose `mega_block` takes the MOSS meta
 * enum (moss/hexagon/mega/blk_meta.h:3-4) and a 6 x DIM modulation; mossrun calls it by that name
 * (moss/mossrun/mossrun.cpp:182-188). libhexanima_moss.so exports exactly that symbol, so a mossrun-style caller links
 * `-lhexanima_moss -lhexanima_hip` (in that order) unchanged: mega_block resolves to this library, mega_open,
 * mega_close and the buffer registration (include/hexanima_hip.h) to libhexanima_hip.so.
 */
#pragma once
#include "hexanima_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* replaces the MOSS mega_block (moss/hexagon/mega/blk.c:269-281, IDL mega.idl:10): one MOSS-class DiT block, MODE 0
 * (the DiT block with its rapid-moss LoRA, blk.c:234-259); meta[] per moss blk_meta.h:3-4, weights registered with
 * HXA_KIND_WEIGHTS_MOSS (export_moss.py layout at byte offset meta[M_WOFF]), mod = 6 x 3072 fp32. Other modes (the
 * text refiner 1 / 2 and the text-encoder layers 10 / 11 / 20 / 21 / 30) return *rc = HXA_E_MODE. */
int mega_block(remote_handle64 h, const int *meta, int nmeta, int wfd, int bfd, const uint8_t *mod, int modlen, int *times,
               int ntimes, int *rc);

#ifdef __cplusplus
}
#endif
