// Host interface of the static device scratch (scratch.hip): internal to libmtk.so.
#pragma once

#include <stddef.h>

namespace mtk_scratch {

// Takes the device address of `device`'s copy of the scratch array (hipGetSymbolAddress), once;
// the device must be current. 0 on success.
int setup(int device);

// The address taken by setup; -1 with a message in err if there is none.
int address(int device, void **out, char *err, size_t errlen);

}  // namespace mtk_scratch
