/* Umbrella header of the CDCN system-library target: the libdcn C ABI. */
#include "../../../../include/dcn/dcn.h"
