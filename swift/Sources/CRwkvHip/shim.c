/* SwiftPM needs one source file in a C target; the module is header-only. */
#include "CRwkvHip.h"
