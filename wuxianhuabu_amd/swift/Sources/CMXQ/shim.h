/* The C ABI of libmxq for the Swift module CMXQ: include/mxq.h of this tree. */
#include "../../../../include/mxq.h"
