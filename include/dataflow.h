/* Umbrella header (reference: include/dataflow.h:1-8). */
#ifndef DATAFLOW_LIB
#define DATAFLOW_LIB

#include "dataflow_common.h"
#include "dataflow_datatype.h"

#endif
