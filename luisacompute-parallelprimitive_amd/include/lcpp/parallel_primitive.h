// Umbrella header of the MI355X host facade: the device-level modules of the LCPP hot path
// (the reference's src/lcpp/parallel_primitive.h includes every family; these are the ones provided).
#pragma once

#include "lcpp/runtime/core.h"
#include "lcpp/device/device_reduce.h"
#include "lcpp/device/device_scan.h"
#include "lcpp/device/device_radix_sort.h"
#include "lcpp/device/device_spmv.h"
#include "lcpp/device/device_select.h"
#include "lcpp/device/device_partition.h"
#include "lcpp/device/device_run_length_encode.h"
#include "lcpp/device/device_segment_reduce.h"
#include "lcpp/device/device_segmented_scan.h"
#include "lcpp/device/device_segmented_sort.h"
#include "lcpp/device/device_segmented_radix_sort.h"
