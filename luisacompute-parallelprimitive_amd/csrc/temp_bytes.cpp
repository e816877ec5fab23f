// Temp-storage byte counts of the reference's Get*TempStorageBytes, restated so that a buffer sized
// for LCPP is accepted unchanged.  Pure host arithmetic; every formula cites the reference lines it
// restates (paths relative to the LCPP source root).
#include "../../include/lcpp_hip.h"

#include <algorithm>
#include <cstdint>
#include <cstddef>

namespace {

constexpr size_t kWarpSize = 32;     // details::WARP_SIZE, runtime/core.h:17-23
constexpr size_t kAlign = 256;       // TEMP_STORAGE_VIEW_ALIGNMENT / descriptor_view_alignment, common/utils.h:194-222
constexpr size_t kAlignUints = kAlign / sizeof(uint32_t);

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }
size_t bytes_to_uint_count(size_t bytes) { return (bytes + 3) / 4; }  // common/utils.h:247-250

// radix_effective_items_v (agent/policy.h:85-89)
size_t radix_effective_items(size_t nominal, size_t key_bytes) {
    if (key_bytes <= 4) return nominal;
    const size_t scaled = nominal * 4 / key_bytes;
    return scaled < 4 ? 4 : scaled;
}

// compute_onesweep_temp_layout(...).total_bytes (device/device_radix_sort.h:267-317) for
// begin_bit = 0, end_bit = 8 * key_bytes.
size_t onesweep_layout_bytes(uint32_t n, size_t key_bytes, size_t value_bytes, uint32_t block_threads,
                             uint32_t items_per_thread) {
    const uint32_t radix_bits = 8;     // OneSweepSmallKeyTunedPolicy::ONESWEEP_RADIX_BITS, policy.h:71-76
    const uint32_t radix_digits = 1u << radix_bits;
    const uint32_t tile_items = block_threads * items_per_thread;
    const uint32_t portion_size = ((1u << 28u) - 1u) / tile_items * tile_items;
    const uint32_t num_passes = static_cast<uint32_t>(ceil_div(key_bytes * 8, radix_bits));
    const uint32_t num_portions = static_cast<uint32_t>(ceil_div(n, portion_size));
    const uint32_t max_num_blocks = static_cast<uint32_t>(ceil_div(std::min(n, portion_size), tile_items));

    const size_t bins_count = static_cast<size_t>(num_portions) * num_passes * radix_digits;
    const size_t lookback_count = static_cast<size_t>(max_num_blocks) * radix_digits;
    const size_t ctrs_count = static_cast<size_t>(num_portions) * num_passes * kAlignUints;
    const size_t keys_tmp2_count = bytes_to_uint_count(static_cast<size_t>(n) * key_bytes);
    const size_t values_tmp2_count = bytes_to_uint_count(static_cast<size_t>(n) * value_bytes);

    size_t off = bins_count * 4;
    off = align_up(off);
    off += lookback_count * 4;
    if (num_passes > 1) {
        off = align_up(off);
        off += keys_tmp2_count * 4;
        off = align_up(off);
        off += values_tmp2_count * 4;
    }
    off = align_up(off);
    off += ctrs_count * 4;
    return off;
}

}  // namespace

extern "C" {

// DeviceReduce::reduce_temp_storage_bytes (device/device_reduce.h:517-536).
size_t lcpp_hip_reduce_temp_bytes_policy(uint64_t n, size_t elem_bytes, uint32_t block_size,
                                         uint32_t items_per_thread) {
    const size_t tile = static_cast<size_t>(block_size) * items_per_thread;
    if (tile == 0 || elem_bytes == 0) return 0;
    size_t bytes = 0;
    size_t level_items = n;
    bool first = true;
    do {
        const size_t num_blocks = std::max<size_t>(1, ceil_div(level_items, tile));
        if (!first) bytes = align_up(bytes);
        bytes += num_blocks * elem_bytes;
        level_items = num_blocks;
        first = false;
    } while (level_items > 1);
    return bytes;
}

// DeviceReduce<256, 32, 8> (REDUCE_ITEMS_PER_THREAD = 8, device_reduce.h:54,102-113).
size_t lcpp_hip_reduce_temp_bytes(uint64_t n, size_t elem_bytes) {
    return lcpp_hip_reduce_temp_bytes_policy(n, elem_bytes, 256, 8);
}

// DeviceReduce<>::GetArgTempStorageBytes (device_reduce.h:198-210): the reduce temp of (index, value)
// pairs (a 4-byte index beside the value, padded to the value's alignment), then n pairs and one pair,
// each 256-byte aligned.
size_t lcpp_hip_reduce_arg_temp_bytes(uint64_t n, size_t elem_bytes) {
    if (elem_bytes != 4 && elem_bytes != 8) return 0;
    const size_t pair = elem_bytes == 4 ? 8 : 16;
    size_t bytes = lcpp_hip_reduce_temp_bytes(n, pair);
    bytes = align_up(bytes);
    bytes += n * pair;
    bytes = align_up(bytes);
    return bytes + pair;
}

// DeviceScan::GetTempStorageBytes (device/device_scan.h:295-308) with scan_temp_storage_bytes
// (:111-126) and num_tiles_for (:102-109).  `default_policy` selects the extra reservation for the
// runtime-chosen 320x25 packed layout that the default template arguments add for 4-byte values.
size_t lcpp_hip_scan_temp_bytes_policy(uint64_t n, size_t elem_bytes, uint32_t block_size, uint32_t items_per_thread,
                                       int default_policy, int packed_tile_state) {
    const size_t tile = static_cast<size_t>(block_size) * items_per_thread;
    if (tile == 0 || elem_bytes == 0) return 0;
    const size_t tiles = std::max<size_t>(1, ceil_div(n, tile));
    const size_t tile_count = kWarpSize + tiles;
    size_t bytes = 0;
    if (packed_tile_state && elem_bytes == 4) {
        bytes = align_up(tile_count * 8);
    } else {
        bytes = tile_count * 4;
        bytes = align_up(bytes);
        bytes += bytes_to_uint_count(tile_count * elem_bytes) * 4;
        bytes = align_up(bytes);
        bytes += bytes_to_uint_count(tile_count * elem_bytes) * 4;
    }
    if (default_policy && elem_bytes == 4) {
        const size_t cuda_tiles = kWarpSize + std::max<size_t>(1, ceil_div(n, 320 * 25));
        bytes = std::max(bytes, align_up(cuda_tiles * 8));
    }
    return bytes;
}

// DeviceScan<256, 32, 15, DIRECT, DIRECT, false, false> (device_scan.h:40-49).
size_t lcpp_hip_scan_temp_bytes(uint64_t n, size_t elem_bytes) {
    return lcpp_hip_scan_temp_bytes_policy(n, elem_bytes, 256, 15, 1, 0);
}

// onesweep_sizing_bytes (device/device_radix_sort.h:330-340): the larger of the conservative
// (BLOCK x radix_effective_items<ITEMS>) and tuned (384x20 for 4-byte key-only sorts under
// CUB_SMALL_KEY_POLICY) layouts.  Keys-only sorts size values_tmp2 with the key type
// (GetSortKeysTempStorageBytes passes ValueType = KeyType, :358-362).
size_t lcpp_hip_radix_sort_temp_bytes_policy(uint32_t n, size_t key_bytes, size_t value_bytes, int keys_only,
                                             uint32_t block_size, uint32_t items_per_thread,
                                             int cub_small_key_policy) {
    if (key_bytes == 0 || block_size == 0 || items_per_thread == 0) return 0;
    const size_t vbytes = keys_only ? key_bytes : value_bytes;
    const uint32_t cb = block_size;
    const uint32_t ci = static_cast<uint32_t>(radix_effective_items(items_per_thread, key_bytes));
    const bool tuned_small = keys_only && cub_small_key_policy && key_bytes == 4;
    const uint32_t tb = tuned_small ? 384u : block_size;
    const uint32_t ti = static_cast<uint32_t>(radix_effective_items(tuned_small ? 20u : items_per_thread, key_bytes));
    const size_t cons = onesweep_layout_bytes(n, key_bytes, vbytes, cb, ci);
    const size_t tuned = onesweep_layout_bytes(n, key_bytes, vbytes, tb, ti);
    return std::max(cons, tuned);
}

// DeviceRadixSort<256, 32, 16, true> (RADIX_ITEMS_PER_THREAD = 16, device_radix_sort.h:48-56).
size_t lcpp_hip_radix_sort_keys_temp_bytes(uint32_t n, size_t key_bytes) {
    return lcpp_hip_radix_sort_temp_bytes_policy(n, key_bytes, key_bytes, 1, 256, 16, 1);
}

size_t lcpp_hip_radix_sort_pairs_temp_bytes(uint32_t n, size_t key_bytes, size_t value_bytes) {
    return lcpp_hip_radix_sort_temp_bytes_policy(n, key_bytes, value_bytes, 0, 256, 16, 1);
}

// DeviceSpmv::GetTempStorageBytes (device/device_spmv.h:43-46).
size_t lcpp_hip_spmv_temp_bytes(uint64_t, uint64_t, uint64_t) { return 0; }

// sizeof(KeyValuePair<int, V>) (common/util_type.h:17-21): an int and a V with natural alignment.
static size_t flag_value_pair_bytes(size_t value_bytes) { return value_bytes <= 4 ? 8 : 2 * value_bytes; }

// DeviceScan<BLOCK, 32, ITEMS>::GetScanByKeyTempStorageBytes<K, V> (device/device_scan.h:310-315) =
// scan_by_key_temp_storage_bytes (:129-142) with num_tiles_for (:102-109), raised to what the
// by-key kernel carves when a policy's tiles are so large that the reference layout is smaller.
size_t lcpp_hip_scan_by_key_temp_bytes_policy(uint64_t n, size_t key_bytes, size_t value_bytes, uint32_t block_size,
                                              uint32_t items_per_thread) {
    const size_t tile = static_cast<size_t>(block_size) * items_per_thread;
    if (tile == 0 || key_bytes == 0 || value_bytes == 0) return 0;
    const size_t tiles = std::max<size_t>(1, ceil_div(n, tile));
    const size_t tile_count = kWarpSize + tiles;
    const size_t pair = flag_value_pair_bytes(value_bytes);
    size_t bytes = tile_count * 4;
    bytes = align_up(bytes);
    bytes += bytes_to_uint_count(tile_count * pair) * 4;
    bytes = align_up(bytes);
    bytes += bytes_to_uint_count(tile_count * pair) * 4;
    bytes = align_up(bytes);
    bytes += bytes_to_uint_count(tiles * key_bytes) * 4;
    return std::max(bytes, lcpp_hip_internal_by_key_needed_bytes(n, value_bytes));
}

// DeviceScan<> (256 x 15 items, device/device_scan.h:40-49).
size_t lcpp_hip_scan_by_key_temp_bytes(uint64_t n, size_t key_bytes, size_t value_bytes) {
    return lcpp_hip_scan_by_key_temp_bytes_policy(n, key_bytes, value_bytes, 256, 15);
}

// DeviceReduce<BLOCK>::GetReduceByKeyTempStorageBytes<K, V> (device/device_reduce.h:207-223) with
// the fixed REDUCE_BY_KEY_ITEMS_PER_THREAD = 4 (:100), raised like the scan-by-key query above.
size_t lcpp_hip_reduce_by_key_temp_bytes_policy(uint64_t n, size_t key_bytes, size_t value_bytes,
                                                uint32_t block_size) {
    const size_t tile = static_cast<size_t>(block_size) * 4;
    if (tile == 0 || key_bytes == 0 || value_bytes == 0) return 0;
    const size_t tiles = std::max<size_t>(1, ceil_div(n, tile));
    const size_t tile_count = kWarpSize + tiles;
    const size_t pair = flag_value_pair_bytes(value_bytes);
    size_t bytes = tile_count * 4;
    bytes = align_up(bytes);
    bytes += tile_count * pair;
    bytes = align_up(bytes);
    bytes += tile_count * pair;
    return std::max(bytes, lcpp_hip_internal_by_key_needed_bytes(n, value_bytes));
}

// DeviceReduce<> (BLOCK_SIZE = 256).
size_t lcpp_hip_reduce_by_key_temp_bytes(uint64_t n, size_t key_bytes, size_t value_bytes) {
    return lcpp_hip_reduce_by_key_temp_bytes_policy(n, key_bytes, value_bytes, 256);
}

// DeviceScan<BLOCK, 32, ITEMS>::GetTempStorageBytes<uint>, the scan the compaction modules size for
// (device_select.h:22,56-63): the default-policy reservation applies only to the 256 x 15 tile.
static size_t compaction_scan_bytes(uint64_t n, uint32_t block_size, uint32_t items_per_thread) {
    const int default_policy = block_size == 256 && items_per_thread == 15 ? 1 : 0;
    return lcpp_hip_scan_temp_bytes_policy(n, 4, block_size, items_per_thread, default_policy, 0);
}

// DeviceSelect<BLOCK, 32, ITEMS>::GetTempStorageBytes (device_select.h:56-63) and
// DevicePartition<>::GetTempStorageBytes (device_partition.h:55-62): 2 n uints + the scan's bytes;
// raised to the compaction kernels' need (in-place staging of 8-byte items) where a policy's scan
// layout is smaller.
size_t lcpp_hip_select_temp_bytes_policy(uint64_t n, uint32_t block_size, uint32_t items_per_thread) {
    if (n == 0 || block_size == 0 || items_per_thread == 0) return 0;
    const size_t bytes = 2 * n * 4 + compaction_scan_bytes(n, block_size, items_per_thread);
    return std::max(bytes, lcpp_hip_internal_compact_needed_bytes(n, 8, 1, 1));
}

size_t lcpp_hip_select_temp_bytes(uint64_t n) { return lcpp_hip_select_temp_bytes_policy(n, 256, 4); }

// DevicePartition<BLOCK, 32, ITEMS>::GetThreeWayTempStorageBytes (device_partition.h:64-71).
size_t lcpp_hip_partition_three_way_temp_bytes_policy(uint64_t n, uint32_t block_size, uint32_t items_per_thread) {
    if (n == 0 || block_size == 0 || items_per_thread == 0) return 0;
    const size_t bytes = 3 * n * 4 + compaction_scan_bytes(n, block_size, items_per_thread);
    return std::max(bytes, lcpp_hip_internal_compact_needed_bytes(n, 8, 2, 1));
}

size_t lcpp_hip_partition_three_way_temp_bytes(uint64_t n) {
    return lcpp_hip_partition_three_way_temp_bytes_policy(n, 256, 4);
}

// DeviceRunLengthEncode<BLOCK, 32, ITEMS>::GetTempStorageBytes (device_run_length_encode.h:56-69):
// six n-sized uint arrays and a run counter, 256-byte aligned, then the scan's bytes.
size_t lcpp_hip_run_length_encode_temp_bytes_policy(uint64_t n, uint32_t block_size, uint32_t items_per_thread) {
    if (n == 0 || block_size == 0 || items_per_thread == 0) return 0;
    const size_t bytes = align_up((6 * n + 1) * 4) + compaction_scan_bytes(n, block_size, items_per_thread);
    return std::max(bytes, lcpp_hip_internal_compact_needed_bytes(n, 8, 2, 1));
}

size_t lcpp_hip_run_length_encode_temp_bytes(uint64_t n) {
    return lcpp_hip_run_length_encode_temp_bytes_policy(n, 256, 4);
}

// DeviceSegmentReduce<>::GetTempStorageBytes (device_segment_reduce.h:87-91) and
// DeviceSegmentedScan<>::GetTempStorageBytes (device_segmented_scan.h:52-56): no temp storage.
size_t lcpp_hip_segment_reduce_temp_bytes(uint64_t) { return 0; }
size_t lcpp_hip_segmented_scan_temp_bytes(uint64_t, uint64_t) { return 0; }

// DeviceSegmentReduce<>::GetArgTempStorageBytes<T> (device_segment_reduce.h:95-104): n and
// num_segments (index, value) pairs of 8 bytes, the second array 256-byte aligned.  The ArgMin / ArgMax
// kernels here carve none of it.
size_t lcpp_hip_segment_reduce_arg_temp_bytes(uint64_t n, uint64_t num_segments) {
    return align_up(n * 8) + num_segments * 8;
}

}  // extern "C"
