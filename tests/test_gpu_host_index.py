"""The bit-exact index and tile-map checks of tests/test_host_abi.py, collected again
under the `gpu` marker so that the GPU box's own run of the library (the record of a
`-m gpu` run) pins the Block-ELL sampler and transpose and the attention tile kinds
and work lists against the oracle too, not only the CPU run here. Same functions,
same cases."""
import pytest

import test_host_abi as h

pytestmark = pytest.mark.gpu

test_sampler_and_transpose_bit_exact_on_gpu_box = h.test_sampler_and_transpose_bit_exact
test_sampler_matches_golden_on_gpu_box = h.test_sampler_matches_golden
test_tile_kinds_bit_exact_on_gpu_box = h.test_tile_kinds_bit_exact
test_work_list_bit_exact_on_gpu_box = h.test_work_list_bit_exact
test_work_list_kv_bit_exact_on_gpu_box = h.test_work_list_kv_bit_exact
test_mask_spans_bit_exact_on_gpu_box = h.test_mask_spans_bit_exact
test_tile_map_golden_on_gpu_box = h.test_tile_map_golden
