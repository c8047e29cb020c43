"""A probe of the plug-in ABI: sizeof/offsetof of every public and plug-in
struct, enum values and capacity macros, printed as JSON by a small C
program compiled against a given set of headers.

make_abi_fixture.py runs it against the reference's headers and commits
the result (abi_reference.json); tests/test_abi_reference_cpu.py runs it
against include/ and compares.
"""
import json
import os
import subprocess
import tempfile

STRUCTS = {
    "m3_error": ["status", "message"],
    "m3_graph_value_desc": ["dtype", "rank", "shape", "role"],
    "m3_graph_node_desc": ["kind", "inputs", "outputs", "parameters"],
    "m3_coreml_partition_desc": ["compiled_model_path", "inputs",
                                 "input_names", "input_count", "outputs",
                                 "output_names", "output_count"],
    "m3_session_options": ["allow_neural_engine", "allow_metal",
                           "allow_cpu"],
    "m3_session_plan_info": ["value_count", "node_count",
                             "storage_slot_count", "allocated_bytes"],
    "m3_tensor_metadata": ["dtype", "rank", "shape", "element_count",
                           "byte_count"],
    "m3_tensor_view": ["metadata", "byte_offset", "byte_strides",
                       "storage"],
    "m3_scratch_arena": ["data", "capacity", "offset"],
    "m3_backend_info": ["name", "kind", "unified_memory",
                        "recommended_working_set_bytes",
                        "maximum_storage_bytes"],
    "m3_backend_allocation_stats": ["live_allocated_bytes",
                                    "peak_allocated_bytes",
                                    "live_storage_count",
                                    "peak_storage_count"],
    # the four hooks of the reference; this library appends more
    "m3_backend_vtable": ["destroy_context", "allocate", "free_storage",
                          "execute"],
    "m3_op_unary": ["input", "output"],
    "m3_op_binary": ["left", "right", "output"],
    "m3_op_snake1d": ["input", "alpha", "output"],
    "m3_op_embedding": ["ids", "table", "output"],
    "m3_op_matmul": ["left", "right", "output"],
    "m3_op_linear": ["input", "weight", "bias", "output"],
    "m3_op_rms_norm": ["input", "scale", "output", "epsilon"],
    "m3_op_layer_norm": ["input", "scale", "bias", "output", "epsilon"],
    "m3_op_rope": ["input", "cosines", "sines", "output", "position_offset",
                   "rotary_dimension", "mode"],
    "m3_op_attention": ["query", "key", "value", "mask", "output", "scale",
                        "causal_offset", "causal"],
    "m3_op_top_k": ["logits", "values", "indices", "k"],
    "m3_op_categorical": ["probabilities", "uniforms", "output"],
    "m3_op_conv1d": ["input", "weight", "bias", "output", "groups",
                     "stride", "dilation", "pad_left", "pad_right"],
    "m3_op_conv_transpose1d": ["input", "weight", "bias", "output",
                               "groups", "stride", "dilation", "pad_left",
                               "pad_right", "output_padding"],
    "m3_command": ["kind", "descriptor"],
}

# sizes that may differ because this library appends members
GROWN = {"sizeof m3_backend_vtable"}

ENUMS = [
    "M3_STATUS_OK", "M3_STATUS_INVALID_ARGUMENT", "M3_STATUS_OUT_OF_RANGE",
    "M3_STATUS_OVERFLOW", "M3_STATUS_OUT_OF_MEMORY", "M3_STATUS_IO",
    "M3_STATUS_INVALID_FORMAT", "M3_STATUS_UNSUPPORTED",
    "M3_STATUS_CANCELLED", "M3_STATUS_INTERNAL",
    "M3_DTYPE_F32", "M3_DTYPE_F16", "M3_DTYPE_BF16", "M3_DTYPE_I32",
    "M3_OP_COPY", "M3_OP_CAST", "M3_OP_ADD", "M3_OP_MUL", "M3_OP_EMBEDDING",
    "M3_OP_MATMUL", "M3_OP_LINEAR", "M3_OP_RMS_NORM", "M3_OP_LAYER_NORM",
    "M3_OP_ROPE", "M3_OP_ATTENTION", "M3_OP_GATED_SILU", "M3_OP_SOFTMAX",
    "M3_OP_TOP_K", "M3_OP_CATEGORICAL", "M3_OP_CONV1D",
    "M3_OP_CONV_TRANSPOSE1D", "M3_OP_NEAREST_RESIZE1D", "M3_OP_SNAKE1D",
    "M3_OP_TANH", "M3_ROPE_HALF_SPLIT", "M3_ROPE_INTERLEAVED",
    "M3_PROVIDER_NEURAL_ENGINE", "M3_PROVIDER_METAL", "M3_PROVIDER_CPU",
    "M3_GRAPH_INPUT", "M3_GRAPH_CONSTANT", "M3_GRAPH_TEMPORARY",
    "M3_GRAPH_OUTPUT", "M3_BACKEND_HOST", "M3_BACKEND_METAL",
    "M3_TENSOR_MAX_RANK", "M3_GRAPH_NODE_INPUT_CAPACITY",
    "M3_GRAPH_NODE_OUTPUT_CAPACITY", "M3_GRAPH_VALUE_NONE",
    "M3_ERROR_MESSAGE_CAPACITY",
]


def probe_source(includes):
    lines = ["#include <stddef.h>", "#include <stdio.h>"]
    lines += ['#include "%s"' % name for name in includes]
    lines.append("int main(void)\n{\n    printf(\"{\\n\");")
    for struct, fields in STRUCTS.items():
        lines.append('    printf("\\"sizeof %s\\": %%zu,\\n", sizeof(%s));'
                     % (struct, struct))
        for field in fields:
            lines.append(
                '    printf("\\"offsetof %s.%s\\": %%zu,\\n", '
                'offsetof(%s, %s));' % (struct, field, struct, field))
    for name in ENUMS:
        lines.append('    printf("\\"value %s\\": %%lld,\\n", '
                     '(long long)(%s));' % (name, name))
    lines.append('    printf("\\"end\\": 0\\n}\\n");\n    return 0;\n}')
    return "\n".join(lines) + "\n"


def run_probe(include_dirs, includes):
    """Compiles and runs the probe; returns its JSON as a dict (without the
    closing "end" entry)."""
    with tempfile.TemporaryDirectory() as work:
        source = os.path.join(work, "probe.c")
        binary = os.path.join(work, "probe")
        with open(source, "w") as handle:
            handle.write(probe_source(includes))
        command = ["gcc", "-std=c11", "-D_POSIX_C_SOURCE=200809L"]
        for directory in include_dirs:
            command += ["-I", directory]
        command += ["-o", binary, source]
        subprocess.run(command, check=True)
        output = subprocess.run([binary], check=True, capture_output=True,
                                text=True).stdout
    values = json.loads(output)
    values.pop("end")
    return values
