"""The reference-side patch of INTEGRATION.md route 2, as data.

Each edit names a reference header (path under the reference root), a
short anchor that occurs once in it, and the text that replaces the
anchor. `apply_patch` copies the headers the HIP backend's source reaches
into a build folder and applies the edits there; the reference tree itself
is only read. The edits are the declarations route 2 adds:

  1. the op kinds SUB and DIV and the provider HIP, appended to their
     enums (include/m3.h);
  2. the backend kind HIP (src/m3_backend.h);
  3. the optional vtable hooks write, read, reserve and finish
     (src/m3_backend_internal.h);
  4. a tag for the command struct, the SUB/DIV descriptors and the
     elementwise-program descriptor in the command union (src/m3_op.h).

tests/test_route2_cpu.py compiles m3.c_amd/csrc/host/m3_backend_hip.c
against the patched headers with gcc -fsyntax-only.
"""
import os
import shutil

HEADERS = ["include/m3.h", "src/m3_error.h", "src/m3_backend.h",
           "src/m3_backend_internal.h", "src/m3_op.h", "src/m3_scratch.h",
           "src/m3_tensor.h"]

PROGRAM_DESCRIPTOR = """struct m3_command_s;

/* A run of elementwise commands fused into one program (m3_hip.h). */
#define M3_OP_ELEMENTWISE_PROGRAM ((m3_op_kind)0x1000)

typedef struct {
    const struct m3_command_s *commands;
    size_t command_count;
    const uint32_t *words;
    size_t word_count;
    m3_storage *storage;
    size_t byte_offset;
} m3_op_elementwise_program;

typedef struct m3_command_s {
    m3_op_kind kind;
    union {"""

HOOKS = """    m3_status (*write)(void *context, void *data, size_t byte_offset,
                       const void *source, size_t byte_count,
                       m3_error *error);
    m3_status (*read)(void *context, const void *data, size_t byte_offset,
                      void *destination, size_t byte_count,
                      m3_error *error);
    m3_status (*reserve)(void *context, size_t byte_count, m3_error *error);
    m3_status (*finish)(void *context, m3_error *error);
} m3_backend_vtable;"""

EDITS = [
    ("include/m3.h", "    M3_OP_TANH\n",
     "    M3_OP_TANH,\n    M3_OP_SUB,\n    M3_OP_DIV\n"),
    ("include/m3.h", "    M3_PROVIDER_CPU\n",
     "    M3_PROVIDER_CPU,\n    M3_PROVIDER_HIP\n"),
    ("src/m3_backend.h", "    M3_BACKEND_METAL\n} m3_backend_kind;",
     "    M3_BACKEND_METAL,\n    M3_BACKEND_HIP\n} m3_backend_kind;"),
    ("src/m3_backend_internal.h", "} m3_backend_vtable;", HOOKS),
    ("src/m3_op.h", "typedef struct {\n    m3_op_kind kind;\n    union {",
     PROGRAM_DESCRIPTOR),
    ("src/m3_op.h", "        m3_op_unary tanh;\n    } descriptor;",
     "        m3_op_unary tanh;\n        m3_op_binary sub;\n"
     "        m3_op_binary div;\n"
     "        m3_op_elementwise_program elementwise_program;\n"
     "    } descriptor;"),
]


def apply_patch(reference_root, out_dir, edits=EDITS):
    """Copies HEADERS under out_dir (as include/ and src/) and applies
    `edits`. Raises if an anchor is missing or not unique."""
    for relative in HEADERS:
        target = os.path.join(out_dir, relative)
        os.makedirs(os.path.dirname(target), exist_ok=True)
        shutil.copyfile(os.path.join(reference_root, relative), target)
    for relative, anchor, text in edits:
        path = os.path.join(out_dir, relative)
        with open(path) as handle:
            source = handle.read()
        if source.count(anchor) != 1:
            raise ValueError("anchor %r occurs %d times in %s"
                             % (anchor, source.count(anchor), relative))
        with open(path, "w") as handle:
            handle.write(source.replace(anchor, text))
