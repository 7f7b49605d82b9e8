"""Names an application body may use (``import ninetoothed_amd.language as ntl``).

Application bodies are parsed, never executed (as in the reference, whose
``ninetoothed.language`` only provides names, ``src/ninetoothed/language.py:1-26``).
The frontend recognises these objects by identity; calling one directly raises.
"""

float16 = "float16"
bfloat16 = "bfloat16"
float32 = "float32"
float64 = "float64"
int8 = "int8"
int16 = "int16"
int32 = "int32"
int64 = "int64"
uint8 = "uint8"


def _parsed_only(name):
    def fn(*args, **kwargs):
        raise RuntimeError(f"ntl.{name} is only meaningful inside an application body, which is parsed, not run.")

    fn.__name__ = name
    fn.__qualname__ = name
    fn._ntl_name = name
    return fn


_FUNCTIONS = (
    "zeros", "full", "dot", "trans", "where", "max", "min", "sum", "maximum", "minimum",
    "exp", "exp2", "log", "log2", "sqrt", "rsqrt", "abs", "sigmoid", "cast", "arange",
)
for _name in _FUNCTIONS:
    globals()[_name] = _parsed_only(_name)

__all__ = list(_FUNCTIONS) + ["float16", "bfloat16", "float32", "float64", "int8", "int16", "int32", "int64", "uint8"]
