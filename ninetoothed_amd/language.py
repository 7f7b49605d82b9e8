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
float8_e4m3fn = "float8_e4m3fn"
float8_e5m2 = "float8_e5m2"


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
    "rand", "randint", "randn", "load", "store", "atomic_add",
)
for _name in _FUNCTIONS:
    globals()[_name] = _parsed_only(_name)



class _LibDevice:
    """``ntl.libdevice``: device math functions by name (``libdevice.pow(x, y)``), as in
    the reference's ``ninetoothed.language.libdevice``.  Run by the generic kernels with
    the device math library of the HIP toolchain."""

    FUNCTIONS = ("pow", "exp", "exp2", "expm1", "log", "log2", "log10", "log1p", "sqrt", "rsqrt", "sin", "cos",
                 "tan", "tanh", "sinh", "cosh", "asin", "acos", "atan", "atan2", "erf", "floor", "ceil", "trunc",
                 "round", "fabs", "fmax", "fmin", "fmod", "hypot")

    def __init__(self):
        for name in self.FUNCTIONS:
            fn = _parsed_only(f"libdevice.{name}")
            fn._ntl_name = f"libdevice.{name}"
            setattr(self, name, fn)


libdevice = _LibDevice()

__all__ = list(_FUNCTIONS) + ["float16", "bfloat16", "float32", "float64", "int8", "int16", "int32", "int64", "uint8",
                              "libdevice"]
