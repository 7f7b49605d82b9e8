"""Exception types, named as the reference names them."""


class KernelLaunchError(RuntimeError):
    """A library entry point returned a non-zero status.

    Same role and message as the reference's ``KernelLaunchError``
    (``src/ninetoothed/compiler/runtime.py:31-35``).
    """

    def __init__(self, error_code, entry_point=None):
        self.error_code = error_code
        self.entry_point = entry_point
        super().__init__(f"Kernel launch failed with error code: {error_code}.")


class LoweringError(ValueError):
    """The application or arrangement cannot be lowered for the MI355X backend.

    The reference raises ``LoweringError`` from its frontend
    (``src/ninetoothed/frontend/python.py``); here it is also raised when a program
    matches none of the hand-written kernel families.
    """
