"""Stand-in for comfy.patcher_extension, for tests only."""


class CallbacksMP:
    ON_CLEANUP = "on_cleanup"
