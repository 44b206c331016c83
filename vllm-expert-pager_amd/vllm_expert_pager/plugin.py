"""vLLM general-plugin entry point (pyproject: vllm.general_plugins expert_pager).

Same entry as the reference (plugin.py:1-6): the hook module is imported
inside the function because it can only be imported after vLLM has loaded.
"""


def register() -> None:
    from vllm_expert_pager import experts

    experts.register()
