"""ExpertExecutor's constructor contract on the CPU: the reference's keyword
validation (expertbench/executor.py:166-178) runs before any device work."""
import pytest

from pdscope_amd.executor import ExpertExecutor


@pytest.mark.parametrize("kw,msg", [(dict(cpu_staging_copy="mmap"), "CPU staging copy"),
                                    (dict(initialize_cpu_worker=1), "explicitly boolean"),
                                    (dict(profile_stages="yes"), "explicitly boolean"),
                                    (dict(pinned_source_mode="single"), "pinned source mode")])
def test_invalid_executor_keywords_raise_before_device_work(kw, msg):
    with pytest.raises(ValueError, match=msg):
        ExpertExecutor(None, {}, 0, **kw)
