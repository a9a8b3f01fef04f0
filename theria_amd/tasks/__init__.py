from .batch import TaskBatch
from .teacher_readout import teacher_readout_task
from .token_count import label_sequences, sample_token_count_task

__all__ = ["TaskBatch", "teacher_readout_task", "label_sequences", "sample_token_count_task"]
